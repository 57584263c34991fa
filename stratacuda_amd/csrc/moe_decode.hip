// One MoE layer for a single token (decode), without any host round trip:
//
//   1. route      k_route_t1 (moe_route.hip): router logits + shared-expert
//                 gate logit, exact reference order; the last wave to finish
//                 runs the top-k and writes ids / weights.
//   2. gate/up    k_decode_gate_up: for the topk routed experts (IDs read on
//                 the device) and the shared expert, hidden[k][j] =
//                 SiLU(g_j . x) * (u_j . x) over the interleaved gate/up rows.
//   3. down       k_decode_down: every block owns 8 output rows and computes
//                 them for all topk+1 experts, then combines them in the
//                 reference order (kernels/strata.cu:360-365):
//                 y = shared * sigmoid(gate) + sum_k part_k * w_k.
//
// Q2 GEMV layout: a 64-weight scale group of one row is 16 bytes of codes, so
// one lane reads one group with a single 16-byte load. In gate/up the 32
// lanes of each half-wave cover the 32 groups of a 2048-wide row (gate row in
// lanes 0-31, the adjacent up row in lanes 32-63: 1 KiB contiguous per wave);
// in down 8 lanes cover the 8 groups of a 512-wide row and a wave covers 8
// rows. Per group the lane accumulates sum(c_i * x_i) over the raw codes
// c in {0..3} and applies the group as scale * (sum - sum(x_i)), i.e.
// sum((c_i - 1) * scale * x_i) of the reference with the "-1" and the scale
// factored out of the inner loop. Codes are spread to bytes four at a time
// ((w >> 2s) & 0x03030303) and converted with the byte-select conversions.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

// acc += sum over the 16 codes of word w of code * x[base + i] (code i at bits 2i).
__device__ __forceinline__ float dot16(uint32_t w, const float *x, float acc) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        uint32_t m = (w >> (2 * s)) & 0x03030303u;
        acc = fmaf((float)(m & 0xffu), x[s], acc);
        acc = fmaf((float)((m >> 8) & 0xffu), x[4 + s], acc);
        acc = fmaf((float)((m >> 16) & 0xffu), x[8 + s], acc);
        acc = fmaf((float)(m >> 24), x[12 + s], acc);
    }
    return acc;
}

// sum_{i<64} code_i * x_i for one 16-byte code group.
__device__ __forceinline__ float dot64(uint4 c, const float *x) {
    float acc = 0.0f;
    acc = dot16(c.x, x, acc);
    acc = dot16(c.y, x + 16, acc);
    acc = dot16(c.z, x + 32, acc);
    acc = dot16(c.w, x + 48, acc);
    return acc;
}

// Blob of expert slot k (k < topk: routed ID ids[k]; k == topk: shared).
// An ID outside [0, experts) (only possible for non-finite router input)
// yields nullptr and the slot produces NaN instead of reading out of bounds.
__device__ __forceinline__ const uint8_t *expert_blob(const uint8_t *arena, uint64_t stride, const uint8_t *shared,
                                                      const int *ids, int k, int topk, int experts) {
    if (k >= topk) return shared;
    const int id = ids[k];
    return id >= 0 && id < experts ? arena + (uint64_t)id * stride : nullptr;
}

// Grid: (ff / 16, topk + 1). Block: 4 waves x 4 hidden rows. Dynamic LDS: x.
// Requires width <= 2048 * 32 / 32 groups per half-wave: groups g = lane%32,
// lane%32 + 32, ... so any width that is a multiple of 64 works.
__global__ void __launch_bounds__(256) k_decode_gate_up(const float *__restrict__ X, const uint8_t *__restrict__ arena,
                                                        uint64_t stride, const uint8_t *__restrict__ shared_blob,
                                                        const int *__restrict__ ids, float *__restrict__ hidden,
                                                        int width, int ff, int topk, int experts, uint64_t gu_scales) {
    extern __shared__ float xs[];  // [width] x, then [width/64] group sums
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = width / 64, half = lane >> 5, gl = lane & 31;
    float *xg = xs + width;
    for (int i = tid * 4; i < width; i += 1024) *(float4 *)(xs + i) = *(const float4 *)(X + i);
    __syncthreads();
    for (int g = tid; g < G; g += 256) {
        float s = 0.0f;
        for (int i = 0; i < 64; i++) s += xs[g * 64 + i];
        xg[g] = s;
    }
    __syncthreads();
    const int k = blockIdx.y;
    const uint8_t *blob = expert_blob(arena, stride, shared_blob, ids, k, topk, experts);
    const uint64_t row_bytes = (uint64_t)width / 4;
    const int j0 = blockIdx.x * 16 + wave * 4;
    for (int jj = 0; jj < 4; jj++) {
        const int j = j0 + jj;
        if (j >= ff) break;
        const int wrow = 2 * j + half;  // interleaved gate/up weight row
        float v = blob ? 0.0f : __builtin_nanf("");
        if (blob) {
            for (int g = gl; g < G; g += 32) {
                uint4 c = *(const uint4 *)(blob + (uint64_t)wrow * row_bytes + (uint64_t)g * 16);
                uint32_t sb = *(const uint16_t *)(blob + gu_scales + ((uint64_t)wrow * G + g) * 2);
                v = fmaf(sm::half_bits(sb), dot64(c, xs + g * 64) - xg[g], v);
            }
        }
        // reduce within each half-wave (32 lanes)
#pragma unroll
        for (int s = 16; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
        float u = __shfl(v, 32, 64);
        if (lane == 0) hidden[(uint64_t)k * ff + j] = sm::silu(v) * u;
    }
}

// Grid: width / 8 blocks of 256 threads; each wave handles experts
// k = wave, wave + 4, ... for the block's 8 rows. Dynamic LDS: hidden of all
// topk + 1 experts, their 64-group sums and the per-expert partial rows.
__global__ void __launch_bounds__(256) k_decode_down(const float *__restrict__ hidden, const uint8_t *__restrict__ arena,
                                                     uint64_t stride, const uint8_t *__restrict__ shared_blob,
                                                     const int *__restrict__ ids, const float *__restrict__ weights,
                                                     const float *__restrict__ gate, float *__restrict__ Y, int width,
                                                     int ff, int topk, int experts, uint64_t down_codes,
                                                     uint64_t down_scales) {
    extern __shared__ float lds[];
    const int nexp = topk + 1, GF = ff / 64;
    float *hs = lds;                             // [nexp][ff]
    float *hsum = hs + (size_t)nexp * ff;        // [nexp][GF]
    float *parts = hsum + (size_t)nexp * GF;     // [nexp][8]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid * 4; i < nexp * ff; i += 1024) *(float4 *)(hs + i) = *(const float4 *)(hidden + i);
    __syncthreads();
    for (int q = tid; q < nexp * GF; q += 256) {
        const float *h = hs + (size_t)(q / GF) * ff + (q % GF) * 64;
        float s = 0.0f;
        for (int i = 0; i < 64; i++) s += h[i];
        hsum[q] = s;
    }
    __syncthreads();
    const int r = blockIdx.x * 8 + (lane >> 3), gl = lane & 7;
    const uint64_t row_bytes = (uint64_t)ff / 4;
    for (int k = wave; k < nexp; k += 4) {
        const uint8_t *blob = expert_blob(arena, stride, shared_blob, ids, k, topk, experts);
        float v = blob ? 0.0f : __builtin_nanf("");
        if (blob && r < width) {
            for (int g = gl; g < GF; g += 8) {
                uint4 c = *(const uint4 *)(blob + down_codes + (uint64_t)r * row_bytes + (uint64_t)g * 16);
                uint32_t sb = *(const uint16_t *)(blob + down_scales + ((uint64_t)r * GF + g) * 2);
                v = fmaf(sm::half_bits(sb), dot64(c, hs + (size_t)k * ff + g * 64) - hsum[k * GF + g], v);
            }
        }
#pragma unroll
        for (int s = 4; s > 0; s >>= 1) v += __shfl_xor(v, s, 64);
        if (gl == 0) parts[k * 8 + (lane >> 3)] = v;
    }
    __syncthreads();
    if (tid < 8) {
        const int row = blockIdx.x * 8 + tid;
        if (row < width) {
            float value = parts[topk * 8 + tid] * sm::sigmoid(gate[0]);
            for (int k = 0; k < topk; k++) value = value + parts[k * 8 + tid] * weights[k];
            Y[row] = value;
        }
    }
}

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct DecodeWs {
    uint64_t logits, gate, hidden, end;
};
DecodeWs decode_ws(int width, int ff, int experts, int topk) {
    (void)width;
    DecodeWs w;
    w.logits = 0;
    w.gate = up(w.logits + (uint64_t)experts * 4);
    w.hidden = up(w.gate + 4);
    w.end = up(w.hidden + (uint64_t)(topk + 1) * ff * 4);
    return w;
}

}  // namespace

namespace smi {

uint64_t moe_decode_workspace(int width, int ff, int experts, int topk) { return decode_ws(width, ff, experts, topk).end; }

int moe_decode(sm_ctx *ctx, uint64_t X, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
               uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y, uint64_t ids,
               uint64_t weights, uint64_t workspace, uint64_t workspace_bytes) {
    (void)workspace_bytes;
    DecodeWs w = decode_ws(width, ff, experts, topk);
    char *ws = (char *)workspace;
    BlobLayout L = blob_layout(width, ff);
    const size_t down_lds = ((size_t)(topk + 1) * ff + (size_t)(topk + 1) * (ff / 64) + (size_t)(topk + 1) * 8) * 4;
    if ((width + width / 64) * 4 > 64 * 1024 || down_lds > 64 * 1024)
        return fail(ctx, SM_E_ARG, "decode geometry exceeds the 64 KiB LDS budget of one workgroup");
    // 1. routing (ids/weights) + shared gate logit; logits kept in the workspace.
    if (int rc = route_launch(ctx, (const float *)X, 1, width, (const float *)Wr, (const float *)bias, experts, topk,
                              (float *)(ws + w.logits), (int *)ids, (float *)weights, (const float *)Wsg,
                              (float *)(ws + w.gate)))
        return rc;
    // 2. gate/up for the routed experts and the shared expert.
    dim3 g1((unsigned)ceil_div(ff, 16), (unsigned)(topk + 1));
    k_decode_gate_up<<<g1, 256, (size_t)(width + width / 64) * 4, ctx->stream>>>(
        (const float *)X, (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob, (const int *)ids,
        (float *)(ws + w.hidden), width, ff, topk, experts, L.gate_up_scales);
    if (int rc = launched(ctx)) return rc;
    // 3. down for all experts + combine.
    k_decode_down<<<(unsigned)ceil_div(width, 8), 256, down_lds, ctx->stream>>>(
        (const float *)(ws + w.hidden), (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob,
        (const int *)ids, (const float *)weights, (const float *)(ws + w.gate), (float *)Y, width, ff, topk, experts,
        L.down_codes, L.down_scales);
    return launched(ctx);
}

}  // namespace smi
