// One MoE layer for a single token (decode), three kernels, no host round trip:
//
//   K1 k_decode_route   router logits and the shared-expert gate logit in the
//                       reference's exact f32 order (one wave per row), and, in
//                       extra blocks of the same grid, the shared expert's
//                       gate/up rows (they do not depend on the routing).
//   K2 k_decode_gate_up every block first runs the top-k over the 512 logits
//                       (router_wave, identical in every block; block 0 also
//                       publishes ids / weights), then computes hidden rows
//                       SiLU(g_j . x) * (u_j . x) of one routed expert.
//   K3 k_decode_down    each block owns 8 output rows for all topk+1 experts,
//                       then combines them in the reference order
//                       (kernels/strata.cu:360-365):
//                       y = shared * sigmoid(gate) + sum_k part_k * w_k.
//
// Kernel boundaries are the synchronisation: on MI355X a kernel in a graph
// costs ~1.6 us even when empty, while a device-scope release fence per block
// (needed for an in-kernel completion counter) costs far more at 500 blocks.
// Running the top-k redundantly in every gate/up block removes one boundary.
//
// Q2 GEMV layout: a 64-weight scale group of one row is 16 bytes of codes, so
// one lane reads one group with one 16-byte load. In gate/up the 32 lanes of
// each half-wave cover the 32 groups of a 2048-wide row (gate row in lanes
// 0-31, the adjacent up row in lanes 32-63: 1 KiB contiguous per wave); in
// down 8 lanes cover the 8 groups of a 512-wide row and a wave covers 8 rows.
// Per group the lane accumulates sum(c_i * x_i) over the raw codes c in {0..3}
// and applies scale * (sum - sum(x_i)) = sum((c_i - 1) * scale * x_i). Every
// load of a wave is issued before its arithmetic; reductions use DPP.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

// acc += sum over the 16 codes of word w of code * x[i] (code i at bits 2i).
__device__ __forceinline__ float dot16(uint32_t w, const float *x, float acc) {
#pragma unroll
    for (int i = 0; i < 16; i++) acc = fmaf((float)((w >> (2 * i)) & 3u), x[i], acc);
    return acc;
}
// sum_{i<64} code_i * x_i for one 16-byte code group (two chains for ILP).
__device__ __forceinline__ float dot64(uint4 c, const float *x) {
    float a = dot16(c.x, x, 0.0f), b = dot16(c.y, x + 16, 0.0f);
    a = dot16(c.z, x + 32, a);
    b = dot16(c.w, x + 48, b);
    return a + b;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// One 16-byte code group, streamed (non-temporal: weights are read once).
__device__ __forceinline__ uint4 load_codes(const uint8_t *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void load_group(const float *src, float *x) {
#pragma unroll
    for (int q = 0; q < 16; q++) {
        float4 v = *(const float4 *)(src + 4 * q);
        x[4 * q] = v.x;
        x[4 * q + 1] = v.y;
        x[4 * q + 2] = v.z;
        x[4 * q + 3] = v.w;
    }
}
__device__ __forceinline__ float sum64(const float *x) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 64; i += 2) {
        a += x[i];
        b += x[i + 1];
    }
    return a + b;
}

// Blob of expert slot k (k < topk: routed ID id; k == topk: shared). An ID
// outside [0, experts) (only possible for non-finite router input) yields
// nullptr and the slot produces NaN instead of reading out of bounds.
__device__ __forceinline__ const uint8_t *slot_blob(const uint8_t *arena, uint64_t stride, const uint8_t *shared,
                                                    int id, int k, int topk, int experts) {
    if (k >= topk) return shared;
    return id >= 0 && id < experts ? arena + (uint64_t)id * stride : nullptr;
}

constexpr int GU_ROWS = 4;  // hidden rows per wave
constexpr int GU_WAVES = 4; // waves per block -> 16 hidden rows per block

// The activations of a lane's first group (group lane % 32), loaded before
// the expert is known so the loads overlap the routing.
struct XFirst {
    float x[64];
    float xs;
};
__device__ __forceinline__ void load_x_first(const float *__restrict__ X, int width, XFirst &f) {
    const int gl = threadIdx.x & 31;
    f.xs = 0.0f;
    if (gl < width / 64) {
        load_group(X + gl * 64, f.x);
        f.xs = sum64(f.x);
    }
}

// Four hidden rows j0..j0+3 of one expert by one wave (width <= 2048 in one
// pass of the 32 lanes of each half-wave; wider rows loop over groups).
__device__ __forceinline__ void gate_up_rows(const float *__restrict__ X, const XFirst &xf, const uint8_t *blob,
                                             uint64_t gu_scales, float *__restrict__ hidden_row, int j0, int width,
                                             int ff, const uint64_t *tab) {
    const int lane = threadIdx.x & 63, half = lane >> 5, gl = lane & 31;
    const int G = width / 64;
    const uint64_t row_bytes = (uint64_t)width / 4;
    float acc[GU_ROWS];
#pragma unroll
    for (int r = 0; r < GU_ROWS; r++) acc[r] = 0.0f;
    auto group = [&](int g, const float *x, float xs) {
        uint4 c[GU_ROWS];
        uint32_t sb[GU_ROWS];
#pragma unroll
        for (int r = 0; r < GU_ROWS; r++) {
            const int wrow = 2 * min(j0 + r, ff - 1) + half;
            c[r] = load_codes(blob + (uint64_t)wrow * row_bytes + (uint64_t)g * 16);
            sb[r] = *(const uint16_t *)(blob + gu_scales + ((uint64_t)wrow * G + g) * 2);
        }
#pragma unroll
        for (int r = 0; r < GU_ROWS; r++) acc[r] = fmaf(sm::half_bits(sb[r]), dot64(c[r], x) - xs, acc[r]);
    };
    if (blob) {
        if (gl < G) group(gl, xf.x, xf.xs);
        for (int g = gl + 32; g < G; g += 32) {
            float x[64];
            load_group(X + g * 64, x);
            group(g, x, sum64(x));
        }
    }
#pragma unroll
    for (int r = 0; r < GU_ROWS; r++) {
        const float v = sm::half32_sum(acc[r]);  // lane 31: gate row, lane 63: up row
        const float g = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
        const float u = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        const int j = j0 + r;
        if (lane == 0 && j < ff) hidden_row[j] = blob ? sm::silu(g, tab) * u : __builtin_nanf("");
    }
}

// K1. Blocks [0, route_blocks): 4 router rows each (row `experts` = shared
// gate, exact reference order). Blocks after that: shared-expert gate/up,
// 16 hidden rows per block.
template <int NJ>
__global__ void __launch_bounds__(256) k_decode_route(const float *__restrict__ X, const float *__restrict__ Wr,
                                                      const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                      const uint8_t *__restrict__ shared_blob,
                                                      float *__restrict__ logits, float *__restrict__ gate_out,
                                                      float *__restrict__ hidden_shared, int width, int ff,
                                                      int experts, int route_blocks, uint64_t gu_scales) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if ((int)blockIdx.x >= route_blocks) {
        __shared__ uint64_t s_tab[32];
        XFirst xf;
        load_x_first(X, width, xf);
        if (threadIdx.x < 32) s_tab[threadIdx.x] = sm::kExp2Tab[threadIdx.x];
        __syncthreads();
        const int j0 = ((blockIdx.x - route_blocks) * GU_WAVES + wave) * GU_ROWS;
        if (j0 < ff) gate_up_rows(X, xf, shared_blob, gu_scales, hidden_shared, j0, width, ff, s_tab);
        return;
    }
    const int row = blockIdx.x * 4 + wave;
    if (row > experts) return;
    const float *w = row < experts ? Wr + (int64_t)row * width : Wsg;
    float sum = 0.0f;
    if (NJ > 0) {
        float wv[NJ > 0 ? NJ : 1], xv[NJ > 0 ? NJ : 1];
#pragma unroll
        for (int j = 0; j < NJ; j++) wv[j] = __builtin_nontemporal_load(w + lane + 64 * j);
#pragma unroll
        for (int j = 0; j < NJ; j++) xv[j] = X[lane + 64 * j];
#pragma unroll
        for (int j = 0; j < NJ; j++) sum = sum + wv[j] * xv[j];
    } else {
        for (int i = lane; i < width; i += 64) sum = sum + w[i] * X[i];
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) {
        if (row < experts) logits[row] = bias ? sum + bias[row] : sum;
        else gate_out[0] = sum;
    }
}

// K2. Grid (ceil(ff / 16), topk). Wave 0 runs the top-k into LDS (block (0,0)
// also writes ids / weights to memory); then every wave computes 4 hidden
// rows of routed expert blockIdx.y.
__global__ void __launch_bounds__(256) k_decode_gate_up(const float *__restrict__ X, const uint8_t *__restrict__ arena,
                                                        uint64_t stride, const float *__restrict__ logits,
                                                        int *__restrict__ ids, float *__restrict__ weights,
                                                        float *__restrict__ hidden, int width, int ff, int topk,
                                                        int experts, uint64_t gu_scales) {
    __shared__ int s_ids[32];
    __shared__ float s_w[32];
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    const int wave = threadIdx.x >> 6;
    const bool publish = blockIdx.x == 0 && blockIdx.y == 0;
    XFirst xf;
    load_x_first(X, width, xf);
    if (threadIdx.x < 32) s_tab[threadIdx.x] = sm::kExp2Tab[threadIdx.x];
    sm::router_block(logits, experts, topk, s_tab, s_router, s_ids, s_w);
    __syncthreads();
    if (publish && (int)threadIdx.x < topk) {
        ids[threadIdx.x] = s_ids[threadIdx.x];
        weights[threadIdx.x] = s_w[threadIdx.x];
    }
    const int k = blockIdx.y;
    const uint8_t *blob = slot_blob(arena, stride, nullptr, s_ids[k], k, topk, experts);
    const int j0 = (blockIdx.x * GU_WAVES + wave) * GU_ROWS;
    if (j0 < ff) gate_up_rows(X, xf, blob, gu_scales, hidden + (uint64_t)k * ff, j0, width, ff, s_tab);
}

// K3. Grid ceil(width / 8), 256 threads: wave w handles experts w, w+4, ...
// Lane (r = lane / 8, gl = lane % 8) covers groups gl, gl+8, ... of down row
// r. All code loads of a wave are issued first; partial rows go to LDS and are
// combined in the reference order.
constexpr int DN_MAX_SLOTS = 9;  // experts per wave with up-front loads (33 slots / 4 waves)
__global__ void __launch_bounds__(256) k_decode_down(const float *__restrict__ hidden, const uint8_t *__restrict__ arena,
                                                     uint64_t stride, const uint8_t *__restrict__ shared_blob,
                                                     const int *__restrict__ ids, const float *__restrict__ weights,
                                                     const float *__restrict__ gate, float *__restrict__ Y, int width,
                                                     int ff, int topk, int experts, uint64_t down_codes,
                                                     uint64_t down_scales) {
    __shared__ float parts[33 * 8];
    __shared__ uint64_t s_tab[32];
    const int nexp = topk + 1, GF = ff / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 32) s_tab[tid] = sm::kExp2Tab[tid];
    const int r = min((int)blockIdx.x * 8 + (lane >> 3), width - 1), gl = lane & 7;
    const uint64_t row_bytes = (uint64_t)ff / 4;
    if (GF <= 8) {
        // One group per lane: issue every code load of this wave first.
        uint4 c[DN_MAX_SLOTS];
        uint32_t sb[DN_MAX_SLOTS];
        const uint8_t *blobs[DN_MAX_SLOTS];
#pragma unroll
        for (int q = 0; q < DN_MAX_SLOTS; q++) {
            const int k = wave + 4 * q;
            blobs[q] = nullptr;
            c[q] = make_uint4(0, 0, 0, 0);
            sb[q] = 0;
            if (k < nexp) {
                blobs[q] = slot_blob(arena, stride, shared_blob, k < topk ? ids[k] : 0, k, topk, experts);
                if (blobs[q] && gl < GF) {
                    c[q] = load_codes(blobs[q] + down_codes + (uint64_t)r * row_bytes + (uint64_t)gl * 16);
                    sb[q] = *(const uint16_t *)(blobs[q] + down_scales + ((uint64_t)r * GF + gl) * 2);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < DN_MAX_SLOTS; q++) {
            const int k = wave + 4 * q;
            if (k >= nexp) break;
            float v = blobs[q] ? 0.0f : __builtin_nanf("");
            if (blobs[q] && gl < GF) {
                float h[64];
                load_group(hidden + (uint64_t)k * ff + gl * 64, h);
                v = sm::half_bits(sb[q]) * (dot64(c[q], h) - sum64(h));
            }
            v = sm::group8_sum(v);
            if (gl == 0) parts[k * 8 + (lane >> 3)] = v;
        }
    } else {
        for (int k = wave; k < nexp; k += 4) {
            const uint8_t *blob = slot_blob(arena, stride, shared_blob, k < topk ? ids[k] : 0, k, topk, experts);
            float v = blob ? 0.0f : __builtin_nanf("");
            if (blob) {
                for (int g = gl; g < GF; g += 8) {
                    const uint4 c = load_codes(blob + down_codes + (uint64_t)r * row_bytes + (uint64_t)g * 16);
                    const uint32_t sb = *(const uint16_t *)(blob + down_scales + ((uint64_t)r * GF + g) * 2);
                    float h[64];
                    load_group(hidden + (uint64_t)k * ff + g * 64, h);
                    v = fmaf(sm::half_bits(sb), dot64(c, h) - sum64(h), v);
                }
            }
            v = sm::group8_sum(v);
            if (gl == 0) parts[k * 8 + (lane >> 3)] = v;
        }
    }
    __syncthreads();
    if (tid < 8) {
        const int row = blockIdx.x * 8 + tid;
        if (row < width) {
            float value = parts[topk * 8 + tid] * sm::sigmoid(gate[0], s_tab);
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
    float *hidden = (float *)(ws + w.hidden);
    const int blocks_per_expert = ceil_div(ff, GU_ROWS * GU_WAVES);
    // 1. router logits + shared gate logit + shared-expert gate/up
    if (stage_on(ctx, kStageDecodeRoute)) {
        if (int rc = stage_mark(ctx, kStageDecodeRoute)) return rc;
        const int route_blocks = ceil_div(experts + 1, 4);
        const unsigned grid = (unsigned)(route_blocks + blocks_per_expert);
        if (width == 2048)
            k_decode_route<32><<<grid, 256, 0, ctx->stream>>>(
                (const float *)X, (const float *)Wr, (const float *)bias, (const float *)Wsg,
                (const uint8_t *)shared_blob, (float *)(ws + w.logits), (float *)(ws + w.gate),
                hidden + (uint64_t)topk * ff, width, ff, experts, route_blocks, L.gate_up_scales);
        else
            k_decode_route<0><<<grid, 256, 0, ctx->stream>>>(
                (const float *)X, (const float *)Wr, (const float *)bias, (const float *)Wsg,
                (const uint8_t *)shared_blob, (float *)(ws + w.logits), (float *)(ws + w.gate),
                hidden + (uint64_t)topk * ff, width, ff, experts, route_blocks, L.gate_up_scales);
        if (int rc = launched(ctx)) return rc;
    }
    // 2. top-k (per block) + gate/up of the routed experts
    if (stage_on(ctx, kStageDecodeGateUp)) {
        if (int rc = stage_mark(ctx, kStageDecodeGateUp)) return rc;
        dim3 g1((unsigned)blocks_per_expert, (unsigned)topk);
        k_decode_gate_up<<<g1, 64 * GU_WAVES, 0, ctx->stream>>>((const float *)X, (const uint8_t *)arena, blob_stride,
                                                                (const float *)(ws + w.logits), (int *)ids,
                                                                (float *)weights, hidden, width, ff, topk, experts,
                                                                L.gate_up_scales);
        if (int rc = launched(ctx)) return rc;
    }
    // 3. down for all experts + combine
    if (stage_on(ctx, kStageDecodeDown)) {
        if (int rc = stage_mark(ctx, kStageDecodeDown)) return rc;
        k_decode_down<<<(unsigned)ceil_div(width, 8), 256, 0, ctx->stream>>>(
            hidden, (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob, (const int *)ids,
            (const float *)weights, (const float *)(ws + w.gate), (float *)Y, width, ff, topk, experts, L.down_codes,
            L.down_scales);
        if (int rc = launched(ctx)) return rc;
    }
    return stage_mark(ctx, -1);
}

}  // namespace smi
