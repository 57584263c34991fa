// One MoE layer for a single token (decode), three kernels, no host round trip:
//
//   K1 k_decode_route   router logits and the shared-expert gate logit in the
//                       reference's exact f32 order (one wave per row), and, in
//                       extra blocks of the same grid, the token's activations
//                       as per-group fixed point for the integer gate/up dots.
//   K2 k_decode_gate_up hidden rows SiLU(g_j . x) * (u_j . x) of the topk
//                       routed experts and the shared one (grid.y = slot).
//                       Routed blocks first run the top-k over the logits
//                       (router_block, identical in every block; block (0,0)
//                       publishes ids / weights); shared blocks start at once.
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
// and applies scale * (sum - sum(x_i)) = sum((c_i - 1) * scale * x_i): with
// int8 dot products against fixed-point x in gate/up, in f32 in down. Every
// load of a wave is issued before its arithmetic; reductions use DPP.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

// acc += sum over the 16 codes of word w of code * x[i] (code i at bits 2i).
// (w >> 2k) & 0x03030303 holds codes k, 4+k, 8+k, 12+k in its four bytes,
// which v_cvt_f32_ubyte0..3 convert directly; the empty asm keeps the
// compiler from folding the mask back into one bit-field extract per code.
__device__ __forceinline__ float dot16(uint32_t w, const float *x, float acc) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t m = (w >> (2 * k)) & 0x03030303u;
        asm("" : "+v"(m));
        acc = fmaf((float)(m & 255u), x[k], acc);
        acc = fmaf((float)((m >> 8) & 255u), x[4 + k], acc);
        acc = fmaf((float)((m >> 16) & 255u), x[8 + k], acc);
        acc = fmaf((float)(m >> 24), x[12 + k], acc);
    }
    return acc;
}
// sum_{i<64} code_i * x_i for one 16-byte code group (two chains for ILP).
__device__ __forceinline__ float dot64(uint4 c, const float *x) {
    float a = dot16(c.x, x, 0.0f), b = dot16(c.y, x + 16, 0.0f);
    a = dot16(c.z, x + 32, a);
    b = dot16(c.w, x + 48, b);
    return a + b;
}
// The same with four independent chains (one per code word).
__device__ __forceinline__ float dot64_4(uint4 c, const float *x) {
    const float a = dot16(c.x, x, 0.0f), b = dot16(c.y, x + 16, 0.0f);
    const float d = dot16(c.z, x + 32, 0.0f), e = dot16(c.w, x + 48, 0.0f);
    return (a + b) + (d + e);
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

// ---------------------------------------------------------------- gate/up
// The gate/up products run on integer dot products. Each 64-value group g of
// the token's activations is stored once per step as fixed point:
//   X_i = rint(x_i * 2^(21 - E_g)),  2^E_g <= max_i |x_i| < 2^(E_g + 1),
// so |X_i| <= 2^22, split into three balanced base-256 limbs
// X_i = x0_i + 256 x1_i + 65536 x2_i (each an int8). A 16-code word w of a
// row holds code 4b + k in byte b of (w >> 2k) & 0x03030303, so one
// v_dot4_i32_i8 of that mask with the limb bytes of x positions
// {k, 4 + k, 8 + k, 12 + k} adds four code * limb products. Per group:
//   sum_i (c_i - 1) X_i = sum_l 256^l sum_i c_i xl_i - sum_i X_i
// exactly (modulo 2^32 arithmetic; the true value is below 2^30), and the
// group's contribution is scale_g * (that integer) * 2^(E_g - 21). The only
// rounding beyond f32 arithmetic is X_i itself (relative 2^-22 of the
// group's largest value).
constexpr int XQ_WORDS = 64;  // per group: 48 limb words, scale, sum, padding
struct XQ {
    uint32_t limb[48];  // limb[16 l + 4 q + k] byte b: limb l of x[16 q + 4 b + k]
    float unit;         // 2^(E_g - 21) (0 for an all-zero group, NaN if non-finite)
    int sum;            // sum_i X_i
};
__device__ __forceinline__ void load_xq(const uint32_t *__restrict__ xq, int g, XQ &q) {
    const uint4 *p = (const uint4 *)(xq + (uint64_t)g * XQ_WORDS);
#pragma unroll
    for (int i = 0; i < 12; i++) {
        const uint4 v = p[i];
        q.limb[4 * i] = v.x;
        q.limb[4 * i + 1] = v.y;
        q.limb[4 * i + 2] = v.z;
        q.limb[4 * i + 3] = v.w;
    }
    const uint2 t = *(const uint2 *)(xq + (uint64_t)g * XQ_WORDS + 48);
    q.unit = __builtin_bit_cast(float, t.x);
    q.sum = (int)t.y;
}
// sum_i (c_i - 1) x_i of one 16-byte code group against quantized x.
__device__ __forceinline__ float dot64_q(uint4 c, const XQ &q) {
    int a0 = 0, a1 = 0, a2 = 0;
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int m = (int)((w[qq] >> (2 * k)) & 0x03030303u);
            a0 = __builtin_amdgcn_sdot4(m, (int)q.limb[4 * qq + k], a0, false);
            a1 = __builtin_amdgcn_sdot4(m, (int)q.limb[16 + 4 * qq + k], a1, false);
            a2 = __builtin_amdgcn_sdot4(m, (int)q.limb[32 + 4 * qq + k], a2, false);
        }
    }
    const uint32_t d = (uint32_t)a0 + ((uint32_t)a1 << 8) + ((uint32_t)a2 << 16) - (uint32_t)q.sum;
    return (float)(int)d * q.unit;
}

// Quantizes group g of X (one wave, lane i <-> x[64 g + i]) into its record.
// `bytes` is 192 bytes of this wave's LDS; the caller synchronises the block
// between the two halves (writes to LDS, then the packed words to memory).
__device__ __forceinline__ void quantize_group_bytes(float x, uint8_t *bytes, float &unit, int &sum) {
    const int lane = threadIdx.x & 63;
    const bool bad = __ballot(!(fabsf(x) <= 3.402823466e38f)) != 0;
    const float m = sm::wave_max(fabsf(x));
    int X_ = 0;
    unit = 0.0f;
    if (bad) {
        unit = __builtin_nanf("");
    } else if (m > 0.0f) {
        const int E = __builtin_amdgcn_frexp_expf(m) - 1;
        X_ = (int)__builtin_rintf(__builtin_amdgcn_ldexpf(x, 21 - E));
        unit = __builtin_amdgcn_ldexpf(1.0f, E - 21);
    }
    const int l0 = ((X_ + 128) & 255) - 128;
    const int r1 = (X_ - l0) >> 8;
    const int l1 = ((r1 + 128) & 255) - 128;
    const int l2 = (r1 - l1) >> 8;
    const int q = lane >> 4, b = (lane >> 2) & 3, k = lane & 3;
    const int at = (4 * q + k) * 4 + b;
    bytes[at] = (uint8_t)l0;
    bytes[64 + at] = (uint8_t)l1;
    bytes[128 + at] = (uint8_t)l2;
    sum = sm::wave_sum_i32(X_);
}

// RMSNorm of one row by one wave, exactly as strata_norm mode 0 with scale 1
// (kernels/strata.cu:214-227): lane-strided sum of squares, the 64-lane
// tree, inv = 1 / sqrt(ss / cols + eps); element i is then (x_i * inv) * g_i.
__device__ __forceinline__ float rms_inv_wave(const float *__restrict__ x, int cols, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.0f;
    for (int i0 = lane; i0 < cols; i0 += 8 * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = x[min(i0 + 64 * u, cols - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + 64 * u < cols) ss = ss + v[u] * v[u];
    }
    ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm::tree_sum64(ss)), 0));
    return 1.0f / sqrtf(ss / (float)cols + eps);
}

constexpr int GU_ROWS = 4;  // hidden rows per wave
constexpr int GU_WAVES = 4; // waves per block -> 16 hidden rows per block

// Four hidden rows j0..j0+3 of one expert by one wave. Lane (half = lane/32,
// gl = lane%32) covers group gl (then gl + 32, ...) of gate row j (half 0)
// or up row j (half 1); `first` is the lane's first group, loaded early.
template <bool EXTRA>
__device__ __forceinline__ void gate_up_rows(const uint32_t *__restrict__ xq, const XQ &first, const XQ &second,
                                             const uint8_t *blob,
                                             uint64_t gu_scales, float *__restrict__ hidden_row, int j0, int width,
                                             int ff, const uint64_t *tab) {
    const int lane = threadIdx.x & 63, half = lane >> 5, gl = lane & 31;
    const int G = width / 64;
    const uint64_t row_bytes = (uint64_t)width / 4;
    float acc[GU_ROWS];
#pragma unroll
    for (int r = 0; r < GU_ROWS; r++) acc[r] = 0.0f;
    auto group = [&](int g, const XQ &q) {
        uint4 c[GU_ROWS];
        uint32_t sb[GU_ROWS];
#pragma unroll
        for (int r = 0; r < GU_ROWS; r++) {
            const int wrow = 2 * min(j0 + r, ff - 1) + half;
            c[r] = load_codes(blob + (uint64_t)wrow * row_bytes + (uint64_t)g * 16);
            sb[r] = *(const uint16_t *)(blob + gu_scales + ((uint64_t)wrow * G + g) * 2);
        }
#pragma unroll
        for (int r = 0; r < GU_ROWS; r++) acc[r] = fmaf(sm::half_bits(sb[r]), dot64_q(c[r], q), acc[r]);
    };
    if (blob) {
        if (gl < G) group(gl, first);
        if (EXTRA) {
            // 33-40 groups (the real model's 2560 = 40): the (row, group)
            // pairs of groups 32.. are spread one per lane instead of a
            // second pass over the first lanes, so every lane makes five code
            // loads. `second` is the lane's record, loaded with `first`.
            const int G2 = G - 32, item = gl < 4 * G2 ? gl : 0, r2 = item / G2, g2 = 32 + item % G2;
            const int wrow = 2 * min(j0 + r2, ff - 1) + half;
            const uint4 c = load_codes(blob + (uint64_t)wrow * row_bytes + (uint64_t)g2 * 16);
            const uint32_t sb = *(const uint16_t *)(blob + gu_scales + ((uint64_t)wrow * G + g2) * 2);
            const float v = gl < 4 * G2 ? sm::half_bits(sb) * dot64_q(c, second) : 0.0f;
#pragma unroll
            for (int r = 0; r < GU_ROWS; r++) acc[r] += r == r2 ? v : 0.0f;
        } else {
            for (int g = gl + 32; g < G; g += 32) {
                XQ q;
                load_xq(xq, g, q);
                group(g, q);
            }
        }
    }
    // Row r's gate and up sums (lanes 31 and 63 after the half-wave sums)
    // go to lane r, so the rows' SiLU run side by side and one store writes them.
    float g = 0.0f, u = 0.0f;
#pragma unroll
    for (int r = 0; r < GU_ROWS; r++) {
        const float v = sm::half32_sum(acc[r]);
        const float gr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
        const float ur = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
        g = lane == r ? gr : g;
        u = lane == r ? ur : u;
    }
    const int j = j0 + lane;
    if (lane < GU_ROWS && j < ff) hidden_row[j] = blob ? sm::silu(g, tab) * u : __builtin_nanf("");
}

// K1. Blocks [0, route_blocks): 4 router rows each (row `experts` = shared
// gate), one wave per row in the reference's exact f32 order. Blocks after
// that: one wave per 64-value group of X writes the group's fixed-point record.
// NORM: the layer input is RMSNorm(X; gamma, eps) (strata_norm mode 0), which
// every wave forms itself from X, bit-identical to the separate kernel.
template <int NJ, bool NORM>
__global__ void __launch_bounds__(256) k_decode_route(const float *__restrict__ X, const float *__restrict__ Wr,
                                                      const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                      float *__restrict__ logits, float *__restrict__ gate_out,
                                                      uint32_t *__restrict__ xq, int width, int experts,
                                                      int route_blocks, const float *__restrict__ gamma, float eps) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    {  // token blockIdx.y
        const int t = blockIdx.y;
        X += (int64_t)t * width;
        logits += (int64_t)t * experts;
        gate_out += t;
        xq += (uint64_t)t * (width / 64) * XQ_WORDS;
    }
    if ((int)blockIdx.x >= route_blocks) {
        __shared__ uint8_t s_bytes[4][192];
        const int g = ((int)blockIdx.x - route_blocks) * 4 + wave;  // past the groups: padding blocks
        const bool live = g < width / 64;
        float unit = 0.0f;
        int sum = 0;
        if (live) {
            const int i = g * 64 + lane;
            float x = X[i];
            if (NORM) x = (x * rms_inv_wave(X, width, eps)) * gamma[i];
            quantize_group_bytes(x, s_bytes[wave], unit, sum);
        }
        __syncthreads();
        if (live) {
            uint32_t *rec = xq + (uint64_t)g * XQ_WORDS;
            if (lane < 48) rec[lane] = ((const uint32_t *)s_bytes[wave])[lane];
            else if (lane == 48) rec[48] = __builtin_bit_cast(uint32_t, unit);
            else if (lane == 49) rec[49] = (uint32_t)sum;
        }
        return;
    }
    const int row = blockIdx.x * 4 + wave;
    if (row > experts) return;
    const float *w = row < experts ? Wr + (int64_t)row * width : Wsg;
    float sum = 0.0f;
    if (NJ > 0) {
        float wv[NJ > 0 ? NJ : 1], xv[NJ > 0 ? NJ : 1], gv[NJ > 0 && NORM ? NJ : 1];
#pragma unroll
        for (int j = 0; j < NJ; j++) wv[j] = __builtin_nontemporal_load(w + lane + 64 * j);
#pragma unroll
        for (int j = 0; j < NJ; j++) xv[j] = X[lane + 64 * j];
        if (NORM) {
#pragma unroll
            for (int j = 0; j < NJ; j++) gv[j] = gamma[lane + 64 * j];
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < NJ; j++) ss = ss + xv[j] * xv[j];
            ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm::tree_sum64(ss)), 0));
            const float inv = 1.0f / sqrtf(ss / (float)width + eps);
#pragma unroll
            for (int j = 0; j < NJ; j++) xv[j] = (xv[j] * inv) * gv[j];
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) sum = sum + wv[j] * xv[j];
    } else {
        const float inv = NORM ? rms_inv_wave(X, width, eps) : 1.0f;
        for (int i = lane; i < width; i += 64) sum = sum + w[i] * (NORM ? (X[i] * inv) * gamma[i] : X[i]);
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) {
        if (row < experts) logits[row] = bias ? sum + bias[row] : sum;
        else gate_out[0] = sum;
    }
}

// K2. Grid (ceil(ff / 16), topk + 1). Slot blockIdx.y < topk: wave 0 runs the
// top-k into LDS (block (0,0) also writes ids / weights to memory), then every
// wave computes 4 hidden rows of that routed expert. Slot topk is the shared
// expert and needs no routing.
// EXTRA: 33-40 groups per row (the real model's 2560), whose groups 32..
// are spread one (row, group) pair per lane.
template <bool EXTRA>
__global__ void __launch_bounds__(256) k_decode_gate_up(const uint32_t *__restrict__ xq,
                                                        const uint8_t *__restrict__ arena, uint64_t stride,
                                                        const uint8_t *__restrict__ shared_blob,
                                                        const float *__restrict__ logits, int *__restrict__ ids,
                                                        float *__restrict__ weights, float *__restrict__ hidden,
                                                        int width, int ff, int topk, int experts, uint64_t gu_scales,
                                                        int routed) {
    __shared__ int s_ids[32];
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    const int wave = threadIdx.x >> 6, gl = threadIdx.x & 31;
    const int k = blockIdx.y;
    {  // token blockIdx.z
        const int t = blockIdx.z;
        xq += (uint64_t)t * (width / 64) * XQ_WORDS;
        logits += (int64_t)t * experts;
        ids += (int64_t)t * topk;
        weights += (int64_t)t * topk;
        hidden += (uint64_t)t * (topk + 1) * ff;
    }
    // routed: the IDs are already in memory (a top-k kernel ran per token)
    // and the block reads its slot's ID instead of selecting it itself.
    float lg[8];
    if (k < topk && !routed) sm::router_load(logits, experts, lg);
    XQ first, second;
    load_xq(xq, min(gl, width / 64 - 1), first);  // unconditional: the wait for the logits leaves these in flight
    if (EXTRA) {
        // Groups 32..39 of widths 2112..2560: the lane's item of the second set.
        const int G2 = width / 64 - 32;
        load_xq(xq, 32 + (gl < 4 * G2 ? gl : 0) % G2, second);
    }
    sm::fill_exp_table(s_tab);
    if (k < topk && routed) {
        if (threadIdx.x == 0) s_ids[k] = ids[k];
    } else if (k < topk) {
        sm::router_block(lg, experts, topk, s_tab, s_router, s_ids);
    }
    __syncthreads();
    const uint8_t *blob = slot_blob(arena, stride, shared_blob, k < topk ? s_ids[k] : 0, k, topk, experts);
    const int j0 = (blockIdx.x * GU_WAVES + wave) * GU_ROWS;
    if (j0 < ff)
        gate_up_rows<EXTRA>(xq, first, second, blob, gu_scales, hidden + (uint64_t)k * ff, j0, width, ff, s_tab);
    // Block (0, 0) publishes the token's IDs and routing weights, after its
    // own expert work so that no block's loads wait for the weights.
    if (k == 0 && !routed && blockIdx.x == 0 && wave == 0) {
        const int lane = threadIdx.x;
        if (lane < topk) ids[lane] = s_ids[lane];
        sm::router_weights(lane < topk ? s_router.val[lane] : 0.0f, topk, weights);
    }
}

// K3, the combine at its end shared by both variants (kernels/strata.cu:360-365):
// y = shared * sigmoid(gate) + sum_k part_k * w_k, in that order.
// With `resid`, Y = resid + y (strata_elementwise mode 5, scale 1).
// Its inputs do not depend on the expert work, so they are loaded when the
// kernel starts (unconditional loads on valid addresses) and the tail after
// the last barrier makes no memory round trip: thread k < topk holds w_k,
// threads < 8 the gate and the residual of their row.
struct CombineIn {
    float w, gate, res;
};
template <int ROWS = 8>
__device__ __forceinline__ CombineIn combine_load(const float *__restrict__ weights, const float *__restrict__ gate,
                                                  const float *__restrict__ resid, int width, int topk) {
    const int tid = threadIdx.x;
    const int row = min((int)blockIdx.x * ROWS + (tid & 7) % ROWS, width - 1);
    CombineIn in;
    in.w = weights[min(tid, topk - 1)];
    in.gate = gate[0];
    in.res = *(resid ? resid + row : gate);
    return in;
}
// Before the last barrier: the weights into LDS and, in the combining
// threads, sigmoid(gate) (s_tab must hold this wave's copy of the table).
__device__ __forceinline__ float combine_stage(const CombineIn &in, float *s_w, int topk, const uint64_t *s_tab) {
    const int tid = threadIdx.x;
    if (tid < topk) s_w[tid] = in.w;
    return tid < 8 ? sm::sigmoid(in.gate, s_tab) : 0.0f;
}
// parts[k * ROWS + r]: slot k's value of the block's row r.
template <int ROWS = 8>
__device__ __forceinline__ void down_combine(const float *parts, const float *s_w, float sig, const CombineIn &in,
                                             float *__restrict__ Y, int width, int topk, bool has_resid) {
    const int tid = threadIdx.x;
    if (tid < ROWS) {
        const int row = blockIdx.x * ROWS + tid;
        if (row < width) {
            float value = parts[topk * ROWS + tid] * sig;
            for (int k = 0; k < topk; k++) value = value + parts[k * ROWS + tid] * s_w[k];
            Y[row] = has_resid ? in.res + value : value;
        }
    }
}

// K3 for ff <= 512 (one 64-value group per lane). Grid ceil(width / 8),
// 512 threads, 8 output rows per block. Wave w handles slots w, w+8, ...;
// lane (r = lane / 8, gl = lane % 8) dots group gl of down row r with group
// gl of the slot's hidden vector. The 8 lanes that need the same hidden
// group each load an eighth of it and pass it on through a wave-private LDS
// area (every hidden value is read from memory once per wave, not 8 times);
// the same 8 lanes form the group's sum with three cross-lane adds. Slot IDs
// are one vector load read back per slot with v_readlane; loads go out on
// clamped addresses without branches, so each wait covers only what it
// needs. Partial rows meet in LDS for the combine.
constexpr int DN_WAVES = 8;
constexpr int DN_MAX_SLOTS = 5;  // slots per wave (33 slots / 8 waves)
constexpr int DN_PITCH = 68;     // floats per group in the exchange area (16-byte skew per group)
template <int NQ>  // slots per wave: ceil((topk + 1) / DN_WAVES)
__global__ void __launch_bounds__(64 * DN_WAVES) k_decode_down(const float *__restrict__ hidden,
                                                              const uint8_t *__restrict__ arena, uint64_t stride,
                                                              const uint8_t *__restrict__ shared_blob,
                                                              const int *__restrict__ ids,
                                                              const float *__restrict__ weights,
                                                              const float *__restrict__ gate, float *__restrict__ Y,
                                                              int width, int ff, int topk, int experts,
                                                              uint64_t down_codes, uint64_t down_scales,
                                                              const float *__restrict__ resid) {
    static_assert(NQ >= 1 && NQ <= DN_MAX_SLOTS, "slots per wave");
    {  // token blockIdx.y
        const int t = blockIdx.y;
        hidden += (uint64_t)t * (topk + 1) * ff;
        ids += (int64_t)t * topk;
        weights += (int64_t)t * topk;
        gate += t;
        Y += (int64_t)t * width;
        if (resid) resid += (int64_t)t * width;
    }
    __shared__ float parts[33 * 8];
    __shared__ float s_w[32];
    __shared__ uint64_t s_tab[32];
    __shared__ __attribute__((aligned(16))) float s_h[DN_WAVES][8 * DN_PITCH];
    const int nexp = topk + 1, GF = ff / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rr = lane >> 3, gl = lane & 7;
    const int r = min((int)blockIdx.x * 8 + rr, width - 1);
    const int gc = min(gl, GF - 1);
    const uint64_t row_bytes = (uint64_t)ff / 4;
    const int my_id = ids[min(lane, topk - 1)];
    const CombineIn cin = combine_load(weights, gate, resid, width, topk);
    // The lane's eighth (8 values) of its hidden group, for every slot.
    float4 hq[NQ][2];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const float *src = hidden + (uint64_t)min(wave + DN_WAVES * q, nexp - 1) * ff + gc * 64 + 8 * rr;
        hq[q][0] = *(const float4 *)src;
        hq[q][1] = *(const float4 *)(src + 4);
    }
    uint4 c[NQ];
    uint32_t sb[NQ];
    bool ok[NQ];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int k = wave + DN_WAVES * q;
        const int lid = __builtin_amdgcn_readlane(my_id, min(k, 63));
        const int id = k < topk ? lid : 0;
        const uint8_t *blob = k < nexp ? slot_blob(arena, stride, shared_blob, id, k, topk, experts) : shared_blob;
        ok[q] = blob != nullptr;
        blob = blob ? blob : shared_blob;  // an invalid ID reads the shared blob; the slot yields NaN
        c[q] = load_codes(blob + down_codes + (uint64_t)r * row_bytes + (uint64_t)gc * 16);
        sb[q] = *(const uint16_t *)(blob + down_scales + ((uint64_t)r * GF + gc) * 2);
    }
    sm::fill_exp_table(s_tab);
    float *xh = s_h[wave];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int k = wave + DN_WAVES * q;
        // group sum: own eighth, then over the lanes gl + 8j: lane ^ 8
        // (row_ror:8 inside a 16-lane row), lane ^ 16 and lane ^ 32 (the two
        // results of a v_permlane16/32_swap of a value with itself hold, in
        // every lane, the lane's own value and its partner's).
        const float4 a = hq[q][0], b = hq[q][1];
        float s8 = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
        s8 = s8 + sm::dpp_f32<0x128>(0.0f, s8);
        {
            const int u = __builtin_bit_cast(int, s8);
            const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            s8 = __builtin_bit_cast(float, (int)p16[0]) + __builtin_bit_cast(float, (int)p16[1]);
            const int w = __builtin_bit_cast(int, s8);
            const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
            s8 = __builtin_bit_cast(float, (int)p32[0]) + __builtin_bit_cast(float, (int)p32[1]);
        }
        // exchange: lane (rr, gl) stores values 8 rr .. 8 rr + 7 of group gl
        *(float4 *)&xh[gl * DN_PITCH + 8 * rr] = a;
        *(float4 *)&xh[gl * DN_PITCH + 8 * rr + 4] = b;
        __builtin_amdgcn_wave_barrier();
        float h[64];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 v = *(const float4 *)&xh[gl * DN_PITCH + 4 * i];
            h[4 * i] = v.x;
            h[4 * i + 1] = v.y;
            h[4 * i + 2] = v.z;
            h[4 * i + 3] = v.w;
        }
        __builtin_amdgcn_wave_barrier();
        float v = ok[q] ? 0.0f : __builtin_nanf("");
        if (ok[q] && gl < GF) v = sm::half_bits(sb[q]) * (dot64_4(c[q], h) - s8);
        v = sm::group8_sum(v);
        if (gl == 0 && k < nexp) parts[k * 8 + rr] = v;
    }
    const float sig = combine_stage(cin, s_w, topk, s_tab);
    __syncthreads();
    down_combine(parts, s_w, sig, cin, Y, width, topk, resid != nullptr);
}

// K3 for 9-10 groups per down row (the real model's ff 640). Grid
// ceil(width / 6), 512 threads, 6 output rows per block; lane (rr = lane / 10,
// gl = lane % 10) dots group gl of down row rr with group gl of the slot's
// hidden vector (lanes 60-63 idle). Wave w handles slots w, w+8. A slot's
// hidden vector comes into a wave-private LDS area by one cooperative load
// (10 values per lane); the 10 partial sums of a row are added in order by
// its first lane through a wave-private LDS line.
constexpr int D10_ROWS = 6;
template <int NQ>
__global__ void __launch_bounds__(64 * DN_WAVES) k_decode_down10(const float *__restrict__ hidden,
                                                                const uint8_t *__restrict__ arena, uint64_t stride,
                                                                const uint8_t *__restrict__ shared_blob,
                                                                const int *__restrict__ ids,
                                                                const float *__restrict__ weights,
                                                                const float *__restrict__ gate, float *__restrict__ Y,
                                                                int width, int ff, int topk, int experts,
                                                                uint64_t down_codes, uint64_t down_scales,
                                                                const float *__restrict__ resid) {
    static_assert(NQ >= 1 && NQ <= DN_MAX_SLOTS, "slots per wave");
    {  // token blockIdx.y
        const int t = blockIdx.y;
        hidden += (uint64_t)t * (topk + 1) * ff;
        ids += (int64_t)t * topk;
        weights += (int64_t)t * topk;
        gate += t;
        Y += (int64_t)t * width;
        if (resid) resid += (int64_t)t * width;
    }
    __shared__ float parts[33 * D10_ROWS];
    __shared__ float s_w[32];
    __shared__ uint64_t s_tab[32];
    __shared__ __attribute__((aligned(16))) float s_h[DN_WAVES][10 * DN_PITCH];
    __shared__ float s_red[DN_WAVES][64];
    const int nexp = topk + 1, GF = ff / 64;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rr = lane / 10, gl = lane - 10 * rr;
    const bool live = rr < D10_ROWS && gl < GF;
    const int r = min((int)blockIdx.x * D10_ROWS + min(rr, D10_ROWS - 1), width - 1);
    const int gc = min(gl, GF - 1);
    const uint64_t row_bytes = (uint64_t)ff / 4;
    const int my_id = ids[min(lane, topk - 1)];
    const CombineIn cin = combine_load<D10_ROWS>(weights, gate, resid, width, topk);
    // Values 10 lane .. 10 lane + 9 of every slot's hidden vector (clamped
    // addresses past ff; those values are never stored).
    float2 hq[NQ][5];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const float *src = hidden + (uint64_t)min(wave + DN_WAVES * q, nexp - 1) * ff;
#pragma unroll
        for (int i = 0; i < 5; i++) hq[q][i] = *(const float2 *)(src + min(10 * lane + 2 * i, ff - 2));
    }
    uint4 c[NQ];
    uint32_t sb[NQ];
    bool ok[NQ];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int k = wave + DN_WAVES * q;
        const int lid = __builtin_amdgcn_readlane(my_id, min(k, 63));
        const int id = k < topk ? lid : 0;
        const uint8_t *blob = k < nexp ? slot_blob(arena, stride, shared_blob, id, k, topk, experts) : shared_blob;
        ok[q] = blob != nullptr;
        blob = blob ? blob : shared_blob;  // an invalid ID reads the shared blob; the slot yields NaN
        c[q] = load_codes(blob + down_codes + (uint64_t)r * row_bytes + (uint64_t)gc * 16);
        sb[q] = *(const uint16_t *)(blob + down_scales + ((uint64_t)r * GF + gc) * 2);
    }
    sm::fill_exp_table(s_tab);
    float *xh = s_h[wave], *red = s_red[wave];
#pragma unroll
    for (int q = 0; q < NQ; q++) {
        const int k = wave + DN_WAVES * q;
#pragma unroll
        for (int i = 0; i < 5; i++) {
            const int idx = 10 * lane + 2 * i;  // even, so both values share a group
            if (idx < ff) *(float2 *)&xh[(idx >> 6) * DN_PITCH + (idx & 63)] = hq[q][i];
        }
        __builtin_amdgcn_wave_barrier();
        float h[64];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4 v = *(const float4 *)&xh[gc * DN_PITCH + 4 * i];
            h[4 * i] = v.x;
            h[4 * i + 1] = v.y;
            h[4 * i + 2] = v.z;
            h[4 * i + 3] = v.w;
        }
        float v = ok[q] ? 0.0f : __builtin_nanf("");
        if (ok[q] && live) v = sm::half_bits(sb[q]) * (dot64_4(c[q], h) - sum64(h));
        red[lane] = v;
        __builtin_amdgcn_wave_barrier();
        if (gl == 0 && rr < D10_ROWS && k < nexp) {
            float t = red[lane];
            for (int j = 1; j < GF; j++) t = t + red[lane + j];
            parts[k * D10_ROWS + rr] = t;
        }
        __builtin_amdgcn_wave_barrier();
    }
    const float sig = combine_stage(cin, s_w, topk, s_tab);
    __syncthreads();
    down_combine<D10_ROWS>(parts, s_w, sig, cin, Y, width, topk, resid != nullptr);
}

// K3 for any other shape: hidden groups read from memory, lanes loop over
// groups gl, gl+8, ... of row r.
__global__ void __launch_bounds__(256) k_decode_down_wide(const float *__restrict__ hidden,
                                                          const uint8_t *__restrict__ arena, uint64_t stride,
                                                          const uint8_t *__restrict__ shared_blob,
                                                          const int *__restrict__ ids, const float *__restrict__ weights,
                                                          const float *__restrict__ gate, float *__restrict__ Y,
                                                          int width, int ff, int topk, int experts, uint64_t down_codes,
                                                          uint64_t down_scales, const float *__restrict__ resid) {
    {  // token blockIdx.y
        const int t = blockIdx.y;
        hidden += (uint64_t)t * (topk + 1) * ff;
        ids += (int64_t)t * topk;
        weights += (int64_t)t * topk;
        gate += t;
        Y += (int64_t)t * width;
        if (resid) resid += (int64_t)t * width;
    }
    __shared__ float parts[33 * 8];
    __shared__ float s_w[32];
    __shared__ uint64_t s_tab[32];
    const int nexp = topk + 1, GF = ff / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const CombineIn cin = combine_load(weights, gate, resid, width, topk);
    sm::fill_exp_table(s_tab);
    const int r = min((int)blockIdx.x * 8 + (lane >> 3), width - 1), gl = lane & 7;
    const uint64_t row_bytes = (uint64_t)ff / 4;
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
    const float sig = combine_stage(cin, s_w, topk, s_tab);
    __syncthreads();
    down_combine(parts, s_w, sig, cin, Y, width, topk, resid != nullptr);
}

// ------------------------------------------------- fused single-token layer
// The whole layer for one token in one launch of kFusedBlocks blocks of 8
// waves (one block per CU), for hidden 2048 / ff 512. Two hand-offs between
// blocks go through memory:
//   A. router logits: waves 0 and 1 of every block compute two router rows
//      (reference order) while waves 2-7 build the block's fixed-point
//      activation records in LDS. Each logit is published as one 64-bit word
//      holding the launch number beside the value, so a block's wave 0
//      polls the 512 words themselves until every one is current (no flag
//      or go word for this hand-off), and the block runs the exact top-k
//      itself (no hand-off for the IDs).
//   B. hidden rows: every wave computes kFusedRows of the 11 x 512 hidden
//      rows (10 routed experts and the shared one), then loads the down
//      codes of its block's 8 output rows for its slots. Every block waits
//      for all hidden rows, forms its 8 output rows and combines them
//      (kernels/strata.cu:360-365).
// Cross-block data is written and read with agent-scope coherent accesses
// (global/buffer accesses with the sc1 policy, which bypass the non-coherent
// per-XCD L2 lines). Hand-off B: once its stores are complete, a block
// writes the launch number into its own flag word; one collector wave reads
// all 256 flags (16 bytes per lane) until every block is in and then
// publishes the launch number in the go word, which the other blocks poll.
// Plain stores and loads only: atomics on one address serialize (~14 ns
// each on MI355X). The launch number is the go word's value when the block
// starts plus one (the previous launch left it there), so nothing needs
// resetting. Every wait gives up after kFusedSpinLimit polls (a launch
// argument, so a test can lower it), setting a sticky fault word and its
// host-visible mirror; the layer's outputs are then NaN, and so are those
// of every later launch until sm_fused_reset. The kernel needs all
// kFusedBlocks blocks resident at once: sm_init enables it only when the
// device's CU count times its occupancy (one block per CU) covers them.
constexpr int kFusedBlocks = 256, kFusedWaves = 8;
constexpr int kFusedRows = 3;  // hidden rows per wave: ceil(11 x 512 / 2048)
constexpr int kFusedMaxTopk = 10;
constexpr int kFusedCollector = kFusedBlocks - 1;  // block whose wave 7 collects the flags
constexpr uint32_t kFusedSpinLimit = 1u << 20;
// Word offsets in the synchronisation area (ctx->counters + kFusedSyncBase):
// the flags of hand-off B (one word per block) and the fault word on a line
// of its own, then kFusedGoCopies copies of the go word, one per 128-byte
// line, and kFusedLogitCopies copies of the tagged logits (two words per
// expert, 4 KiB per copy). Block b polls go copy b % kFusedGoCopies and
// logit copy b % kFusedLogitCopies: polls of 256 blocks on one line queue at
// its memory channel, copies spread them. The tagged logits live in this
// area so that only this kernel ever writes them: a stale tag is an earlier
// launch's number, never the current one.
constexpr int kFusedGoCopies = 8, kFusedLogitCopies = 8;
constexpr int kFusedFlagsB = 0, kFusedFaultWord = kFusedBlocks + 32;
constexpr int kFusedGoB = 512, kFusedLogitWords = kFusedGoB + kFusedGoCopies * 32;
constexpr int kFusedSyncWords = kFusedLogitWords + kFusedLogitCopies * 1024;
static_assert(kFusedGoCopies <= kFusedBlocks && kFusedLogitCopies <= 64, "copies");
__device__ __forceinline__ uint32_t *fused_go(uint32_t *sync, int copy) { return sync + kFusedGoB + copy * 32; }
// tagged logit of expert e in copy c (logits = sync + kFusedLogitWords as
// 8-byte words)
__device__ __forceinline__ uint64_t *fused_logit(uint64_t *logits, int c, int e) { return logits + c * 512 + e; }

struct FusedArgs {
    const float *X, *Wr, *bias, *Wsg, *gamma;
    const uint8_t *arena, *shared;
    uint64_t stride, gu_scales, down_codes, down_scales;
    float *Y, *weights, *gate, *hidden;
    uint64_t *logits;  // (launch number << 32) | logit bits, per expert
    int *ids;
    uint32_t *sync;
    float eps;
    int experts, topk;
    // Polls before a wait gives up (kFusedSpinLimit unless a test lowers it)
    // and, for tests of the give-up path only, a non-zero `withhold`: the
    // collector then waits for a flag value no block writes.
    uint32_t spin_limit, withhold;
    // Host-visible mirror of the fault word (pinned host memory): written
    // only when a wait gives up, read by the host after a synchronisation.
    uint32_t *fault_host;
    // The next layer's router matrix (rows of width next_width), or null:
    // block b pulls its rows b and b + 256 into its XCD's L2 while it waits
    // for the other blocks, where the next launch's block b (same XCD) reads
    // them.
    const float *next_wr;
    int next_rows, next_width;
};

__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t load_coherent_u32(uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until this wave's earlier stores are complete (at the coherence point
// for the coherent ones) and keeps the compiler from moving memory accesses
// across; what the wave does next is ordered after them.
__device__ __forceinline__ void stores_complete() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
}
__device__ __forceinline__ void loads_ordered() {
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}
// Marks a give-up: the device fault word (read by later launches, which
// then write NaN) and its host-visible mirror (read by sm_sync / sm_read).
__device__ __forceinline__ void set_fault(uint32_t *fault, uint32_t *fault_host) {
    if ((threadIdx.x & 63) == 0) {
        __hip_atomic_fetch_or(fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(fault_host, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}
// 16 coherent bytes at byte offset `off` of a buffer (buffer load with the sc1
// policy: served from the coherence point, not a stale L2 line).
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const f32x4 v = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16));
    return make_float4(v.x, v.y, v.z, v.w);
}
// Whole-wave wait for the go word to reach `launch`. Returns false (and sets
// the sticky fault word) after `limit` polls.
__device__ bool wait_go(uint32_t *go, uint32_t launch, uint32_t limit, uint32_t *fault, uint32_t *fault_host) {
    const uint32_t want = (uint32_t)__builtin_amdgcn_readfirstlane((int)launch);
    for (uint32_t i = 0; i < limit; i++) {
        const uint32_t v = (uint32_t)__builtin_amdgcn_readfirstlane((int)load_coherent_u32(go));
        if ((int)(v - want) >= 0) {
            loads_ordered();
            return true;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    set_fault(fault, fault_host);
    return false;
}
// The collector: one wave reads the 256 flags of a phase (4 per lane) until
// all hold `launch` (launch + withhold: a test's flag value that never comes),
// then publishes `launch` in every copy of the go word. A collector that
// gives up sets the fault word first and publishes the go word all the same:
// the waiting blocks then see the fault at once (they read it after the go
// word) instead of each spending its own poll limit, and the next launch
// takes the number after this one, so no tag or flag this launch wrote can
// pass as current there.
__device__ bool collect(uint32_t *flags, uint32_t *sync, uint32_t launch, uint32_t limit, uint32_t withhold,
                        uint32_t *fault, uint32_t *fault_host) {
    const uint32_t want = (uint32_t)__builtin_amdgcn_readfirstlane((int)(launch + withhold));
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(flags, (short)0, kFusedBlocks * 4, 0x00020000);
    const uint32_t off = (uint32_t)(threadIdx.x & 63) * 16;
    const uint32_t go = (uint32_t)__builtin_amdgcn_readfirstlane((int)launch);
    bool all = false;
    for (uint32_t i = 0; i < limit; i++) {
        const uint4 f = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16));
        const bool in = (int)(f.x - want) >= 0 && (int)(f.y - want) >= 0 && (int)(f.z - want) >= 0 &&
                        (int)(f.w - want) >= 0;
        if (__ballot(!in) == 0) {
            loads_ordered();
            all = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
        // the flags change under this wave: no poll may reuse an earlier one's value
        __asm__ volatile("" ::: "memory");
    }
    if (!all) {
        set_fault(fault, fault_host);
        stores_complete();  // the fault word before the go word
    }
    for (int c = threadIdx.x & 63; c < kFusedGoCopies; c += 64)
        __hip_atomic_store(fused_go(sync, c), go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return all;
}
// 16 bytes per lane from global memory into LDS (lane l's at base + 16 l).
__device__ __forceinline__ void fused_dma16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
}
// Records in LDS sit kRecPitch words apart: 16 bytes more than a record, so
// the 16-byte reads of lanes reading different groups fall in different
// banks (a 256-byte pitch puts every lane in the same banks).
constexpr int kRecPitch = XQ_WORDS + 4;
// Record of group g from the block's LDS copy (the layout of load_xq).
__device__ __forceinline__ void load_xq_lds(const uint32_t *rec, int g, XQ &q) {
    const uint4 *p = (const uint4 *)(rec + g * kRecPitch);
#pragma unroll
    for (int i = 0; i < 12; i++) {
        const uint4 v = p[i];
        q.limb[4 * i] = v.x;
        q.limb[4 * i + 1] = v.y;
        q.limb[4 * i + 2] = v.z;
        q.limb[4 * i + 3] = v.w;
    }
    q.unit = __builtin_bit_cast(float, rec[g * kRecPitch + 48]);
    q.sum = (int)rec[g * kRecPitch + 49];
}

// Whole-wave wait for a block-local LDS flag set by another wave of the
// block (a relaxed store after a release fence): once the flag reads
// non-zero, the LDS writes made before it are visible.
__device__ __forceinline__ void lds_wait(int *flag) {
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The same for a count that `n` waves raise by one each.
__device__ __forceinline__ void lds_wait_count(int *count, int n) {
    while (__builtin_amdgcn_readfirstlane(__hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < n)
        __builtin_amdgcn_s_sleep(1);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Timeline hook, compiled in only with -DSM_FUSED_TRACE (profiling builds):
// lane 0 of the calling wave records the real-time clock (100 MHz) at mark k
// of its block in LDS (no memory store that a later wait would cover); the
// block's marks go to g_fused_trace when it ends.
#ifdef SM_FUSED_TRACE
__device__ uint64_t g_fused_trace[kFusedBlocks * 32];
#define FUSED_MARK(k) \
    do { if ((threadIdx.x & 63) == 0) s_marks[k] = __builtin_amdgcn_s_memrealtime(); } while (0)
// the same once the wave's outstanding loads are in (profiling builds only)
#define FUSED_MARK_LOADED(k) \
    do { __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8)); FUSED_MARK(k); } while (0)
#else
#define FUSED_MARK(k) \
    do { } while (0)
#define FUSED_MARK_LOADED(k) \
    do { } while (0)
#endif

// W x F: hidden 2048 / ff 512 (the benchmark geometry) or hidden 2560 / ff
// 640 (the real model's, RG below). RG differs in three places: 40 groups
// per gate/up row (groups 32-39 spread one (row, group) pair per lane, as
// in k_decode_gate_up<true>), 7,040 hidden rows (waves 0-3 of a block take
// four, waves 4-7 three: at most seven per SIMD), and 10 output rows per
// block whose 1,100 (slot, row, group) down products are spread over the
// block's threads with every slot's hidden vector in LDS, summed per row in
// group order as k_decode_down10 does, so both geometries give the bits of
// their three-kernel paths.
template <bool NORM, int W, int F>
__global__ void __launch_bounds__(64 * kFusedWaves, 1) k_decode_fused(FusedArgs a) {
    static_assert((W == 2048 && F == 512) || (W == 2560 && F == 640), "fused geometries");
    constexpr bool RG = W == 2560;
    constexpr int G = W / 64, GD = F / 64, ROW_BYTES = W / 4;
    constexpr int DR = W / kFusedBlocks;  // output rows per block: 8, or 10 for RG
    constexpr int RB = RG ? 4 : kFusedRows;  // hidden rows per wave at most
    constexpr int RG_ITEMS = 4 * 4 + 3 * 4;  // RG hidden rows per block
    constexpr int RG_PAIRS = (kFusedMaxTopk + 1) * DR * GD;  // RG down products per block
    __shared__ __attribute__((aligned(16))) uint32_t s_rec[G * kRecPitch];
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    __shared__ int s_ids[32];
    __shared__ float s_w[32];
    __shared__ float s_parts[(kFusedMaxTopk + 2) * DR];
    __shared__ __attribute__((aligned(16))) float s_h[RG ? 1 : kFusedWaves][2][8 * DN_PITCH];
    // RG: every slot's hidden vector (group g of slot k at (k GD + g) DN_PITCH)
    // and the down products v[slot][row][group]
    __shared__ __attribute__((aligned(16))) float s_hid[RG ? (kFusedMaxTopk + 1) * GD * DN_PITCH : 1];
    __shared__ float s_red[RG ? RG_PAIRS : 1];
    __shared__ uint32_t s_arrive;
    __shared__ float s_sig;
    __shared__ int s_ok, s_spec, s_reload, s_staged, s_selected, s_recs;
    __shared__ float s_logit[512];
    __shared__ __attribute__((aligned(16))) uint4 s_pf[2][64];  // prefetch DMA target, never read
#ifdef SM_FUSED_TRACE
    __shared__ uint64_t s_marks[32];
#endif
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x, gw = b * kFusedWaves + wave;
    const int half = lane >> 5, gl = lane & 31;
    const int topk = a.topk, experts = a.experts, nslot = topk + 1;
    uint32_t *fault = a.sync + kFusedFaultWord;
    // This launch's number: the go word as the previous launch left it, plus
    // one (consumed only by the tags, flags and waits).
    const uint32_t launch = load_coherent_u32(fused_go(a.sync, b % kFusedGoCopies)) + 1u;
    // LDS holds garbage at launch: the arrival counter is cleared before any
    // wave can use it.
    if (tid == 0) {
        s_arrive = 0;
        s_staged = 0;
        s_selected = 0;
        s_recs = 0;
    }
    __syncthreads();
    bool ok = true;
    if (wave == 0) FUSED_MARK(0);

    // ---- phase A. Waves 0-1: router row `row` (reference order). Waves 2-7:
    // the block's activation records (group g by wave 2 + g % 6). Block 0's
    // wave 2 also the shared gate logit. x is loaded first: vector loads
    // return in order.
    float xv[G];
#pragma unroll
    for (int j = 0; j < G; j++) xv[j] = a.X[lane + 64 * j];
    float xres = 0.0f;  // the block entry's residual for combine thread tid < 8
    if (NORM) xres = a.X[RG ? min(b * DR + min(tid, DR - 1), W - 1) : min(b * 8 + (tid & 7), W - 1)];
    const bool router = wave < 2;
    const int row = b + kFusedBlocks * wave;
    const bool gate_wave = b == 0 && wave == 2;
    // One weight-row load site for the router row and the shared gate vector
    // (the registers then have a single writer on every path).
    const float *wsrc = router ? a.Wr + (int64_t)min(row, experts - 1) * W : gate_wave ? a.Wsg : nullptr;
    float wv[G];
    if (wsrc) {
#pragma unroll
        for (int j = 0; j < G; j++) wv[j] = __builtin_nontemporal_load(wsrc + lane + 64 * j);
    }
    const float rbias = router && a.bias ? a.bias[min(row, experts - 1)] : 0.0f;
    if (NORM) {
        float gv[G];
#pragma unroll
        for (int j = 0; j < G; j++) gv[j] = a.gamma[lane + 64 * j];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < G; j++) ss = ss + xv[j] * xv[j];
        ss = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sm::tree_sum64(ss)), 0));
        const float inv = 1.0f / sqrtf(ss / (float)W + a.eps);
#pragma unroll
        for (int j = 0; j < G; j++) xv[j] = (xv[j] * inv) * gv[j];
    }
    sm::fill_exp_table(s_tab);

    if (router) {
        // logit = the reference's lane-strided sequential sum, then its tree
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < G; j++) sum = sum + wv[j] * xv[j];
        sum = sm::tree_sum64(sum);
        if (lane == 0 && row < experts) {
            const float logit = a.bias ? sum + rbias : sum;
            const uint64_t tagged = ((uint64_t)launch << 32) | __builtin_bit_cast(uint32_t, logit);
#pragma unroll
            for (int c = 0; c < kFusedLogitCopies; c++)
                __hip_atomic_store(fused_logit(a.logits, c, row), tagged, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (wave == 0) FUSED_MARK(2);
    } else {
        // records of groups g = wave - 2, wave + 4, ... (lane l of group g is xv[g])
#pragma unroll
        for (int q = 0; q < (G + 5) / 6; q++) {
            const int g = wave - 2 + 6 * q;
            if (g >= G) break;
            float v = xv[0];
#pragma unroll
            for (int j = 1; j < G; j++) v = g == j ? xv[j] : v;
            float unit;
            int sum;
            quantize_group_bytes(v, (uint8_t *)(s_rec + g * kRecPitch), unit, sum);
            if (lane == 0) {
                s_rec[g * kRecPitch + 48] = __builtin_bit_cast(uint32_t, unit);
                s_rec[g * kRecPitch + 49] = (uint32_t)sum;
            }
        }
        // this wave's records are written: counted for the waves that load
        // them before the block's next barrier
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __hip_atomic_fetch_add(&s_recs, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (wave == 2) FUSED_MARK(1);
        if (gate_wave) {
            float gs = 0.0f;
#pragma unroll
            for (int j = 0; j < G; j++) gs = gs + wv[j] * xv[j];
            gs = sm::tree_sum64(gs);
            if (lane == 0) store_coherent(a.gate, gs);
        }
    }

    // ---- hand-off A: wave 0 polls the tagged logits until all are this
    // launch's, stages them in LDS and picks the top-k by logit (the
    // reference's selection in all but near-tie cases); every wave issues its
    // phase-B code loads for those experts at once, forms one exponential,
    // and wave 0 then confirms the selection from the probabilities (or
    // replaces it, and the loads are issued again).
    if (wave == 0) {
        // One round reads all 512 tagged words of this block's copy. While
        // the next round is in flight, the selection threshold is searched
        // over the logits already in (valid for the complete set), which
        // takes the search off the path after the last round.
        auto poll = [&](uint64_t (&d)[8]) {
#pragma unroll
            for (int j = 0; j < 8; j++)
                d[j] = __hip_atomic_load(fused_logit(a.logits, b % kFusedLogitCopies, min(lane + 64 * j, experts - 1)),
                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        };
        uint64_t t[8];
        // The first round waits 256 clocks after the block's own router rows:
        // issued at once it nearly always came back incomplete (the other
        // blocks' rows were still on their way) and cost a whole extra round
        // (A/B on one GPU, medians of 50 graph replays: 13.02 -> 12.74 us per
        // step; 512 clocks no better, 1,024 slower).
        __builtin_amdgcn_s_sleep(4);
        poll(t);
        bool all = false;
        uint32_t T0 = 0;
        for (uint32_t i = 0; i < a.spin_limit; i++) {
            bool mine = true;
#pragma unroll
            for (int j = 0; j < 8; j++) mine = mine && (uint32_t)(t[j] >> 32) == launch;
            if (__ballot(!mine) == 0) {
                all = true;
                break;
            }
            uint64_t tn[8];
            poll(tn);
            uint32_t hk = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const bool cur = (uint32_t)(t[j] >> 32) == launch && lane + 64 * j < experts;
                hk = max(hk, cur ? sm::logit_key(__builtin_bit_cast(float, (uint32_t)t[j])) : 0u);
            }
            T0 = max(T0, sm::logit_threshold(hk, topk));
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < 8; j++) t[j] = tn[j];
        }
        if (!all) set_fault(fault, a.fault_host);
        ok = all;
        float lg[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            lg[j] = lane + 64 * j < experts ? __builtin_bit_cast(float, (uint32_t)t[j]) : -3.402823e38f;
            s_logit[lane + 64 * j] = lg[j];
        }
        if (lane == 0) {
            s_ok = ok;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __hip_atomic_store(&s_staged, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        FUSED_MARK(3);
        const bool spec = sm::select_by_logit(lg, experts, topk, T0, s_router, s_ids);
        // without a candidate the first loads read experts 0..topk-1 (in
        // bounds; replaced once the selection is made)
        if (!spec && lane < topk) s_ids[lane] = lane;
        if (lane == 0) {
            s_spec = spec;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __hip_atomic_store(&s_selected, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    // Wave 1 forms the probabilities meanwhile (the logits staged by wave 0).
    float prob[8];
    if (wave == 1) {
        lds_wait(&s_staged);
        float lg[8];
#pragma unroll
        for (int j = 0; j < 8; j++) lg[j] = s_logit[lane + 64 * j];
        sm::router_probs_wave(lg, experts, s_tab, s_router, prob);
    }
    // Every wave waits for the candidate IDs (LDS flag, no barrier: wave 1
    // may still be forming probabilities) and issues its phase-B code loads.
    // Nothing earlier is outstanding by now (the wait tells the compiler so,
    // which keeps it from waiting for everything before the first code load).
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0)
    if (wave != 0) lds_wait(&s_selected);
    if (wave == 0) FUSED_MARK(12);
    ok = s_ok;

    // ---- phase B: the wave's hidden rows items base .. base + nrow - 1 of
    // the 11 x F (item = slot x F + row; the shared expert is slot topk):
    // three per wave, or for RG four (waves 0-3) or three (waves 4-7), 28
    // per block. Code loads from s_ids; a row past nrow reloads the last one.
    const int rr = lane >> 3, g8 = lane & 7;
    const int drow = b * 8 + rr;
    const int nitems = nslot * F;
    const int nrow = RG ? (wave < 4 ? 4 : 3) : kFusedRows;
    const int base = RG ? b * RG_ITEMS + (wave < 4 ? 4 * wave : 16 + 3 * (wave - 4)) : gw * kFusedRows;
    // RG: the lane's (row, group) pair of groups 32-39: group g2 of the
    // wave's row r2 whose item is gl / 8 modulo 4. k_decode_gate_up<true>
    // gives item i's pairs to lanes 8 (i % 4) .. + 7 (its waves start at
    // multiples of 4), and the lane a product lands on fixes the rounding of
    // the half-wave sum; a wave's rows are at most 4 consecutive items, so
    // each residue is at most one row (r2 >= nrow: no row, the lane idles).
    const int r2 = ((gl >> 3) - base) & 3, g2 = 32 + (gl & 7);
    uint4 c[RB], ce;
    uint32_t sb[RB], sbe;
    bool rok[RB];
    auto issue_codes = [&]() {
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const int item = min(base + (RG ? min(r, nrow - 1) : r), nitems - 1);
            const int k = item / F, j = item - k * F;
            const uint8_t *blob = slot_blob(a.arena, a.stride, a.shared, k < topk ? s_ids[k] : 0, k, topk, experts);
            rok[r] = blob != nullptr;
            blob = blob ? blob : a.shared;
            const uint64_t wrow = 2 * (uint64_t)j + half;
            c[r] = load_codes(blob + wrow * ROW_BYTES + gl * 16);
            sb[r] = *(const uint16_t *)(blob + a.gu_scales + (wrow * G + gl) * 2);
        }
        if constexpr (RG) {
            const int item = min(base + min(r2, nrow - 1), nitems - 1);
            const int k = item / F, j = item - k * F;
            const uint8_t *blob = slot_blob(a.arena, a.stride, a.shared, k < topk ? s_ids[k] : 0, k, topk, experts);
            blob = blob ? blob : a.shared;  // (its row's rok covers it)
            const uint64_t wrow = 2 * (uint64_t)j + half;
            ce = load_codes(blob + wrow * ROW_BYTES + g2 * 16);
            sbe = *(const uint16_t *)(blob + a.gu_scales + (wrow * G + g2) * 2);
        }
    };
    issue_codes();
    // The activation records of the lane's group (RG: and of its pair's
    // group) into registers while the codes are in flight (once the six
    // record waves have written them).
    lds_wait_count(&s_recs, kFusedWaves - 2);
    XQ xq, xq2;
    load_xq_lds(s_rec, gl, xq);
    if constexpr (RG) load_xq_lds(s_rec, g2, xq2);
    // Wave 1 confirms the candidate from the probabilities (or replaces it:
    // the loads are then issued again) and forms the weights; the barrier
    // orders LDS only, so every wave's code loads stay in flight.
    if (wave == 1) {
        const bool stood = sm::router_confirm(prob, experts, topk, s_spec, s_router, s_ids);
        FUSED_MARK(4);
        if (lane == 0) s_reload = !stood;
    }
    sm::lds_barrier();
    if (wave == 0) FUSED_MARK(5);
    if (s_reload) issue_codes();
    {
        FUSED_MARK_LOADED(16 + wave);
        float acc[RB];
        if constexpr (RG) {
            // k_decode_gate_up<true>'s sums: group gl by fma onto 0, then the
            // pair's product added to its row (and +0 to the others)
#pragma unroll
            for (int r = 0; r < RB; r++) acc[r] = fmaf(sm::half_bits(sb[r]), dot64_q(c[r], xq), 0.0f);
            const float v = sm::half_bits(sbe) * dot64_q(ce, xq2);
#pragma unroll
            for (int r = 0; r < RB; r++) acc[r] += r == r2 ? v : 0.0f;
        } else {
#pragma unroll
            for (int r = 0; r < RB; r++) acc[r] = sm::half_bits(sb[r]) * dot64_q(c[r], xq);
        }
        // row r's gate and up sums (lanes 31 and 63) go to lane r: one SiLU
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const float v = sm::half32_sum(acc[r]);
            const float gr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31));
            const float ur = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
            g = lane == r ? gr : g;
            u = lane == r ? ur : u;
        }
        bool mine_ok = true;
#pragma unroll
        for (int r = 0; r < RB; r++) mine_ok = lane == r ? rok[r] : mine_ok;
        const float h = mine_ok ? sm::silu(g, s_tab) * u : __builtin_nanf("");
        const int item = base + lane;
        if (lane < nrow && item < nitems) store_coherent(a.hidden + item, h);
    }
    stores_complete();
    FUSED_MARK(24 + wave);
    // the block's flag once all eight waves are done
    if (lane == 0 && atomicAdd(&s_arrive, 1u) == kFusedWaves - 1)
        __hip_atomic_store(a.sync + kFusedFlagsB + b, launch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Waves 2 and 3: the next layer's router rows b and b + 256 (the rows
    // the next launch's block b, on this block's XCD, reads first) into L2,
    // by DMA into a scratch kilobyte of LDS that nothing reads. Issued here,
    // after the block's flag: earlier they slow this layer's loads, later the
    // hidden-row loads after the go word would wait for them (loads complete
    // in order); the down-code loads issued next are needed only ~2 us later.
    // (A/B on one GPU, 48-layer graphs: 13.0 -> 12.5 us per step; issued
    // after the records, 12.9; after the down-code loads, 12.6-12.7; with the
    // hidden loads, 13.2.)
    if ((wave == 2 || wave == 3) && a.next_wr) {
        const int nrow = b + kFusedBlocks * (wave - 2);
        if (nrow < a.next_rows) {
            const float *src = a.next_wr + (int64_t)nrow * a.next_width;
            for (int off = lane * 4; off < a.next_width; off += 256) fused_dma16(src + off, &s_pf[wave - 2][0]);
        }
    }
    // The down codes of this block's 8 output rows for the wave's slots
    // (wave and wave + 8): in flight while the hidden rows come in.
    // RG: thread tid < 440 takes (slot, group) pair tid / 4 (slot
    // pair / 10, group pair % 10) and rows rg_row0 .. + rg_rows - 1 of the
    // block's 10 (3, 3, 2, 2 rows for tid % 4 = 0..3), so that it reads
    // the group's hidden values and forms their sum once; the down codes of
    // those rows (a row past the last reloads it).
    constexpr int DQ = RG ? 3 : 2;
    const int rg_pair = min(tid >> 2, (kFusedMaxTopk + 1) * GD - 1), rg_sub = tid & 3;
    const int rg_row0 = rg_sub < 2 ? 3 * rg_sub : 6 + 2 * (rg_sub - 2), rg_rows = rg_sub < 2 ? 3 : 2;
    uint4 dc[DQ];
    uint32_t dsb[DQ];
    bool dok[DQ];
#pragma unroll
    for (int q = 0; q < DQ; q++) {
        int s, row, grp;
        if constexpr (RG) {
            s = min(rg_pair / GD, nslot - 1);
            row = b * DR + rg_row0 + min(q, rg_rows - 1);
            grp = rg_pair % GD;
        } else {
            s = min(wave + kFusedWaves * q, nslot - 1);
            row = drow;
            grp = g8;
        }
        const uint8_t *blob = slot_blob(a.arena, a.stride, a.shared, s < topk ? s_ids[s] : 0, s, topk, experts);
        dok[q] = blob != nullptr;
        blob = blob ? blob : a.shared;
        dc[q] = load_codes(blob + a.down_codes + (uint64_t)row * (F / 4) + grp * 16);
        dsb[q] = *(const uint16_t *)(blob + a.down_scales + ((uint64_t)row * GD + grp) * 2);
    }
    // The collector runs whatever its own block's state: every block writes
    // its flag (a block that gave up included), and only the collector
    // advances the go word.
    if (b == kFusedCollector && wave == kFusedWaves - 1) {
        collect(a.sync + kFusedFlagsB, a.sync, launch, a.spin_limit, a.withhold, fault, a.fault_host);
        FUSED_MARK(13);
    }

    // ---- phase B wait; then the block's 8 output rows. Wave 1 forms the
    // routing weights meanwhile (only the combine uses them):
    // weights = selected / max(sum of selected, 2^-14), sum in k order.
    if (wave == 0) {
        if (ok) ok = wait_go(fused_go(a.sync, b % kFusedGoCopies), launch, a.spin_limit, fault, a.fault_host);
        FUSED_MARK(8);
    } else if (wave == 1) {
        float denom = 0.0f;
        for (int k = 0; k < topk; ++k) denom = denom + s_router.val[k];
        denom = fmaxf(denom, 0.00006103515625f);
        if (lane < topk) {
            const float wk = s_router.val[lane] / denom;
            s_w[lane] = wk;
            if (b == 0) {
                a.ids[lane] = s_ids[lane];
                a.weights[lane] = wk;
            }
        }
    }
    __syncthreads();
    const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
        a.hidden, (short)0, (int)((uint32_t)nslot * F * 4), 0x00020000);
    if constexpr (RG) {
        // Every slot's hidden vector into LDS (16-byte coherent loads, all
        // issued before any is stored), group g of slot k at (k GD + g) x
        // DN_PITCH; then the thread's down products, each over its group
        // from LDS (lanes of one group read the same addresses); then per
        // (slot, row) the groups' products in group order; then the combine.
        constexpr int N4MAX = (kFusedMaxTopk + 1) * F / 4, HQ = (N4MAX + 64 * kFusedWaves - 1) / (64 * kFusedWaves);
        const int n4 = nitems / 4;
        float4 hv[HQ];
#pragma unroll
        for (int i = 0; i < HQ; i++) hv[i] = load16_coherent(hr, (uint32_t)min(tid + 64 * kFusedWaves * i, n4 - 1) * 16);
        if (wave == kFusedWaves - 1) {
            const float sig = sm::sigmoid(load_coherent(a.gate), s_tab);
            if (lane == 0) s_sig = sig;
        }
        const bool faulted = load_coherent_u32(fault) != 0u || !ok;
        if (wave == 0) FUSED_MARK_LOADED(11);
#pragma unroll
        for (int i = 0; i < HQ; i++) {
            const int idx = tid + 64 * kFusedWaves * i;
            if (idx < n4) {
                const int e = 4 * idx, k = e / F, o = e - k * F;
                *(float4 *)&s_hid[(k * GD + (o >> 6)) * DN_PITCH + (o & 63)] = hv[i];
            }
        }
        __syncthreads();
        {
            const int k = rg_pair / GD, grp = rg_pair % GD;
            if (tid < 4 * (kFusedMaxTopk + 1) * GD && k < nslot) {
                float h[64];
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float4 v = *(const float4 *)&s_hid[(k * GD + grp) * DN_PITCH + 4 * i];
                    h[4 * i] = v.x;
                    h[4 * i + 1] = v.y;
                    h[4 * i + 2] = v.z;
                    h[4 * i + 3] = v.w;
                }
                const float hs = sum64(h);
#pragma unroll
                for (int q = 0; q < DQ; q++) {
                    if (q < rg_rows) {
                        const float v = dok[q] ? sm::half_bits(dsb[q]) * (dot64_4(dc[q], h) - hs) : __builtin_nanf("");
                        s_red[(k * DR + rg_row0 + q) * GD + grp] = v;
                    }
                }
            }
        }
        __syncthreads();
        if (tid < nslot * DR) {
            const float *v = &s_red[tid * GD];  // slot tid / DR, row tid % DR
            float t = v[0];
#pragma unroll
            for (int j = 1; j < GD; j++) t = t + v[j];
            s_parts[tid] = t;
        }
        __syncthreads();
        if (tid < DR) {
            const int r = b * DR + tid;
            float value = s_parts[topk * DR + tid] * s_sig;
            for (int k = 0; k < topk; k++) value = value + s_parts[k * DR + tid] * s_w[k];
            if (faulted) value = __builtin_nanf("");
            a.Y[r] = NORM ? xres + value : value;
        }
    } else {
        // lane (rr, g8) brings values 8 rr .. 8 rr + 7 of hidden group g8 of each
        // of the wave's slots; all loads issued before any is used (a slot past
        // the last reads the last one again)
        float4 hq[2][2];
    #pragma unroll
        for (int q = 0; q < 2; q++) {
            const int s = min(wave + kFusedWaves * q, nslot - 1);
            const uint32_t off = (uint32_t)(s * F + g8 * 64 + 8 * rr) * 4;
            hq[q][0] = load16_coherent(hr, off);
            hq[q][1] = load16_coherent(hr, off + 16);
        }
        // the shared expert's gate, sigmoid(gate logit), by a wave with one slot
        if (wave == kFusedWaves - 1) {
            const float sig = sm::sigmoid(load_coherent(a.gate), s_tab);
            if (lane == 0) s_sig = sig;
        }
        // Read with the hidden rows rather than after the products: a wait that
        // gave up in any block set the fault word before that block's flag, so
        // before the go word; this block's own give-ups are in wave 0's `ok`
        // (wave 0 forms the outputs).
        const bool faulted = load_coherent_u32(fault) != 0u || !ok;
        if (wave == 0) FUSED_MARK_LOADED(11);
        // The wave's slots are wave and wave + 8 (two for waves 0-2 at top-10);
        // with two, both dots run side by side (independent chains), each slot
        // with its own exchange area. Per slot: the group sum of the hidden
        // values (own eighth, then lanes ^ 8, ^ 16, ^ 32), the exchange (lane
        // (rr, g8) stores values 8 rr .. 8 rr + 7 of group g8, then reads the
        // whole group), the dot in dot64_4's order.
        const bool two = wave + kFusedWaves < nslot;
        float s8[2] = {0.0f, 0.0f};
    #pragma unroll
        for (int q = 0; q < 2; q++) {
            if (q == 1 && !two) break;
            const float4 h0 = hq[q][0], h1 = hq[q][1];
            float t = ((h0.x + h0.y) + (h0.z + h0.w)) + ((h1.x + h1.y) + (h1.z + h1.w));
            t = t + sm::dpp_f32<0x128>(0.0f, t);
            const int u = __builtin_bit_cast(int, t);
            const auto p16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
            t = __builtin_bit_cast(float, (int)p16[0]) + __builtin_bit_cast(float, (int)p16[1]);
            const int w = __builtin_bit_cast(int, t);
            const auto p32 = __builtin_amdgcn_permlane32_swap(w, w, false, false);
            s8[q] = __builtin_bit_cast(float, (int)p32[0]) + __builtin_bit_cast(float, (int)p32[1]);
            float *xh = s_h[wave][q];
            *(float4 *)&xh[g8 * DN_PITCH + 8 * rr] = h0;
            *(float4 *)&xh[g8 * DN_PITCH + 8 * rr + 4] = h1;
        }
        __builtin_amdgcn_wave_barrier();
        // 16 hidden values of group g8 (chunk w4) from exchange area q
        auto chunk = [&](int q, int w4, float (&x)[16]) {
    #pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = *(const float4 *)&s_h[wave][q][g8 * DN_PITCH + 16 * w4 + 4 * i];
                x[4 * i] = v.x;
                x[4 * i + 1] = v.y;
                x[4 * i + 2] = v.z;
                x[4 * i + 3] = v.w;
            }
        };
        auto word = [](const uint4 &c, int w4) { return w4 == 0 ? c.x : w4 == 1 ? c.y : w4 == 2 ? c.z : c.w; };
        float d[2][4];
        if (two) {
    #pragma unroll
            for (int w4 = 0; w4 < 4; w4++) {
                float x0[16], x1[16];
                chunk(0, w4, x0);
                chunk(1, w4, x1);
                d[0][w4] = dot16(word(dc[0], w4), x0, 0.0f);
                d[1][w4] = dot16(word(dc[1], w4), x1, 0.0f);
            }
        } else {
    #pragma unroll
            for (int w4 = 0; w4 < 4; w4++) {
                float x0[16];
                chunk(0, w4, x0);
                d[0][w4] = dot16(word(dc[0], w4), x0, 0.0f);
                d[1][w4] = 0.0f;
            }
        }
    #pragma unroll
        for (int q = 0; q < 2; q++) {
            if (q == 1 && !two) break;
            const float dot = (d[q][0] + d[q][1]) + (d[q][2] + d[q][3]);
            float v = dok[q] ? sm::half_bits(dsb[q]) * (dot - s8[q]) : __builtin_nanf("");
            v = sm::group8_sum(v);
            if (g8 == 0) s_parts[(wave + kFusedWaves * q) * 8 + rr] = v;
        }
        __syncthreads();
        if (tid < 8) {
            const int r = b * 8 + tid;
            float value = s_parts[topk * 8 + tid] * s_sig;
            for (int k = 0; k < topk; k++) value = value + s_parts[k * 8 + tid] * s_w[k];
            if (faulted) value = __builtin_nanf("");
            a.Y[r] = NORM ? xres + value : value;
        }
    }
    if (wave == 0) FUSED_MARK(9);
#ifdef SM_FUSED_TRACE
    __syncthreads();
    if (tid < 32) g_fused_trace[b * 32 + tid] = s_marks[tid];
#endif
}

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct DecodeWs {
    uint64_t logits, gate, xq, hidden, end;
};
DecodeWs decode_ws(int tokens, int width, int ff, int experts, int topk) {
    const uint64_t T = (uint64_t)tokens;
    DecodeWs w;
    w.logits = 0;
    w.gate = up(w.logits + T * experts * 4);
    w.xq = up(w.gate + T * 4);
    w.hidden = up(w.xq + T * (width / 64) * XQ_WORDS * 4);
    w.end = up(w.hidden + T * (topk + 1) * ff * 4);
    return w;
}

}  // namespace

// Device scratch of the allocation-free decode entry (sm_moe_layer_static):
// the decode workspace (logits, activation records, hidden rows) for any
// call whose decode_ws() fits. Each GPU holds its own copy for the life of
// the process; host code never passes this name to a kernel, only the
// address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[smi::kStaticScratchBytes];

namespace smi {

namespace {
// Per device: the scratch address, and the end of the last allocation-free
// call (its stream and an event recorded there), under one lock.
struct StaticScratchState {
    std::mutex lock;
    void *ptr = nullptr;
    hipEvent_t last = nullptr;
    hipStream_t last_stream = nullptr;
    bool pending = false;  // `last` marks the end of a call not yet waited for by its successor
};
StaticScratchState g_static[kMaxDevices];
}  // namespace

int static_scratch_init(sm_ctx *ctx) {
    // One lookup per device; every context on that device shares the array.
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return fail(ctx, SM_E_ARG, "device index out of range");
    StaticScratchState &st = g_static[ctx->device];
    std::lock_guard<std::mutex> g(st.lock);
    if (!st.ptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(ctx, SM_E_HIP, "hipGetSymbolAddress(scratch) returned no address");
        hipEvent_t ev = nullptr;
        const hipError_t e2 = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e2 != hipSuccess) return hip_fail(ctx, e2, "hipEventCreateWithFlags(static scratch)");
        st.last = ev;
        st.ptr = p;
    }
    ctx->scratch = st.ptr;
    return SM_OK;
}

StaticScratchCall::StaticScratchCall(sm_ctx *ctx) : ctx_(ctx), lock_(g_static[ctx->device].lock) {}

int StaticScratchCall::begin() {
    StaticScratchState &st = g_static[ctx_->device];
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(ctx_->stream, &cs);
    if (e != hipSuccess) return hip_fail(ctx_, e, "hipStreamIsCapturing");
    capturing_ = cs != hipStreamCaptureStatusNone;
    // Under capture the call is a graph node: its order is the caller's (an
    // event recorded outside the capture cannot be waited for inside it).
    if (capturing_ || !st.pending || st.last_stream == ctx_->stream) return SM_OK;
    const hipError_t w = hipStreamWaitEvent(ctx_->stream, st.last, 0);
    if (w != hipSuccess) return hip_fail(ctx_, w, "hipStreamWaitEvent(static scratch)");
    return SM_OK;
}

int StaticScratchCall::done() {
    StaticScratchState &st = g_static[ctx_->device];
    // A captured call leaves the record as it is: the next call outside the
    // capture still waits for the last one that ran outside it.
    if (capturing_) return SM_OK;
    const hipError_t e = hipEventRecord(st.last, ctx_->stream);
    if (e != hipSuccess) {
        st.pending = false;
        return hip_fail(ctx_, e, "hipEventRecord(static scratch)");
    }
    st.last_stream = ctx_->stream;
    st.pending = true;
    return SM_OK;
}

uint32_t fused_fault_word() { return kFusedSyncBase + kFusedFaultWord; }
uint32_t fused_sync_words() { return kFusedSyncWords; }

bool fused_fits(int compute_units, int blocks_per_cu) {
    return compute_units > 0 && blocks_per_cu > 0 && (int64_t)compute_units * blocks_per_cu >= kFusedBlocks;
}

int fused_decode_init(sm_ctx *ctx) {
    // Blocks per CU of each instantiation (the one-block-per-CU bound makes
    // this 0 or 1 on a CDNA CU); each geometry is enabled only when both of
    // its instantiations fit.
    using KF = void (*)(FusedArgs);
    const KF kernels[4] = {k_decode_fused<true, 2048, 512>, k_decode_fused<false, 2048, 512>,
                           k_decode_fused<true, 2560, 640>, k_decode_fused<false, 2560, 640>};
    int per_cu[4] = {0, 0, 0, 0};
    for (int i = 0; i < 4; i++) {
        const hipError_t e =
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu[i], kernels[i], 64 * kFusedWaves, 0);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipOccupancyMaxActiveBlocksPerMultiprocessor(k_decode_fused)");
    }
    int cus = 0;
    const hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipDeviceGetAttribute(multiProcessorCount)");
    ctx->fused_capable = fused_fits(cus, per_cu[0] < per_cu[1] ? per_cu[0] : per_cu[1]);
    ctx->fused_capable_rg = fused_fits(cus, per_cu[2] < per_cu[3] ? per_cu[2] : per_cu[3]);
    ctx->fused_spin_limit = kFusedSpinLimit;
    ctx->fused_withhold = 0;
    return SM_OK;
}
static_assert(kFusedSyncBase + kFusedSyncWords <= kCounterWords, "fused decode sync area");
static_assert((kFusedSyncBase + kFusedLogitWords) % 2 == 0, "tagged logits are 8-byte words");

}  // namespace smi

#ifdef SM_FUSED_TRACE
extern "C" int sm_fused_trace_read(uint64_t *out, int n) {
    if (n < kFusedBlocks * 32) return SM_E_ARG;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_fused_trace), sizeof(uint64_t) * kFusedBlocks * 32) == hipSuccess
               ? SM_OK
               : SM_E_HIP;
}
#endif

namespace smi {

uint64_t moe_decode_workspace(int tokens, int width, int ff, int experts, int topk) {
    return decode_ws(tokens, width, ff, experts, topk).end;
}

int moe_decode(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
               uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y, uint64_t ids,
               uint64_t weights, uint64_t workspace, uint64_t workspace_bytes, const BlockArgs *block) {
    const float *gamma = block ? (const float *)block->gamma : nullptr;
    const float eps = block ? block->eps : 0.0f;
    const float *resid = block ? (const float *)X : nullptr;
    (void)workspace_bytes;
    DecodeWs w = decode_ws(tokens, width, ff, experts, topk);
    char *ws = (char *)workspace;
    BlobLayout L = blob_layout(width, ff);
    float *hidden = (float *)(ws + w.hidden);
    const int blocks_per_expert = ceil_div(ff, GU_ROWS * GU_WAVES);
    uint32_t *xq = (uint32_t *)(ws + w.xq);
    // One token at hidden 2048 / ff 512 or 2560 / 640: the whole layer in
    // one launch.
    const uint32_t decode_stages = (1u << kStageDecodeRoute) | (1u << kStageDecodeGateUp) | (1u << kStageDecodeDown);
    const bool geo_2048 = width == 2048 && ff == 512 && ctx->fused_capable;
    const bool geo_2560 = width == 2560 && ff == 640 && ctx->fused_capable_rg;
    if (tokens == 1 && (geo_2048 || geo_2560) && experts <= 2 * kFusedBlocks && topk <= kFusedMaxTopk &&
        stage_on(ctx, kStageDecodeFused) && (ctx->stage_mask & decode_stages) == decode_stages) {
        if (int rc = stage_mark(ctx, kStageDecodeFused)) return rc;
        FusedArgs fa;
        fa.X = (const float *)X;
        fa.Wr = (const float *)Wr;
        fa.bias = (const float *)bias;
        fa.Wsg = (const float *)Wsg;
        fa.gamma = gamma;
        fa.arena = (const uint8_t *)arena;
        fa.shared = (const uint8_t *)shared_blob;
        fa.stride = blob_stride;
        fa.gu_scales = L.gate_up_scales;
        fa.down_codes = L.down_codes;
        fa.down_scales = L.down_scales;
        fa.Y = (float *)Y;
        fa.weights = (float *)weights;
        fa.logits = (uint64_t *)(ctx->counters + kFusedSyncBase + kFusedLogitWords);
        fa.gate = (float *)(ws + w.gate);
        fa.hidden = hidden;
        fa.ids = (int *)ids;
        fa.sync = ctx->counters + kFusedSyncBase;
        fa.eps = eps;
        fa.experts = experts;
        fa.topk = topk;
        fa.spin_limit = ctx->fused_spin_limit;
        fa.withhold = ctx->fused_withhold;
        fa.fault_host = ctx->fault_dev;
        // the next layer's router matrix, when the caller named one
        // (sm_prefetch_router; checked by the entry point)
        fa.next_wr = (const float *)ctx->next_wr;
        fa.next_rows = ctx->next_rows;
        fa.next_width = ctx->next_width;
        const auto kf = geo_2048 ? (gamma ? k_decode_fused<true, 2048, 512> : k_decode_fused<false, 2048, 512>)
                                 : (gamma ? k_decode_fused<true, 2560, 640> : k_decode_fused<false, 2560, 640>);
        kf<<<kFusedBlocks, 64 * kFusedWaves, 0, ctx->stream>>>(fa);
        if (int rc = launched(ctx)) return rc;
        return stage_mark(ctx, -1);
    }
    // 1. router logits + shared gate logit + fixed-point activations
    if (stage_on(ctx, kStageDecodeRoute)) {
        if (int rc = stage_mark(ctx, kStageDecodeRoute)) return rc;
        // grid.x a multiple of 8: block (x, t) runs on XCD x % 8 for every
        // token t, so each XCD reads its share of W_r from memory once.
        const int route_blocks = ceil_div(experts + 1, 4);
        const dim3 grid((unsigned)((route_blocks + ceil_div(width / 64, 4) + 7) / 8 * 8), (unsigned)tokens);
        using K1 = void (*)(const float *, const float *, const float *, const float *, float *, float *, uint32_t *,
                            int, int, int, const float *, float);
        // Register-resident rows for the benchmark width (32 groups) and the
        // real model's (2560: 40 groups); a strided loop otherwise.
        const K1 k1 = width == 2048   ? (gamma ? k_decode_route<32, true> : k_decode_route<32, false>)
                      : width == 2560 ? (gamma ? k_decode_route<40, true> : k_decode_route<40, false>)
                                      : (gamma ? k_decode_route<0, true> : k_decode_route<0, false>);
        k1<<<grid, 256, 0, ctx->stream>>>((const float *)X, (const float *)Wr, (const float *)bias, (const float *)Wsg,
                                          (float *)(ws + w.logits), (float *)(ws + w.gate), xq, width, experts,
                                          route_blocks, gamma, eps);
        if (int rc = launched(ctx)) return rc;
    }
    // 2. top-k + gate/up of the routed and shared experts. Up to
    // kDecodeBlockRouting tokens every routed block selects its token's
    // experts itself (no extra launch); beyond that the per-block selections
    // would cost more than one top-k kernel per token.
    const int routed = tokens > kDecodeBlockRouting ? 1 : 0;
    if (routed && stage_on(ctx, kStageDecodeGateUp))
        if (int rc = topk_launch(ctx, (const float *)(ws + w.logits), (int *)ids, (float *)weights, tokens, experts,
                                 topk))
            return rc;
    if (stage_on(ctx, kStageDecodeGateUp)) {
        if (int rc = stage_mark(ctx, kStageDecodeGateUp)) return rc;
        dim3 g1((unsigned)blocks_per_expert, (unsigned)(topk + 1), (unsigned)tokens);
        const int G = width / 64;
        const auto k2 = G > 32 && G <= 40 ? k_decode_gate_up<true> : k_decode_gate_up<false>;
        k2<<<g1, 64 * GU_WAVES, 0, ctx->stream>>>(
            xq, (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob, (const float *)(ws + w.logits),
            (int *)ids, (float *)weights, hidden, width, ff, topk, experts, L.gate_up_scales, routed);
        if (int rc = launched(ctx)) return rc;
    }
    // 3. down for all experts + combine
    if (stage_on(ctx, kStageDecodeDown)) {
        if (int rc = stage_mark(ctx, kStageDecodeDown)) return rc;
        using K3 = void (*)(const float *, const uint8_t *, uint64_t, const uint8_t *, const int *, const float *,
                            const float *, float *, int, int, int, int, uint64_t, uint64_t, const float *);
        static const K3 by_slots[DN_MAX_SLOTS] = {k_decode_down<1>, k_decode_down<2>, k_decode_down<3>,
                                                  k_decode_down<4>, k_decode_down<5>};
        static const K3 by_slots10[DN_MAX_SLOTS] = {k_decode_down10<1>, k_decode_down10<2>, k_decode_down10<3>,
                                                    k_decode_down10<4>, k_decode_down10<5>};
        const bool narrow = ff <= 512, ten = ff > 512 && ff <= 640;
        const int nq = ceil_div(topk + 1, DN_WAVES) - 1, rows = ten ? D10_ROWS : 8;
        const K3 kernel = narrow ? by_slots[nq] : ten ? by_slots10[nq] : k_decode_down_wide;
        kernel<<<dim3((unsigned)ceil_div(width, rows), (unsigned)tokens), narrow || ten ? 64 * DN_WAVES : 256, 0,
                 ctx->stream>>>(
            hidden, (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob, (const int *)ids,
            (const float *)weights, (const float *)(ws + w.gate), (float *)Y, width, ff, topk, experts, L.down_codes,
            L.down_scales, resid);
        if (int rc = launched(ctx)) return rc;
    }
    return stage_mark(ctx, -1);
}

}  // namespace smi
