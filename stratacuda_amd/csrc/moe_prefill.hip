// One MoE layer for a batch of tokens (prefill):
//
//   route     exact router GEMM + per-token top-k (moe_route.hip)
//   dispatch  expert-contiguous permutation (experts ascending, tokens
//             ascending), plus one segment after the routed rows that holds
//             every token once for the shared expert
//   gate/up   grouped GEMM  H[pos, j] = SiLU(g_j . x_row(pos)) * (u_j . x_row(pos))
//   down      grouped GEMM  P[pos, r] = d_r . H[pos, :]
//   combine   Y[t] = P[shared(t)] * sigmoid(gate_t) + sum_k P[where(t,k)] * w_tk
//             in the reference order (kernels/strata.cu:470-476)
//
// Grouped GEMM on MFMA (v_mfma_f32_32x32x16_f16, f32 accumulation):
//  * Weights: (code - 1) * fp16 scale is exactly representable in fp16, so the
//    B operand holds the exact reference weights. Codes are turned into fp16
//    pairs with one mask ((w >> 2j) & 0x00030003 puts codes j and j+8 of a
//    16-code word into the two halves), an OR with the exponent pattern of
//    1024 (0x6400), a packed subtract of 1025 and a packed multiply by the
//    group scale; all three steps are exact.
//  * Activations: x is split into hi = fp16(x) and lo = fp16(x - hi); two
//    MFMAs (hi and lo) per K step give products accurate to ~2^-22 relative,
//    well inside the 1e-4 / 1e-3 output tolerance, where a single fp16 or bf16
//    pass is not.
//  * K order inside a 64-wide scale group is permuted identically for A and B
//    (the dot product does not depend on it) so that both the code unpacking
//    and the LDS reads of A are plain, conflict-free vector accesses.
//  * Tiles: 32 rows (positions of one expert segment) x 128 weight rows per
//    256-thread block, each wave a 32 x 32 MFMA tile; A (x hi/lo) is staged in
//    LDS per scale group with double buffering, B is dequantised in registers.
//    grid.x = n-block (fastest) so all m-tiles of one (expert, n-block) land
//    on the same XCD and share its L2.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int MT = 32;   // rows (positions) per tile
constexpr int NB = 128;  // weight rows per block (4 waves x 32)

__device__ __forceinline__ half2v codes_to_half2(uint32_t word, int jj, half2v scale) {
    uint32_t t = ((word >> (2 * jj)) & 0x00030003u) | 0x64006400u;  // fp16 (1024 + c, 1024 + c')
    half2v h = __builtin_bit_cast(half2v, t);
    const half2v k1025 = {(_Float16)1025.0f, (_Float16)1025.0f};
    h = h - k1025;  // c - 1, exact
    return h * scale;  // (c - 1) * scale, exact in fp16
}

// B operand (8 fp16 weights) of MFMA step s from the lane's two code words.
__device__ __forceinline__ half8 b_operand(uint32_t w0, uint32_t w1, int s, half2v scale) {
    const uint32_t w = s < 2 ? w0 : w1;
    const int jj0 = 4 * (s & 1);
    half2v p0 = codes_to_half2(w, jj0 + 0, scale), p1 = codes_to_half2(w, jj0 + 1, scale);
    half2v p2 = codes_to_half2(w, jj0 + 2, scale), p3 = codes_to_half2(w, jj0 + 3, scale);
    half8 b = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    return b;
}

// Segment lookup: largest e with tile_base[e] <= tau (segments 0..nseg-1).
__device__ __forceinline__ int find_segment(const int *tile_base, int nseg, int tau) {
    int lo = 0, hi = nseg - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (tile_base[mid] <= tau) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// GATE_UP: A = X rows gathered through rows[], K = width, N = 2*ff, output H
//          [positions x ff] = SiLU(gate) * up of interleaved column pairs.
// else:    A = H rows by position, K = ff, N = width, output P [positions x width].
template <bool GATE_UP>
__global__ void __launch_bounds__(256) k_grouped_gemm(const float *__restrict__ A, const int *__restrict__ rows,
                                                      const int *__restrict__ offsets,
                                                      const int *__restrict__ tile_base,
                                                      const uint8_t *__restrict__ arena, uint64_t stride,
                                                      const uint8_t *__restrict__ shared_blob, int experts,
                                                      uint64_t codes_off, uint64_t scales_off, int K, int N,
                                                      float *__restrict__ out, int out_ld) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][2][4 * 2 * MT * 8];  // [buf][hi/lo][s][h][i][8]
    const int nseg = experts + 1;
    const int tau = blockIdx.y;
    if (tau >= tile_base[nseg]) return;
    const int e = find_segment(tile_base, nseg, tau);
    const int m0 = offsets[e] + (tau - tile_base[e]) * MT, mend = offsets[e + 1];
    const uint8_t *blob = e < experts ? arena + (uint64_t)e * stride : shared_blob;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = K / 64;

    // ---- A staging: thread -> row i = tid / 8, 8 consecutive K values 8c..8c+7
    const int si = tid >> 3, sc = tid & 7;
    const float *arow = nullptr;
    if (m0 + si < mend) arow = GATE_UP ? A + (int64_t)rows[m0 + si] * K : A + (int64_t)(m0 + si) * K;
    // LDS destinations of the 8 values (see the K permutation above).
    const int sh = sc >> 2, ssec = sc & 1, ssw = (sc & 3) >> 1;
    auto stage = [&](int g, int buf) {
        float v[8];
        if (arow) {
            float4 a0 = *(const float4 *)(arow + g * 64 + sc * 8);
            float4 a1 = *(const float4 *)(arow + g * 64 + sc * 8 + 4);
            v[0] = a0.x; v[1] = a0.y; v[2] = a0.z; v[3] = a0.w;
            v[4] = a1.x; v[5] = a1.y; v[6] = a1.z; v[7] = a1.w;
        } else {
#pragma unroll
            for (int q = 0; q < 8; q++) v[q] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int s = 2 * ssw + (q >> 2), slot = 2 * (q & 3) + ssec;
            const int at = ((s * 2 + sh) * MT + si) * 8 + slot;
            _Float16 hi = (_Float16)v[q];
            _Float16 lo = (_Float16)(v[q] - (float)hi);
            lds[buf][0][at] = hi;
            lds[buf][1][at] = lo;
        }
    };

    // ---- B: lane (j = lane % 32, h = lane / 32), weight row n
    const int j = lane & 31, h = lane >> 5;
    const int n = blockIdx.x * NB + wave * 32 + j;
    const uint8_t *brow = blob + codes_off + (uint64_t)n * (K / 4) + h * 8;
    const uint8_t *bscale = blob + scales_off + (uint64_t)n * G * 2;

    float16v acc;
#pragma unroll
    for (int v = 0; v < 16; v++) acc[v] = 0.0f;

    stage(0, 0);
    uint2 cw = *(const uint2 *)(brow);
    uint32_t sb = *(const uint16_t *)(bscale);
    __syncthreads();
    for (int g = 0; g < G; g++) {
        const int buf = g & 1;
        uint2 cw_next = cw;
        uint32_t sb_next = sb;
        if (g + 1 < G) {
            stage(g + 1, buf ^ 1);
            cw_next = *(const uint2 *)(brow + (uint64_t)(g + 1) * 16);
            sb_next = *(const uint16_t *)(bscale + (g + 1) * 2);
        }
        const _Float16 s16 = __builtin_bit_cast(_Float16, (uint16_t)sb);
        const half2v scale = {s16, s16};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half8 b = b_operand(cw.x, cw.y, s, scale);
            const int at = ((s * 2 + h) * MT + j) * 8;
            half8 ahi = *(const half8 *)(&lds[buf][0][at]);
            half8 alo = *(const half8 *)(&lds[buf][1][at]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, b, acc, 0, 0, 0);
        }
        cw = cw_next;
        sb = sb_next;
        __syncthreads();
    }

    // ---- epilogue: acc[v] = D[i][j], i = 8*(v/4) + 4*h + v%4
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int i = 8 * (v >> 2) + 4 * h + (v & 3);
        if (GATE_UP) {
            const float other = __shfl_xor(acc[v], 1, 64);
            if ((j & 1) == 0 && m0 + i < mend)
                out[(int64_t)(m0 + i) * out_ld + (n >> 1)] = sm::silu(acc[v]) * other;
        } else if (m0 + i < mend) {
            out[(int64_t)(m0 + i) * out_ld + n] = acc[v];
        }
    }
}

// Y[t, d] = P[shared(t), d] * sigmoid(gate[t]) + sum_k P[where[t,k], d] * w[t,k]
__global__ void k_combine(const float *__restrict__ P, const int *__restrict__ where_,
                          const float *__restrict__ weights, const float *__restrict__ gate,
                          const int *__restrict__ offsets, float *__restrict__ Y, int tokens, int topk, int width,
                          int experts) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)tokens * width) return;
    const int t = (int)(i / width), d = (int)(i % width);
    const int64_t sb = offsets[experts];
    float value = P[(sb + t) * width + d] * sm::sigmoid(gate[t]);
    for (int k = 0; k < topk; k++) {
        const int pos = where_[(int64_t)t * topk + k];
        const float part = pos >= 0 ? P[(int64_t)pos * width + d] : __builtin_nanf("");
        value = value + part * weights[(int64_t)t * topk + k];
    }
    Y[i] = value;
}

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct PrefillWs {
    uint64_t logits, gate, dispatch, offsets, tile_base, rows, parts, where_, H, P, end;
};
PrefillWs prefill_ws(int tokens, int width, int ff, int experts, int topk) {
    const uint64_t n = (uint64_t)tokens * topk, m = n + tokens;
    PrefillWs w;
    w.logits = 0;
    w.gate = up(w.logits + (uint64_t)tokens * experts * 4);
    w.dispatch = up(w.gate + (uint64_t)tokens * 4);
    w.offsets = up(w.dispatch + dispatch_workspace(tokens, experts));
    w.tile_base = up(w.offsets + ((uint64_t)experts + 2) * 4);
    w.rows = up(w.tile_base + ((uint64_t)experts + 2) * 4);
    w.parts = up(w.rows + m * 4);
    w.where_ = up(w.parts + m * 4);
    w.H = up(w.where_ + n * 4);
    w.P = up(w.H + m * ff * 4);
    w.end = up(w.P + m * width * 4);
    return w;
}

}  // namespace

namespace smi {

uint64_t moe_prefill_workspace(int tokens, int width, int ff, int experts, int topk) {
    return prefill_ws(tokens, width, ff, experts, topk).end;
}

int moe_prefill(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
                uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y, uint64_t ids,
                uint64_t weights, uint64_t workspace, uint64_t workspace_bytes) {
    (void)workspace_bytes;
    PrefillWs w = prefill_ws(tokens, width, ff, experts, topk);
    char *ws = (char *)workspace;
    BlobLayout L = blob_layout(width, ff);
    if ((2 * ff) % NB || width % NB)
        return fail(ctx, SM_E_ARG, "prefill needs width and 2*ff to be multiples of 128");
    if (int rc = stage_mark(ctx, kStagePrefillRoute)) return rc;
    if (int rc = route_launch(ctx, (const float *)X, tokens, width, (const float *)Wr, (const float *)bias, experts,
                              topk, (float *)(ws + w.logits), (int *)ids, (float *)weights, (const float *)Wsg,
                              (float *)(ws + w.gate)))
        return rc;
    int *offsets = (int *)(ws + w.offsets), *tile_base = (int *)(ws + w.tile_base);
    if (int rc = stage_mark(ctx, kStagePrefillDispatch)) return rc;
    if (int rc = dispatch_launch(ctx, (const int *)ids, tokens, topk, experts, offsets, (int *)(ws + w.rows),
                                 (int *)(ws + w.parts), (int *)(ws + w.where_), ws + w.dispatch, 1, tile_base))
        return rc;
    const uint64_t m = (uint64_t)tokens * topk + tokens;
    const unsigned max_tiles = (unsigned)(m / MT + (uint64_t)experts + 2);
    dim3 g1((unsigned)(2 * ff / NB), max_tiles);
    if (int rc = stage_mark(ctx, kStagePrefillGateUp)) return rc;
    k_grouped_gemm<true><<<g1, 256, 0, ctx->stream>>>((const float *)X, (const int *)(ws + w.rows), offsets, tile_base,
                                                      (const uint8_t *)arena, blob_stride, (const uint8_t *)shared_blob,
                                                      experts, L.gate_up_codes, L.gate_up_scales, width, 2 * ff,
                                                      (float *)(ws + w.H), ff);
    if (int rc = launched(ctx)) return rc;
    dim3 g2((unsigned)(width / NB), max_tiles);
    if (int rc = stage_mark(ctx, kStagePrefillDown)) return rc;
    k_grouped_gemm<false><<<g2, 256, 0, ctx->stream>>>((const float *)(ws + w.H), nullptr, offsets, tile_base,
                                                       (const uint8_t *)arena, blob_stride,
                                                       (const uint8_t *)shared_blob, experts, L.down_codes,
                                                       L.down_scales, ff, width, (float *)(ws + w.P), width);
    if (int rc = launched(ctx)) return rc;
    const uint64_t total = (uint64_t)tokens * width;
    if (int rc = stage_mark(ctx, kStagePrefillCombine)) return rc;
    k_combine<<<(unsigned)((total + 255) / 256), 256, 0, ctx->stream>>>(
        (const float *)(ws + w.P), (const int *)(ws + w.where_), (const float *)weights, (const float *)(ws + w.gate),
        offsets, (float *)Y, tokens, topk, width, experts);
    if (int rc = launched(ctx)) return rc;
    return stage_mark(ctx, -1);
}

}  // namespace smi
