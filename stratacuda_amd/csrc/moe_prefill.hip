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
// Grouped GEMM on MFMA (fp16 operands, f32 accumulation):
//  * Weights: (code - 1) * fp16 scale is exactly representable in fp16, so the
//    B operand holds the exact reference weights. In the streaming kernels a
//    pair of codes becomes an fp16 pair in three exact steps: one AND-OR puts
//    the two 2-bit codes under an fp16 exponent that makes each the units
//    digit (no shift per pair), a packed subtract leaves c - 1, a packed
//    multiply applies the group scale. Each wave dequantises its own B
//    fragments in registers once per K step.
//  * Activations are split once into hi = fp16(x) and lo = fp16(x - hi) (the
//    gate/up input by k_split_hilo, the down input by the gate/up epilogue);
//    two MFMAs (hi and lo) per K step give products accurate to ~2^-22
//    relative, well inside the 1e-4 / 1e-3 output tolerance, where a single
//    fp16 or bf16 pass is not. Valid for |x| < 65504.
//  * K order: within every 64-wide scale group, position q = 16w + 2p + o
//    holds element 16w + p + 8o. That is the order in which the pairs
//    (p, p+8) of word w come out of the code unpacking, so B needs no
//    shuffle; the activations are stored in the same order, so staging them
//    into LDS is a plain 16-byte copy and the MFMA A operand one 16-byte read.
//  * Tiles (width and ff among 512 / 2048, the benchmark shapes): below 1,024
//    tokens every segment runs in 16 x 256 blocks on v_mfma_f32_16x16x32_f16
//    (k_moe_gemm_rows16, k_moe_gemm_stream16), one grid; from 1,024 tokens
//    segments of more than 32 rows run in 64 x 256 blocks on
//    v_mfma_f32_32x32x16_f16 (k_moe_gemm_stream), the two grids covering
//    disjoint rows and running on two streams. Each block reads
//    its tile record (segment, first row, end row, segment start) written by
//    the dispatch, which tiles the shared expert's segment (every token) with
//    the routed ones.
//    Other shapes use k_moe_gemm (register-held B, A double-buffered in LDS,
//    64- and 32-row tiles).
//    grid.x = n-block (fastest) so the m-tiles of one (expert, n-block) run
//    on one XCD and share its L2.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int APITCH = 72;  // halves per staged A row: 64 + 8 padding (LDS banks)

// Position of element r (0..63) of a scale group in the MFMA K order.
__device__ __forceinline__ int k_position(int r) {
    const int w = r >> 4, t = r & 15;
    return 16 * w + 2 * (t & 7) + (t >> 3);
}

// X [rows x K] f32 -> hi/lo fp16 [rows][K/64][2][64] in the MFMA K order.
__global__ void __launch_bounds__(256) k_split_hilo(const float *__restrict__ X, _Float16 *__restrict__ out,
                                                    int64_t groups) {
    sm::split_hilo_chunk(X, out, (int64_t)blockIdx.x * blockDim.x + threadIdx.x, groups);
}

// The stack block's RMSNorm for small batches (kernels/strata.cu strata_norm
// mode 0, one gamma row, scale 1: the lane-strided sum of squares and its
// tree, as k_norm_reg forms it, so the f32 rows are bit-identical) writing
// the router's f32 input and, from the same registers, the hi/lo fp16 split
// of k_split_hilo for the expert GEMMs. One wave per row of NJ x 64 values.
template <int NJ>
__global__ void __launch_bounds__(256) k_norm_hilo(const float *__restrict__ X, const float *__restrict__ gamma,
                                                   float *__restrict__ Y, _Float16 *__restrict__ hl, int rows,
                                                   float eps) {
    const int row = (int)(blockIdx.x * 4 + (threadIdx.x >> 6)), lane = threadIdx.x & 63;
    if (row >= rows) return;
    constexpr int cols = NJ * 64;
    const float *xr = X + (int64_t)row * cols;
    float x[NJ], w[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) x[j] = xr[lane + 64 * j];
#pragma unroll
    for (int j = 0; j < NJ; j++) w[j] = gamma[lane + 64 * j];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) ss = ss + x[j] * x[j];
    ss = __shfl(sm::tree_sum64(ss), 0, 64);
    const float inv = 1.0f / sqrtf(ss / (float)cols + eps);
    float *yr = Y + (int64_t)row * cols;
    _Float16 *hr = hl + (int64_t)row * NJ * 128 + k_position(lane);
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        float y = x[j] * inv * w[j];
        yr[lane + 64 * j] = y;
        // The split starts from the stored f32 value: without this the
        // compiler rounds the product to fp16 directly (v_fma_mixlo_f16),
        // which differs from rounding the f32 result at ties.
        asm volatile("" : "+v"(y));
        const _Float16 h = (_Float16)y;
        hr[128 * j] = h;
        hr[128 * j + 64] = (_Float16)(y - (float)h);
    }
}

// SiLU for the fused prefill epilogue, whose outputs are checked to a
// tolerance (1e-4 + 1e-3 |e|): exp through the hardware v_exp_f32 (2^x) and a
// hardware reciprocal, a few ulp from the libm form.
__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ half2v codes_to_half2(uint32_t word, int p, half2v scale) {
    uint32_t t = ((word >> (2 * p)) & 0x00030003u) | 0x64006400u;  // fp16 (1024 + c_p, 1024 + c_{p+8})
    half2v h = __builtin_bit_cast(half2v, t);
    const half2v k1025 = {(_Float16)1025.0f, (_Float16)1025.0f};
    h = h - k1025;     // c - 1, exact
    return h * scale;  // (c - 1) * scale, exact in fp16
}

// B operand of K step s for lane half kh: positions 16s + 8kh .. +7, i.e. the
// pairs (p, p+8) of word s for p = 4kh .. 4kh+3.
__device__ __forceinline__ half8 b_operand(uint4 c, int s, int kh, half2v scale) {
    const uint32_t w = s == 0 ? c.x : s == 1 ? c.y : s == 2 ? c.z : c.w;
    const half2v p0 = codes_to_half2(w, 4 * kh + 0, scale), p1 = codes_to_half2(w, 4 * kh + 1, scale);
    const half2v p2 = codes_to_half2(w, 4 * kh + 2, scale), p3 = codes_to_half2(w, 4 * kh + 3, scale);
    const half8 b = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    return b;
}

// B operand of the streaming kernel, three VALU operations per pair. The lane
// works on w' = word >> 8 kh, whose pair q (q = 0..3) sits at bits 2q and
// 2q + 16, i.e. codes (p, p + 8) with p = 4 kh + q. OR-ing the masked bits
// under the fp16 exponent 10 - 2q makes each code the units digit of
// 2^(10-2q) + c; subtracting 2^(10-2q) + 1 leaves c - 1 exactly, and the
// product with the fp16 scale is exact. No per-pair shift is needed.
struct PairMagic {
    uint32_t mask[4];  // 0x00030003 << 2q, held in VGPRs (v_and_or_b32 takes one SGPR)
};
__device__ __forceinline__ PairMagic pair_magic() {
    PairMagic m;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        m.mask[q] = 0x00030003u << (2 * q);
        asm volatile("" : "+v"(m.mask[q]));
    }
    return m;
}
__device__ __forceinline__ uint32_t and_or_b32(uint32_t a, uint32_t mask, uint32_t bits) {
    return (a & mask) | bits;  // v_and_or_b32: mask in a VGPR, bits in an SGPR
}
template <int Q>
__device__ __forceinline__ half2v pair_q(uint32_t wq, const PairMagic &m, half2v scale) {
    constexpr uint32_t e = 25 - 2 * Q;                  // biased exponent of 2^(10-2q)
    constexpr uint32_t magic = (e << 10) | (e << 26);
    constexpr float sub = (float)((1 << (10 - 2 * Q)) + 1);
    const half2v h = __builtin_bit_cast(half2v, and_or_b32(wq, m.mask[Q], magic));
    const half2v k = {(_Float16)sub, (_Float16)sub};
    return (h - k) * scale;
}
// The four pairs of an already shifted word w'.
__device__ __forceinline__ half8 b_operand_word(uint32_t w, const PairMagic &m, half2v scale) {
    const half2v p0 = pair_q<0>(w, m, scale), p1 = pair_q<1>(w, m, scale);
    const half2v p2 = pair_q<2>(w, m, scale), p3 = pair_q<3>(w, m, scale);
    const half8 b = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
    return b;
}
__device__ __forceinline__ half8 b_operand_stream(uint4 c, int s, uint32_t shift, const PairMagic &m,
                                                  half2v scale) {
    return b_operand_word((s == 0 ? c.x : s == 1 ? c.y : s == 2 ? c.z : c.w) >> shift, m, scale);
}

// GATE_UP: A = X (hi/lo) rows gathered through rows[], K = width, N = 2*ff;
//          output H (hi/lo, K order) [positions][ff/64][2][64] = SiLU(gate) * up
//          of the interleaved column pairs.
// else:    A = H (hi/lo) rows by position, K = ff, N = width; output P f32
//          [positions x width].
template <bool GATE_UP, int MI, int NI, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) k_moe_gemm(const _Float16 *__restrict__ A, const int *__restrict__ rows,
                                                  const int4 *__restrict__ info, const int *__restrict__ tiles,
                                                  const uint8_t *__restrict__ arena, uint64_t stride,
                                                  const uint8_t *__restrict__ shared_blob, int experts,
                                                  uint64_t codes_off, uint64_t scales_off, int K, int N,
                                                  void *__restrict__ out, int out_ld) {
    constexpr int THREADS = 64 * WM * WN, BM = 32 * MI * WM, BN = 32 * NI * WN;
    constexpr int ACH = (BM * 16 + THREADS - 1) / THREADS;  // 16-byte A chunks per thread and group
    __shared__ __attribute__((aligned(16))) _Float16 lds[2][2 * BM * APITCH];  // [buf][hi/lo][row][APITCH]
    // Tile record (segment, first row, end of the segment) from the dispatch.
    const int tau = blockIdx.y;
    if (tau >= tiles[experts + 1]) return;
    const int4 ti = info[tau];
    const int e = ti.x, m0 = ti.y, mend = ti.z;
    const uint8_t *blob = e < experts ? arena + (uint64_t)e * stride : shared_blob;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int G = K / 64;

    // ---- A staging: chunk c = tid + THREADS i covers row c / 16, hi/lo
    // (c / 8) & 1, 8 halves (c & 7) * 8 of the group.
    const _Float16 *asrc[ACH];
    int adst[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const int c = tid + THREADS * i, r = c >> 4, hl = (c >> 3) & 1, part = c & 7;
        const int pos = m0 + r;
        asrc[i] = nullptr;
        adst[i] = -1;
        if (r < BM) adst[i] = (hl * BM + r) * APITCH + part * 8;
        if (r < BM && pos < mend) {
            const int64_t arow = GATE_UP ? rows[pos] : pos;
            asrc[i] = A + (arow * G * 2 + hl) * 64 + part * 8;
        }
    }
    uint4 areg[ACH];
    auto load_a = [&](int g) {
#pragma unroll
        for (int i = 0; i < ACH; i++)
            areg[i] = asrc[i] ? *(const uint4 *)(asrc[i] + (int64_t)g * 128) : make_uint4(0, 0, 0, 0);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; i++)
            if (adst[i] >= 0) *(uint4 *)&lds[buf][adst[i]] = areg[i];
    };

    // ---- B: lane (j = lane % 32, kh = lane / 32), weight rows n of the NI tiles
    const int j = lane & 31, kh = lane >> 5;
    const int nbase = blockIdx.x * BN + wn * 32 * NI;
    const uint8_t *brow[NI];
    const uint8_t *bsc[NI];
#pragma unroll
    for (int ni = 0; ni < NI; ni++) {
        const int n = nbase + ni * 32 + j;
        brow[ni] = blob + codes_off + (uint64_t)n * (K / 4);
        bsc[ni] = blob + scales_off + (uint64_t)n * G * 2;
    }
    uint4 bc[NI], bn[NI];
    uint32_t sc[NI], sn[NI];
    auto load_b = [&](int g, uint4 *c, uint32_t *s) {
#pragma unroll
        for (int ni = 0; ni < NI; ni++) {
            c[ni] = *(const uint4 *)(brow[ni] + (uint64_t)g * 16);
            s[ni] = *(const uint16_t *)(bsc[ni] + g * 2);
        }
    };

    float16v acc[MI][NI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[mi][ni][v] = 0.0f;

    load_a(0);
    load_b(0, bc, sc);
    store_a(0);
    if (G > 1) {
        load_a(1);
        load_b(1, bn, sn);
    }
    __syncthreads();
    for (int g = 0; g < G; g++) {
        const int buf = g & 1;
        half2v scale[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ni++) {
            const _Float16 s16 = __builtin_bit_cast(_Float16, (uint16_t)sc[ni]);
            scale[ni] = (half2v){s16, s16};
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half8 b[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ni++) b[ni] = b_operand(bc[ni], s, kh, scale[ni]);
#pragma unroll
            for (int mi = 0; mi < MI; mi++) {
                const int at = (wm * 32 * MI + mi * 32 + j) * APITCH + 16 * s + 8 * kh;
                const half8 ahi = *(const half8 *)&lds[buf][at];
                const half8 alo = *(const half8 *)&lds[buf][BM * APITCH + at];
#pragma unroll
                for (int ni = 0; ni < NI; ni++) {
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, b[ni], acc[mi][ni], 0, 0, 0);
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, b[ni], acc[mi][ni], 0, 0, 0);
                }
            }
        }
        if (g + 1 < G) {
            store_a(buf ^ 1);
#pragma unroll
            for (int ni = 0; ni < NI; ni++) {
                bc[ni] = bn[ni];
                sc[ni] = sn[ni];
            }
            if (g + 2 < G) {
                load_a(g + 2);
                load_b(g + 2, bn, sn);
            }
        }
        __syncthreads();
    }

    // ---- epilogue: acc[v] = D[i][j], i = 8*(v/4) + 4*kh + v%4 (32x32 tile)
#pragma unroll
    for (int mi = 0; mi < MI; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = wm * 32 * MI + mi * 32 + 8 * (v >> 2) + 4 * kh + (v & 3), pos = m0 + i;
                const int n = nbase + ni * 32 + j;
                if (GATE_UP) {
                    const float other = sm::dpp_f32<sm::kDppQuadXor1>(acc[mi][ni][v], acc[mi][ni][v]);
                    if ((j & 1) == 0 && pos < mend) {
                        const float h = silu_fast(acc[mi][ni][v]) * other;
                        const int jj = n >> 1;
                        _Float16 *dst = (_Float16 *)out + ((int64_t)pos * (out_ld / 64) + (jj >> 6)) * 128 +
                                        k_position(jj & 63);
                        const _Float16 hi = (_Float16)h;
                        dst[0] = hi;
                        dst[64] = (_Float16)(h - (float)hi);
                    }
                } else if (pos < mend) {
                    ((float *)out)[(int64_t)pos * out_ld + n] = acc[mi][ni][v];
                }
            }
}

// ---------------------------------------------------------------------------
// Streaming grouped GEMM: the same tiles and arithmetic as k_moe_gemm, fed by
// a ring of stages (one 64-wide scale group each) filled with direct
// global->LDS loads (global_load_lds_dwordx4: lane l of a wave writes 16 bytes
// at the instruction's LDS base + 16 l), so the next groups of A and B are in
// flight while the current one is multiplied, without occupying registers.
// The group count K / 64 is a template parameter, so the ring is unrolled
// into straight-line code and the compiler's own waits match the ring's.
// Each stage is its own __shared__ array: the compiler then tracks the
// loads into each stage separately and the waits are the explicit vmcnt
// below. Every thread issues the same number of loads per stage (rows past a
// segment's end load a valid row; those results are never stored), so one
// compile-time vmcnt covers all waves. 4 waves side by side in N: block tile
// (32 MI) x (128 NI), wave tile (32 MI) x (32 NI). Each lane keeps the scales
// of its weight rows (every group, K <= 2048) in registers.
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void *)lds_base, 16, 0, 0);
}
// Waits until at most N vector-memory operations of this wave are pending,
// then joins the block at a barrier. The empty asm statements with a memory
// clobber keep the compiler from moving LDS accesses across this point (the
// barrier intrinsic alone does not order memory operations).
template <int N>
__device__ __forceinline__ void ring_sync() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// This block's tile and column block. The hardware hands block L (x
// fastest) to XCD L % 8; block L takes tile (L / 8 / nx) * 8 + L % 8 and
// column block (L / 8) % nx, so all column blocks of one tile run on one XCD
// and read the tile's activation rows through one L2. Needs gridDim.y a
// multiple of 8 (the host rounds the tile bound up).
__device__ __forceinline__ void xcd_tile(int &tau, int &cb) {
    const int nx = gridDim.x, L = blockIdx.y * nx + blockIdx.x, idx = L >> 3;
    tau = (idx / nx) * 8 + (L & 7);
    cb = idx % nx;
}

constexpr int STREAM_MAX_G = 40;  // K <= 2560 for the streaming kernels (the real model's width)

// The G fp16 scales of one weight row (2G contiguous bytes) into G/2 words:
// 16-byte loads when a row is a whole number of them (G % 8 == 0), else
// 4-byte loads (G even: rows start 4-byte aligned).
template <int G>
__device__ __forceinline__ void load_row_scales(const uint8_t *p, uint32_t (&s)[G / 2]) {
    static_assert(G % 2 == 0, "an even number of groups");
    if constexpr (G % 8 == 0) {
        const uint4 *sp = (const uint4 *)p;
#pragma unroll
        for (int c = 0; c < G / 8; c++) {
            const uint4 v = sp[c];
            s[4 * c + 0] = v.x;
            s[4 * c + 1] = v.y;
            s[4 * c + 2] = v.z;
            s[4 * c + 3] = v.w;
        }
    } else {
        const uint32_t *sp = (const uint32_t *)p;
#pragma unroll
        for (int c = 0; c < G / 2; c++) s[c] = sp[c];
    }
}

// Ring stages. Each stage is a separate object at namespace scope: the
// compiler's wait insertion then tells loads into one stage from reads of
// another (stages declared inside the kernel made it wait for every load
// before any read). Big tiles (64 x 256) use three stages (60 KiB, two
// blocks per CU).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
template <int BM>
struct RingStage {
    v4u a[BM * 16];  // [hi/lo][row][8 slots of 16 B], slot = part ^ ((row >> 1) & 7)
    v4u b[256];      // [weight row] 16 B of codes (the tail is filler for 128-wide tiles)
};
__shared__ __attribute__((aligned(16))) RingStage<64> g_big0, g_big1, g_big2;

template <int BM>
struct Ring;
template <>
struct Ring<64> {
    static constexpr int NS = 3;
    template <int S>
    static __device__ __forceinline__ RingStage<64> &stage() {
        return S == 0 ? g_big0 : S == 1 ? g_big1 : g_big2;
    }
};
// 16-row tiles (k_moe_gemm_stream16): 8 KiB stages, six of them (48 KiB,
// three blocks per CU).
__shared__ __attribute__((aligned(16))) RingStage<16> g_tiny0, g_tiny1, g_tiny2, g_tiny3, g_tiny4, g_tiny5;
template <>
struct Ring<16> {
    static constexpr int NS = 6;
    template <int S>
    static __device__ __forceinline__ RingStage<16> &stage() {
        return S == 0 ? g_tiny0 : S == 1 ? g_tiny1 : S == 2 ? g_tiny2 : S == 3 ? g_tiny3 : S == 4 ? g_tiny4 : g_tiny5;
    }
};
// Calls f(stage S) for the S equal to `slot` (slot is a constant once the
// group loop is unrolled).
template <int BM, typename F>
__device__ __forceinline__ void with_stage(int slot, F &&f) {
    switch (slot) {
    case 0: f(Ring<BM>::template stage<0>()); break;
    case 1: f(Ring<BM>::template stage<1 % Ring<BM>::NS>()); break;
    case 2: f(Ring<BM>::template stage<2 % Ring<BM>::NS>()); break;
    case 3: f(Ring<BM>::template stage<3 % Ring<BM>::NS>()); break;
    case 4: f(Ring<BM>::template stage<4 % Ring<BM>::NS>()); break;
    default: f(Ring<BM>::template stage<5 % Ring<BM>::NS>()); break;
    }
}

template <bool GATE_UP, int MI, int NI>
struct StreamGemm {
    static constexpr int BM = 32 * MI, BN = 128 * NI;
    static constexpr int ACH = BM * 16 / 256;             // A loads per thread per stage
    static constexpr int BCH = (BN + 255) / 256;          // B loads per thread per stage
    static constexpr int PER_STAGE = ACH + BCH;
};

template <bool GATE_UP, int MI, int NI, int KG>
__global__ void __launch_bounds__(256) k_moe_gemm_stream(const _Float16 *__restrict__ A, const int *__restrict__ rows,
                                                         const int4 *__restrict__ info, const int *__restrict__ tiles,
                                                         const uint8_t *__restrict__ arena, uint64_t stride,
                                                         const uint8_t *__restrict__ shared_blob, int experts,
                                                         uint64_t codes_off, uint64_t scales_off, int K, int N,
                                                         void *__restrict__ out, int out_ld) {
    using P = StreamGemm<GATE_UP, MI, NI>;
    constexpr int BM = P::BM, BN = P::BN, ACH = P::ACH, BCH = P::BCH;
    using Stage = RingStage<BM>;
    constexpr int NS = Ring<BM>::NS;
    static_assert(KG >= 8 && KG <= STREAM_MAX_G && KG % 2 == 0, "K / 64 groups");
    static_assert(BM <= 64 && BN <= 256, "stage size");
    // Tile record (segment, first row, end of the segment) from the dispatch.
    int tau, cb;
    xcd_tile(tau, cb);
    if (tau >= tiles[experts + 1]) return;
    const int4 ti = info[tau];
    const int e = ti.x, m0 = ti.y, mend = ti.z;
    const uint8_t *blob = e < experts ? arena + (uint64_t)e * stride : shared_blob;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    constexpr int G = KG;  // K / 64, fixed at compile time: the ring is straight-line code
    (void)K;
    const int n0 = cb * BN;

    // Per-thread DMA sources. A chunk c = tid + 256 i: hi/lo c / (8 BM), row
    // (c / 8) % BM, slot c % 8 holding part slot ^ ((row / 2) & 7). A 128-bit
    // LDS read serves 16 lanes per pass; the 16 rows a pass reads (one part
    // each) then fall on 16 distinct 16-byte bank groups.
    const _Float16 *asrc[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const int c = tid + 256 * i, hl = c / (8 * BM), r = (c >> 3) % BM, part = (c & 7) ^ ((r >> 1) & 7);
        const int pos = min(m0 + r, mend - 1);  // rows past the end load the segment's last row
        // gate/up: the routed rows' tokens from the dispatch; the shared
        // expert's segment holds every token in order from its start
        const int64_t arow = GATE_UP ? (e < experts ? rows[pos] : pos - ti.w) : pos;
        asrc[i] = A + (arow * G * 2 + hl) * 64 + part * 8;
    }
    const uint8_t *bsrc[BCH];
#pragma unroll
    for (int i = 0; i < BCH; i++) {
        const int c = tid + 256 * i;
        const int n = n0 + (c < BN ? c : c % BN);  // filler lanes reload rows of the tile
        bsrc[i] = blob + codes_off + (uint64_t)n * (K / 4);
    }
    auto issue = [&](Stage &sg, int g) {
#pragma unroll
        for (int i = 0; i < ACH; i++) dma16(asrc[i] + (int64_t)g * 128, &sg.a[256 * i + 64 * wave]);
#pragma unroll
        for (int i = 0; i < BCH; i++) dma16(bsrc[i] + (uint64_t)g * 16, &sg.b[256 * i + 64 * wave]);
    };
    const int j = lane & 31, kh = lane >> 5;
    // Scales of the lane's weight rows, every group, in registers: the plane
    // is [row][G] fp16, so a row is 2G contiguous bytes and the 32 lanes of a
    // half-wave read 32 consecutive rows. Issued before the ring, so the
    // ring's first wait also covers them.
    uint32_t sreg[NI][G / 2];
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
        load_row_scales<G>(blob + scales_off + (uint64_t)(n0 + wave * 32 * NI + ni * 32 + j) * G * 2, sreg[ni]);
#pragma clang loop unroll(full)
    for (int q = 0; q < NS - 1; q++) with_stage<BM>(q, [&](Stage &sg) { issue(sg, min(q, G - 1)); });

    const PairMagic magic = pair_magic();
    const uint32_t shift = 8 * kh;
    float16v acc[MI][NI];
#pragma unroll
    for (int mi = 0; mi < MI; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[mi][ni][v] = 0.0f;

    auto compute = [&](const Stage &sg, int g) {
        uint4 codes[NI];
        half2v scale[NI];
#pragma unroll
        for (int ni = 0; ni < NI; ni++) {
            const int nl = wave * 32 * NI + ni * 32 + j;
            const v4u cv = sg.b[nl];
            codes[ni] = make_uint4(cv.x, cv.y, cv.z, cv.w);
            const uint16_t s16 = (uint16_t)(sreg[ni][g >> 1] >> (16 * (g & 1)));
            const _Float16 sh = __builtin_bit_cast(_Float16, s16);
            scale[ni] = (half2v){sh, sh};
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half8 b[NI];
#pragma unroll
            for (int ni = 0; ni < NI; ni++) b[ni] = b_operand_stream(codes[ni], s, shift, magic, scale[ni]);
#pragma unroll
            for (int mi = 0; mi < MI; mi++) {
                const int r = mi * 32 + j, slot = (2 * s + kh) ^ ((r >> 1) & 7);
                const half8 ahi = __builtin_bit_cast(half8, sg.a[r * 8 + slot]);
                const half8 alo = __builtin_bit_cast(half8, sg.a[(BM + r) * 8 + slot]);
#pragma unroll
                for (int ni = 0; ni < NI; ni++) {
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ahi, b[ni], acc[mi][ni], 0, 0, 0);
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(alo, b[ni], acc[mi][ni], 0, 0, 0);
                }
            }
        }
    };
    // Ring of NS stages: before step g the groups up to g + NS - 2 have been
    // issued; the wait leaves the NS - 2 after g in flight, and the slot
    // that step g-1 consumed is refilled with group g + NS - 1. Loads past the
    // last group repeat group G-1 (their data is never read), so every step
    // has the same number of loads in flight and no branch separates a load
    // from the reads that follow it.
    constexpr int PS = P::PER_STAGE;
#pragma clang loop unroll(full)
    for (int g = 0; g < G; g++) {
        ring_sync<PS * (NS - 2)>();
        with_stage<BM>((g + NS - 1) % NS, [&](Stage &sg) { issue(sg, min(g + NS - 1, G - 1)); });
        with_stage<BM>(g % NS, [&](Stage &sg) { compute(sg, g); });
    }
    // No load may still be writing LDS when the block ends.
    ring_sync<0>();

    // ---- epilogue: acc[v] = D[i][j], i = 8*(v/4) + 4*kh + v%4 (32x32 tile)
#pragma unroll
    for (int mi = 0; mi < MI; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int i = mi * 32 + 8 * (v >> 2) + 4 * kh + (v & 3), pos = m0 + i;
                const int n = n0 + wave * 32 * NI + ni * 32 + j;
                if (GATE_UP) {
                    const float other = sm::dpp_f32<sm::kDppQuadXor1>(acc[mi][ni][v], acc[mi][ni][v]);
                    if ((j & 1) == 0 && pos < mend) {
                        const float h = silu_fast(acc[mi][ni][v]) * other;
                        const int jj = n >> 1;
                        _Float16 *dst = (_Float16 *)out + ((int64_t)pos * (out_ld / 64) + (jj >> 6)) * 128 +
                                        k_position(jj & 63);
                        const _Float16 hi = (_Float16)h;
                        dst[0] = hi;
                        dst[64] = (_Float16)(h - (float)hi);
                    }
                } else if (pos < mend) {
                    ((float *)out)[(int64_t)pos * out_ld + n] = acc[mi][ni][v];
                }
            }
}

// The streaming kernel for short segments: 16-row tiles on
// v_mfma_f32_16x16x32_f16, so a segment of ~10 rows (the typical expert at a
// few hundred tokens) pays for 16 rows of MFMA work instead of 32. Block:
// 16 rows x 256 weight rows, 4 waves side by side in N, each 16 x 64 (four
// 16 x 16 tiles). The 16x16x32 operands: lane l holds row (or column) l % 16
// and K positions 8 (l / 16) .. +7 of a 32-wide step. With the K order of the
// activations, step s of a 64-wide group and lane quarter kq = l / 16 map to
// code word 2s + kq / 2, byte half kq % 2 (the same unpacking as the 32-row
// kernel's lane halves) and to the 16-byte part 4s + kq of the A row.
// Result: lane l holds rows 4 (l / 16) + i (i = 0..3) of column l % 16.
typedef float float4v __attribute__((ext_vector_type(4)));
template <bool GATE_UP, int KG>
__global__ void __launch_bounds__(256) k_moe_gemm_stream16(const _Float16 *__restrict__ A, const int *__restrict__ rows,
                                                           const int4 *__restrict__ info,
                                                           const int *__restrict__ tiles,
                                                           const uint8_t *__restrict__ arena, uint64_t stride,
                                                           const uint8_t *__restrict__ shared_blob, int experts,
                                                           uint64_t codes_off, uint64_t scales_off, int K, int N,
                                                           void *__restrict__ out, int out_ld) {
    constexpr int BM = 16, BN = 256, NT = 4;  // NT tiles of 16 columns per wave
    using Stage = RingStage<BM>;
    constexpr int NS = Ring<BM>::NS;
    constexpr int G = KG;  // K / 64
    static_assert(KG >= 8 && KG <= STREAM_MAX_G && KG % 2 == 0, "K / 64 groups");
    (void)K;
    (void)N;
    // Tile record (segment, first row, end of the segment) from the dispatch.
    int tau, cb;
    xcd_tile(tau, cb);
    if (tau >= tiles[experts + 1]) return;
    const int4 ti = info[tau];
    const int e = ti.x, m0 = ti.y, mend = ti.z;
    const uint8_t *blob = e < experts ? arena + (uint64_t)e * stride : shared_blob;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = cb * BN;

    // DMA sources, one A and one B load per thread per stage. A chunk
    // c = tid: hi/lo c / 128, row (c / 8) % 16, slot c % 8 holding part
    // slot ^ ((row / 2) & 7).
    const _Float16 *asrc;
    {
        const int hl = tid >> 7, r = (tid >> 3) & 15, part = (tid & 7) ^ ((r >> 1) & 7);
        const int pos = min(m0 + r, mend - 1);  // rows past the end load the segment's last row
        const int64_t arow = GATE_UP ? (e < experts ? rows[pos] : pos - ti.w) : pos;
        asrc = A + (arow * G * 2 + hl) * 64 + part * 8;
    }
    const uint8_t *bsrc = blob + codes_off + (uint64_t)(n0 + tid) * (G * 16);
    auto issue = [&](Stage &sg, int g) {
        dma16(asrc + (int64_t)g * 128, &sg.a[64 * wave]);
        dma16(bsrc + (uint64_t)g * 16, &sg.b[64 * wave]);
    };
    const int col = lane & 15, kq = lane >> 4;
    // Scales of the lane's four weight rows, every group, in registers.
    uint32_t sreg[NT][G / 2];
#pragma unroll
    for (int nt = 0; nt < NT; nt++)
        load_row_scales<G>(blob + scales_off + (uint64_t)(n0 + wave * 64 + nt * 16 + col) * G * 2, sreg[nt]);
#pragma clang loop unroll(full)
    for (int q = 0; q < NS - 1; q++) with_stage<BM>(q, [&](Stage &sg) { issue(sg, min(q, G - 1)); });

    const PairMagic magic = pair_magic();
    // Byte selector of the lane's code word: word x (kq < 2) or y, moved
    // down by one byte for odd kq (v_perm_b32: 0-3 pick bytes of the second
    // source, 4-7 of the first, 0x0c gives zero).
    const uint32_t psel = kq == 0 ? 0x03020100u : kq == 1 ? 0x0c030201u : kq == 2 ? 0x07060504u : 0x0c070605u;
    float4v acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) acc[nt] = (float4v){0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const Stage &sg, int g) {
        uint32_t words[NT][2];  // the lane's code word of step 0 and 1, shifted
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const v4u cv = sg.b[wave * 64 + nt * 16 + col];
            words[nt][0] = __builtin_amdgcn_perm(cv.y, cv.x, psel);
            words[nt][1] = __builtin_amdgcn_perm(cv.w, cv.z, psel);
        }
        half2v scale[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const uint16_t s16 = (uint16_t)(sreg[nt][g >> 1] >> (16 * (g & 1)));
            const _Float16 sh = __builtin_bit_cast(_Float16, s16);
            scale[nt] = (half2v){sh, sh};
        }
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int part = 4 * s + kq, slot = part ^ ((col >> 1) & 7);
            const half8 ahi = __builtin_bit_cast(half8, sg.a[col * 8 + slot]);
            const half8 alo = __builtin_bit_cast(half8, sg.a[(BM + col) * 8 + slot]);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const half8 b = b_operand_word(words[nt][s], magic, scale[nt]);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, b, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, b, acc[nt], 0, 0, 0);
            }
        }
    };
    constexpr int PS = 2;  // loads per thread per stage
#pragma clang loop unroll(full)
    for (int g = 0; g < G; g++) {
        ring_sync<PS * (NS - 2)>();
        with_stage<BM>((g + NS - 1) % NS, [&](Stage &sg) { issue(sg, min(g + NS - 1, G - 1)); });
        with_stage<BM>(g % NS, [&](Stage &sg) { compute(sg, g); });
    }
    // No load may still be writing LDS when the block ends.
    ring_sync<0>();

#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pos = m0 + 4 * kq + i, n = n0 + wave * 64 + nt * 16 + col;
            if (GATE_UP) {
                const float other = sm::dpp_f32<sm::kDppQuadXor1>(acc[nt][i], acc[nt][i]);
                if ((col & 1) == 0 && pos < mend) {
                    const float h = silu_fast(acc[nt][i]) * other;
                    const int jj = n >> 1;
                    _Float16 *dst =
                        (_Float16 *)out + ((int64_t)pos * (out_ld / 64) + (jj >> 6)) * 128 + k_position(jj & 63);
                    const _Float16 hi = (_Float16)h;
                    dst[0] = hi;
                    dst[64] = (_Float16)(h - (float)hi);
                }
            } else if (pos < mend) {
                ((float *)out)[(int64_t)pos * out_ld + n] = acc[nt][i];
            }
        }
}

// The 16-row kernel for K a multiple of 256, in supersteps of four scale
// groups. Weight codes go from HBM straight to the lanes that use them: in
// superstep S, lane (col, kq) of wave w loads the 16 code bytes of group
// 4S + kq of weight rows n0 + 64w + 16nt + col (nt = 0..3). One load
// instruction then reads 64 contiguous bytes of each of 16 rows (reading 16
// bytes of each of 64 rows instead, with the weights staged through LDS,
// streams at about half the rate), and the lane holds exactly its B operands
// of the superstep's eight 32-wide MFMA steps: step t takes word t / 2, byte
// half t % 2 of its group. The four lane quarters of one MFMA thus work on
// four different groups, with the activations read to match; the sum over K
// is the same. Activations (16 rows x 4 groups, hi/lo, 16 KiB a superstep)
// are staged in LDS by DMA, three slots deep: lane (row col, kq) reads part t
// of group 4S + kq. One barrier per superstep.
__shared__ __attribute__((aligned(16))) v4u g_rows16_0[4 * 256], g_rows16_1[4 * 256], g_rows16_2[4 * 256];

// An empty volatile statement that reads and rewrites the registers: code
// using them cannot move above the volatile wait before it.
template <int NT>
__device__ __forceinline__ void pin_operands(v4u (&b)[NT], uint32_t (&s)[NT]) {
#pragma unroll
    for (int i = 0; i < NT; i++) asm volatile("" : "+v"(b[i]), "+v"(s[i]));
}

template <bool GATE_UP, int KG, int NT = 4>
__global__ void __launch_bounds__(256, 3) k_moe_gemm_rows16(const _Float16 *__restrict__ A, const int *__restrict__ rows,
                                                         const int4 *__restrict__ info, const int *__restrict__ tiles,
                                                         const uint8_t *__restrict__ arena, uint64_t stride,
                                                         const uint8_t *__restrict__ shared_blob, int experts,
                                                         uint64_t codes_off, uint64_t scales_off, int K, int N,
                                                         void *__restrict__ out, int out_ld) {
    // NT column tiles of 16 per wave: a block covers 64 NT weight rows (NT = 4
    // for most batches; 1 where few tiles would leave the GPU idle).
    constexpr int BN = 64 * NT, G = KG, NSS = KG / 4;
    static_assert(KG % 4 == 0 && KG >= 8 && KG <= STREAM_MAX_G, "whole supersteps of four groups");
    static_assert(NT == 1 || NT == 2 || NT == 4, "1, 2 or 4 column tiles per wave");
    (void)K;
    (void)N;
    int tau, cb;
    xcd_tile(tau, cb);
    if (tau >= tiles[experts + 1]) return;
    const int4 ti = info[tau];
    const int e = ti.x, m0 = ti.y, mend = ti.z;
    const uint8_t *blob = e < experts ? arena + (uint64_t)e * stride : shared_blob;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = cb * BN, col = lane & 15, kq = lane >> 4;

    // Activation DMA: chunk tid of a group is hi/lo tid / 128, row
    // (tid / 8) % 16, slot tid % 8 holding part slot ^ ((row / 2) & 7).
    const _Float16 *asrc;
    {
        const int hl = tid >> 7, r = (tid >> 3) & 15, part = (tid & 7) ^ ((r >> 1) & 7);
        const int pos = min(m0 + r, mend - 1);  // rows past the end load the segment's last row
        const int64_t arow = GATE_UP ? (e < experts ? rows[pos] : pos - ti.w) : pos;
        asrc = A + (arow * G * 2 + hl) * 64 + part * 8;
    }
    // Group j of superstep S goes to 256 j of the superstep's half.
    auto issue_a = [&](v4u *half, int S) {
#pragma unroll
        for (int j = 0; j < 4; j++) dma16(asrc + (int64_t)(4 * S + j) * 128, &half[256 * j + 64 * wave]);
    };
    // Byte offsets from the block's blob (32 bits: a blob is under 4 GiB),
    // so the loads take the blob address from scalar registers.
    const uint8_t *bcodes = blob + codes_off, *bscales = blob + scales_off;
    uint32_t boff[NT], soff[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const uint32_t n = (uint32_t)(n0 + wave * 16 * NT + nt * 16 + col);
        boff[nt] = n * (G * 16) + kq * 16;
        soff[nt] = n * (G * 2) + kq * 2;
    }
    auto load_b = [&](v4u (&b)[NT], int S) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) b[nt] = *(const v4u *)(bcodes + boff[nt] + S * 64);
    };
    auto load_s = [&](uint32_t (&s)[NT], int S) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) s[nt] = *(const uint16_t *)(bscales + soff[nt] + S * 8);
    };

    const PairMagic magic = pair_magic();
    float4v acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) acc[nt] = (float4v){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const v4u *half, const v4u (&b)[NT], const uint32_t (&s)[NT]) {
        half2v scale[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const _Float16 sh = __builtin_bit_cast(_Float16, (uint16_t)s[nt]);
            scale[nt] = (half2v){sh, sh};
        }
        const v4u *ag = half + 256 * kq;  // the lane's group of the superstep
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int slot = t ^ ((col >> 1) & 7);
            const half8 ahi = __builtin_bit_cast(half8, ag[col * 8 + slot]);
            const half8 alo = __builtin_bit_cast(half8, ag[(16 + col) * 8 + slot]);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const uint32_t w = (t >> 1) == 0 ? b[nt].x : (t >> 1) == 1 ? b[nt].y : (t >> 1) == 2 ? b[nt].z : b[nt].w;
                const half8 bb = b_operand_word(w >> (8 * (t & 1)), magic, scale[nt]);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bb, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bb, acc[nt], 0, 0, 0);
            }
        }
    };
    // Superstep S in flight: 4 DMAs, NT code loads, NT scale loads per
    // thread, issued in that order, all of S before any of S + 1 (memory
    // fences between the supersteps: the waits count loads in issue order).
    // Three slots: superstep S + 2 is issued into the slot of S - 1 once
    // every wave has passed the barrier that starts S.
    constexpr int PER_SS = 4 + 2 * NT;
    v4u b0[NT], b1[NT], b2[NT];
    uint32_t s0[NT], s1[NT], s2[NT];
    auto issue = [&](int S) {
        if (S % 3 == 0) {
            issue_a(g_rows16_0, S);
            load_b(b0, S);
            load_s(s0, S);
        } else if (S % 3 == 1) {
            issue_a(g_rows16_1, S);
            load_b(b1, S);
            load_s(s1, S);
        } else {
            issue_a(g_rows16_2, S);
            load_b(b2, S);
            load_s(s2, S);
        }
        asm volatile("" ::: "memory");
    };
    issue(0);
    if (NSS > 1) issue(1);
#pragma clang loop unroll(full)
    for (int S = 0; S < NSS; S++) {
        // Superstep S complete for this wave (S + 1 may stay in flight),
        // then for every wave.
        if (S + 1 < NSS) ring_sync<PER_SS>();
        else ring_sync<0>();
        if (S + 2 < NSS) issue(S + 2);
        // The unpacking of the superstep's codes stays behind the wait (the
        // compiler would otherwise start it early and wait for every load).
        if (S % 3 == 0) {
            pin_operands(b0, s0);
            compute(g_rows16_0, b0, s0);
        } else if (S % 3 == 1) {
            pin_operands(b1, s1);
            compute(g_rows16_1, b1, s1);
        } else {
            pin_operands(b2, s2);
            compute(g_rows16_2, b2, s2);
        }
    }

#pragma unroll
    for (int nt = 0; nt < NT; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int pos = m0 + 4 * kq + i, n = n0 + wave * 16 * NT + nt * 16 + col;
            if (GATE_UP) {
                const float other = sm::dpp_f32<sm::kDppQuadXor1>(acc[nt][i], acc[nt][i]);
                if ((col & 1) == 0 && pos < mend) {
                    const float h = silu_fast(acc[nt][i]) * other;
                    const int jj = n >> 1;
                    _Float16 *dst =
                        (_Float16 *)out + ((int64_t)pos * (out_ld / 64) + (jj >> 6)) * 128 + k_position(jj & 63);
                    const _Float16 hi = (_Float16)h;
                    dst[0] = hi;
                    dst[64] = (_Float16)(h - (float)hi);
                }
            } else if (pos < mend) {
                ((float *)out)[(int64_t)pos * out_ld + n] = acc[nt][i];
            }
        }
}

// Y[t, d] = P[shared(t), d] * sigmoid(gate[t]) + sum_k P[where[t,k], d] * w[t,k]
// in the reference order (kernels/strata.cu:470-476); with `resid`,
// Y = resid + that (strata_elementwise mode 5). One block per token (and
// column block): each thread combines 4 consecutive outputs per step with
// 16-byte loads. Needs width % 4 == 0 (topk <= 32, checked by the caller's
// geometry check).
__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ P, const int *__restrict__ where_,
                                                 const float *__restrict__ weights, const float *__restrict__ gate,
                                                 int64_t shared_base, float *__restrict__ Y, int tokens,
                                                 int topk, int width, const float *__restrict__ resid) {
    // The token's slot positions, weights and gate are the same for every
    // thread of the block (scalar loads), and the parts of up to
    // kCombineRound slots are loaded before any is added (in slot order), so
    // a top-10 token waits for one round of loads.
    constexpr int kCombineRound = 16;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int *wt = where_ + (int64_t)t * topk;
    const float *ww = weights + (int64_t)t * topk;
    const float sig = sm::sigmoid(gate[t]);
    const float4 *shared_row = (const float4 *)(P + (shared_base + t) * width);
    // block (t, c) covers float4 columns c x 256 + tid, in steps of the
    // grid's column extent
    for (int d4 = blockIdx.y * blockDim.x + tid; d4 < width / 4; d4 += blockDim.x * gridDim.y) {
        const float4 s = shared_row[d4];
        float4 v = {s.x * sig, s.y * sig, s.z * sig, s.w * sig};
        for (int k0 = 0; k0 < topk; k0 += kCombineRound) {
            float4 part[kCombineRound];
            float w[kCombineRound];
#pragma unroll
            for (int j = 0; j < kCombineRound; j++) {
                const int pos = k0 + j < topk ? wt[k0 + j] : -1;
                w[j] = k0 + j < topk ? ww[k0 + j] : 0.0f;
                part[j] = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""));
                if (pos >= 0) part[j] = ((const float4 *)(P + (int64_t)pos * width))[d4];
            }
#pragma unroll
            for (int j = 0; j < kCombineRound; j++) {
                if (k0 + j < topk) {
                    v.x = v.x + part[j].x * w[j];
                    v.y = v.y + part[j].y * w[j];
                    v.z = v.z + part[j].z * w[j];
                    v.w = v.w + part[j].w * w[j];
                }
            }
        }
        if (resid) {
            const float4 h = ((const float4 *)(resid + (int64_t)t * width))[d4];
            v = make_float4(h.x + v.x, h.y + v.y, h.z + v.z, h.w + v.w);
        }
        ((float4 *)(Y + (int64_t)t * width))[d4] = v;
    }
}

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Batches of fewer than kOneGridTokens tokens tile every segment (at most
// `tokens` rows: a token routes to an expert once, and the shared segment
// holds each token once) in 16-row tiles, so the 64-row grid is not launched
// and the products need no second stream; larger ones tile segments of more
// than 32 rows in 64-row tiles, on the second stream beside the 16-row grid.
// (Graph replays on one GPU, the 64-row grid forked beside the 16-row one
// against one grid: 512 tokens, uniform routing, 0.261-0.268 -> 0.229-0.239
// ms per layer; stack blocks of 128 / 256 / 512 tokens 144 / 185 / 225 ->
// 126 / 165 / 211 us. From 1,024 tokens one grid loses once the router is
// skewed: 1,024 tokens with a Zipf-biased router 0.277 -> 0.302 ms, 1,536
// tokens 0.372 -> 0.415 ms; with uniform routing 0.373 -> 0.365 and 0.460 ->
// 0.465 ms.)
constexpr int kOneGridTokens = 1024;
constexpr int kSmallBatch = 64;
constexpr int kSmallBatchColumnTiles = 2;  // column tiles per wave of the 16-row kernel up to kSmallBatch tokens
inline int tiling_split(int tokens) { return tokens < kOneGridTokens ? tokens + 1 : 33; }

// Grid bounds of the two tilings over the experts + 1 segments of m rows:
// a segment of r < split rows takes ceil(r / 16) <= r / 16 + 1 small tiles
// (at most two when split is 33 or less); a longer one ceil(r / 64) big
// tiles, in all at most m / 64 + (number of such segments <= m / 33).
inline uint64_t small_tile_bound(uint64_t m, int experts, int split) {
    const uint64_t segs = (uint64_t)experts + 1;
    const uint64_t any = m / 16 + std::min(segs, m) + 1;
    return split <= 33 ? std::min(any, 2 * segs + 1) : any;
}
inline uint64_t big_tile_bound(uint64_t m, int experts) {
    return m / 64 + std::min((uint64_t)experts + 1, m / 33) + 1;
}

struct PrefillWs {
    uint64_t logits, rcert, gate, dispatch, offsets, tiles_small, tiles_big, info_small, info_big,
        rows, parts, where_, Xhl, Hhl, P, Xn, end;
};
PrefillWs prefill_ws(int tokens, int width, int ff, int experts, int topk, bool block = false) {
    const uint64_t n = (uint64_t)tokens * topk, m = n + tokens;
    PrefillWs w;
    w.logits = 0;
    w.rcert = up(w.logits + (uint64_t)tokens * experts * 4);
    w.gate = up(w.rcert + route_cert_workspace(tokens, width, experts));
    w.dispatch = up(w.gate + (uint64_t)tokens * 4);
    w.offsets = up(w.dispatch + dispatch_workspace(tokens, experts));
    w.tiles_small = up(w.offsets + ((uint64_t)experts + 2) * 4);
    w.tiles_big = up(w.tiles_small + ((uint64_t)experts + 2) * 4);
    w.info_small = up(w.tiles_big + ((uint64_t)experts + 2) * 4);
    w.info_big = up(w.info_small + small_tile_bound(m, experts, tiling_split(tokens)) * 16);
    w.rows = up(w.info_big + big_tile_bound(m, experts) * 16);
    w.parts = up(w.rows + m * 4);
    w.where_ = up(w.parts + m * 4);
    w.Xhl = up(w.where_ + n * 4);
    w.Hhl = up(w.Xhl + (uint64_t)tokens * width * 4);
    w.P = up(w.Hhl + m * ff * 4);
    w.Xn = up(w.P + m * width * 4);
    w.end = block ? up(w.Xn + (uint64_t)tokens * width * 4) : w.Xn;
    return w;
}

}  // namespace

namespace smi {

uint64_t moe_prefill_workspace(int tokens, int width, int ff, int experts, int topk, bool block) {
    return prefill_ws(tokens, width, ff, experts, topk, block).end;
}

int64_t moe_prefill_route_stats_offset(int tokens, int width, int ff, int experts, int topk) {
    if (!route_cert_applies(tokens, width, experts, topk)) return -1;
    return (int64_t)(prefill_ws(tokens, width, ff, experts, topk).rcert +
                     route_cert_stats_offset(tokens, width, experts));
}

int moe_prefill(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
                uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y, uint64_t ids,
                uint64_t weights, uint64_t workspace, uint64_t workspace_bytes, const BlockArgs *block) {
    (void)workspace_bytes;
    PrefillWs w = prefill_ws(tokens, width, ff, experts, topk, block != nullptr);
    char *ws = (char *)workspace;
    const float *resid = nullptr;
    if ((2 * ff) % 128 || width % 128)
        return fail(ctx, SM_E_ARG, "prefill needs width and 2*ff to be multiples of 128");
    // Streaming kernels: N a multiple of 256 and K one of the compiled group
    // counts in both products (512, 640, 2048, 2560: the benchmark's and the
    // real model's shapes). Every segment then runs in 16-row tiles below
    // kOneGridTokens tokens; from there on segments of up to 32 rows do, and
    // longer ones run in 64-row tiles. Other shapes: segments of up to 32
    // rows in one 32-row tile, longer ones in 64-row tiles (k_moe_gemm).
    auto streamable = [](int k) { return k == 512 || k == 640 || k == 2048 || k == 2560; };
    const bool stream = (2 * ff) % 256 == 0 && width % 256 == 0 && streamable(width) && streamable(ff);
    // Streaming shapes issue the split, the router and the dispatch on the
    // library's stream: a fork to the second stream and the join back inside
    // a graph cost more than the overlap they buy (A/B on one GPU, graph
    // replays: 8 stack blocks of 32 tokens 87.8 -> 72.1 us, 64 tokens 108 ->
    // 94, 128 tokens 166 -> 150, 256 tokens 198 -> 186; the T=2048 layer
    // 0.462 -> 0.455 ms, T=512 unchanged; the shared expert's products had
    // run on the second stream beside the router, now the dispatch tiles its
    // segment with the routed ones). In the stack block the normalisation
    // writes the split itself, from the same registers.
    const bool one_stream = stream;
    const bool hilo_in_norm = one_stream && block && (width == 2048 || width == 2560);
    if (block) {
        // The stage runs on RMSNorm(X) and the combine adds X back.
        if (hilo_in_norm) {
            const unsigned nb = (unsigned)((tokens + 3) / 4);
            auto kn = width == 2048 ? k_norm_hilo<32> : k_norm_hilo<40>;
            kn<<<nb, 256, 0, ctx->stream>>>((const float *)X, (const float *)block->gamma, (float *)(ws + w.Xn),
                                            (_Float16 *)(ws + w.Xhl), tokens, block->eps);
            if (int rc = launched(ctx)) return rc;
        } else if (int rc = norm_launch(ctx, (const float *)X, (const float *)block->gamma, (float *)(ws + w.Xn),
                                        width, tokens, block->eps)) {
            return rc;
        }
        resid = (const float *)X;
        X = (uint64_t)(ws + w.Xn);
    }
    BlobLayout L = blob_layout(width, ff);
    const int split = stream ? tiling_split(tokens) : 33;
    const int64_t routed_rows = (int64_t)tokens * topk;  // the shared expert's segment starts here
    const _Float16 *xhl = (const _Float16 *)(ws + w.Xhl), *hhl = (const _Float16 *)(ws + w.Hhl);
    const uint8_t *ar = (const uint8_t *)arena, *sh = (const uint8_t *)shared_blob;

    // Streaming GEMM launchers by K: 64-row tiles, and 16-row tiles in whole
    // supersteps of four groups where K allows (512, 2048, 2560), else one
    // group per ring step (640).
    using KT = decltype(&k_moe_gemm_stream<true, 2, 2, 8>);
    auto big_kernel = [](bool gate_up, int K) -> KT {
        const KT gu[4] = {k_moe_gemm_stream<true, 2, 2, 8>, k_moe_gemm_stream<true, 2, 2, 10>,
                          k_moe_gemm_stream<true, 2, 2, 32>, k_moe_gemm_stream<true, 2, 2, 40>};
        const KT dn[4] = {k_moe_gemm_stream<false, 2, 2, 8>, k_moe_gemm_stream<false, 2, 2, 10>,
                          k_moe_gemm_stream<false, 2, 2, 32>, k_moe_gemm_stream<false, 2, 2, 40>};
        const int kv = K == 512 ? 0 : K == 640 ? 1 : K == 2048 ? 2 : 3;
        return gate_up ? gu[kv] : dn[kv];
    };
    // 16-row tiles: 256 weight rows per block, or 64 (one column tile per
    // wave) for batches of up to kSmallBatch tokens, whose few tiles would
    // otherwise leave most CUs idle (K = 640 always 256).
    const int small_nt = tokens <= kSmallBatch ? kSmallBatchColumnTiles : 4;
    auto small_kernel = [small_nt](bool gate_up, int K) -> KT {
        const KT gu[4] = {k_moe_gemm_rows16<true, 8>, k_moe_gemm_stream16<true, 10>, k_moe_gemm_rows16<true, 32>,
                          k_moe_gemm_rows16<true, 40>};
        const KT dn[4] = {k_moe_gemm_rows16<false, 8>, k_moe_gemm_stream16<false, 10>, k_moe_gemm_rows16<false, 32>,
                          k_moe_gemm_rows16<false, 40>};
        const KT gu_n[4] = {k_moe_gemm_rows16<true, 8, kSmallBatchColumnTiles>, k_moe_gemm_stream16<true, 10>,
                            k_moe_gemm_rows16<true, 32, kSmallBatchColumnTiles>,
                            k_moe_gemm_rows16<true, 40, kSmallBatchColumnTiles>};
        const KT dn_n[4] = {k_moe_gemm_rows16<false, 8, kSmallBatchColumnTiles>, k_moe_gemm_stream16<false, 10>,
                            k_moe_gemm_rows16<false, 32, kSmallBatchColumnTiles>,
                            k_moe_gemm_rows16<false, 40, kSmallBatchColumnTiles>};
        const int kv = K == 512 ? 0 : K == 640 ? 1 : K == 2048 ? 2 : 3;
        if (small_nt != 4) return gate_up ? gu_n[kv] : dn_n[kv];
        return gate_up ? gu[kv] : dn[kv];
    };
    // weight rows per block of the 16-row kernel for K
    auto small_bn = [small_nt](int K) { return K == 640 ? 256 : 64 * small_nt; };

    // Other shapes: the split on the second stream, beside the router.
    const bool aux = !one_stream;  // the second stream holds work from here to the combine
    int rc = aux ? fork_aux(ctx) : SM_OK;
    // With the certified router on one stream the split rides in the router's
    // preparation launch (route_cert_prepare) instead.
    const bool cert = route_cert_applies(tokens, width, experts, topk);
    const bool split_in_prep = cert && !aux && !hilo_in_norm;
    if (rc == SM_OK && !hilo_in_norm && !split_in_prep) {
        const int64_t groups = (int64_t)tokens * (width / 64);
        k_split_hilo<<<(unsigned)((groups * 8 + 255) / 256), 256, 0, aux ? ctx->aux : ctx->stream>>>(
            (const float *)X, (_Float16 *)(ws + w.Xhl), groups);
        rc = launched(ctx);
    }
    if (rc == SM_OK && aux) rc = aux_mark(ctx);  // the hi/lo activations are ready here
    if (rc) {
        if (aux) (void)join_aux(ctx);
        return rc;
    }

    // From here on the second stream may hold work: every early return joins
    // it first, so a capture stays valid and no aux kernel outlives the call.
    auto bail = [ctx, aux](int code) {
        if (aux) (void)join_aux(ctx);
        return code;
    };
    auto wait_split = [ctx, aux]() { return aux ? wait_aux_mark(ctx) : SM_OK; };
    if (int rc2 = stage_mark(ctx, kStagePrefillRoute)) return bail(rc2);
    if (cert) {
        // The certified router: W_r's fp16 copy (with X's split in the same
        // launch, or on the second stream), then the approximate logits from
        // both.
        if (int rc2 = route_cert_prepare(ctx, (const float *)Wr, tokens, width, experts, ws + w.rcert,
                                         split_in_prep ? (const float *)X : nullptr, (_Float16 *)(ws + w.Xhl)))
            return bail(rc2);
        if (int rc2 = wait_split()) return bail(rc2);
        if (int rc2 = route_cert_launch(ctx, (const float *)X, xhl, tokens, width, (const float *)Wr,
                                        (const float *)bias, experts, topk, (int *)ids, (float *)weights,
                                        (const float *)Wsg, (float *)(ws + w.gate), ws + w.rcert))
            return bail(rc2);
    } else if (int rc2 = route_launch(ctx, (const float *)X, tokens, width, (const float *)Wr, (const float *)bias,
                                      experts, topk, (float *)(ws + w.logits), (int *)ids, (float *)weights,
                                      (const float *)Wsg, (float *)(ws + w.gate))) {
        return bail(rc2);
    }
    if (int rc2 = stage_mark(ctx, kStagePrefillDispatch)) return bail(rc2);
    int *offsets = (int *)(ws + w.offsets);
    int *tiles_small = (int *)(ws + w.tiles_small), *tiles_big = (int *)(ws + w.tiles_big);
    const int4 *info_small = (const int4 *)(ws + w.info_small), *info_big = (const int4 *)(ws + w.info_big);
    GemmTiling tiling = {tiles_small, tiles_big, split, stream ? 16 : 32, 64};
    tiling.info_small = (int *)info_small;
    tiling.info_big = (int *)info_big;
    // The dispatch also tiles the shared expert's segment (every token).
    if (int rc2 = dispatch_launch(ctx, (const int *)ids, tokens, topk, experts, offsets, (int *)(ws + w.rows),
                                  (int *)(ws + w.parts), (int *)(ws + w.where_), ws + w.dispatch, 1, &tiling))
        return bail(rc2);
    if (int rc2 = wait_split()) return bail(rc2);
    const uint64_t m = (uint64_t)tokens * topk + tokens;
    const uint64_t segs = (uint64_t)experts + 1;
    // Segment tilings: `split` or more rows in 64-row tiles ("big"), fewer in
    // 16-row tiles (streaming kernels) or one 32-row tile (k_moe_gemm).
    // (the streaming kernels' grids: tile bounds rounded up to a multiple of 8, see xcd_tile)
    auto round8 = [](uint64_t v) { return (unsigned)((v + 7) / 8 * 8); };
    const unsigned big_tiles = stream ? round8(big_tile_bound(m, experts)) : (unsigned)big_tile_bound(m, experts);
    const unsigned small_tiles = stream ? round8(small_tile_bound(m, experts, split)) : (unsigned)(segs + 1);
    const bool any_big = split <= tokens;  // otherwise no segment reaches the big tiling
    const int *rows = (const int *)(ws + w.rows);
    auto gemms = [&](bool gate_up, const _Float16 *a, const int *r, int K, int N, uint64_t codes, uint64_t scales,
                     void *out, int ld) -> int {
        if (stream) {
            // The two tilings cover disjoint rows: the big-tile grid (from
            // kOneGridTokens tokens on) runs on the second stream beside the
            // small-tile grid.
            int rc_big = SM_OK;
            if (any_big) {
                if (int rc3 = fork_aux(ctx)) return rc3;
                big_kernel(gate_up, K)<<<dim3((unsigned)(N / 256), big_tiles), 256, 0, ctx->aux>>>(
                    a, r, info_big, tiles_big, ar, blob_stride, sh, experts, codes, scales, K, N, out, ld);
                rc_big = launched(ctx);
            }
            int rc_small = SM_OK;
            if (rc_big == SM_OK) {
                small_kernel(gate_up, K)<<<dim3((unsigned)(N / small_bn(K)), small_tiles), 256, 0, ctx->stream>>>(
                    a, r, info_small, tiles_small, ar, blob_stride, sh, experts, codes, scales, K, N, out, ld);
                rc_small = launched(ctx);
            }
            const int rc_join = any_big ? join_aux(ctx) : SM_OK;
            return rc_big ? rc_big : rc_small ? rc_small : rc_join;
        }
        if (N % 512 == 0) {
            auto kb = gate_up ? k_moe_gemm<true, 2, 2, 1, 8> : k_moe_gemm<false, 2, 2, 1, 8>;
            kb<<<dim3((unsigned)(N / 512), big_tiles), 512, 0, ctx->stream>>>(a, r, info_big, tiles_big, ar, blob_stride,
                                                                             sh, experts, codes, scales, K, N, out, ld);
        } else {
            auto kb = gate_up ? k_moe_gemm<true, 1, 2, 2, 2> : k_moe_gemm<false, 1, 2, 2, 2>;
            kb<<<dim3((unsigned)(N / 128), big_tiles), 256, 0, ctx->stream>>>(a, r, info_big, tiles_big, ar, blob_stride,
                                                                             sh, experts, codes, scales, K, N, out, ld);
        }
        if (int rc3 = launched(ctx)) return rc3;
        if (N % 1024 == 0) {
            auto ks = gate_up ? k_moe_gemm<true, 1, 4, 1, 8> : k_moe_gemm<false, 1, 4, 1, 8>;
            ks<<<dim3((unsigned)(N / 1024), small_tiles), 512, 0, ctx->stream>>>(
                a, r, info_small, tiles_small, ar, blob_stride, sh, experts, codes, scales, K, N, out, ld);
        } else {
            auto ks = gate_up ? k_moe_gemm<true, 1, 1, 1, 4> : k_moe_gemm<false, 1, 1, 1, 4>;
            ks<<<dim3((unsigned)(N / 128), small_tiles), 256, 0, ctx->stream>>>(
                a, r, info_small, tiles_small, ar, blob_stride, sh, experts, codes, scales, K, N, out, ld);
        }
        return launched(ctx);
    };
    if (int rc2 = stage_mark(ctx, kStagePrefillGateUp)) return bail(rc2);
    if (int rc2 = gemms(true, xhl, rows, width, 2 * ff, L.gate_up_codes, L.gate_up_scales, ws + w.Hhl, ff)) return bail(rc2);
    if (int rc2 = stage_mark(ctx, kStagePrefillDown)) return bail(rc2);
    if (int rc2 = gemms(false, hhl, nullptr, ff, width, L.down_codes, L.down_scales, ws + w.P, width)) return bail(rc2);
    // Everything on the second stream (other shapes' split) is in before
    // the combine reads P.
    if (aux)
        if (int rc2 = join_aux(ctx)) return rc2;
    if (int rc2 = stage_mark(ctx, kStagePrefillCombine)) return rc2;
    // One thread per four output columns: every load of a thread is issued
    // at once (a 2048-wide row is two blocks).
    const dim3 combine_grid((unsigned)tokens, (unsigned)ceil_div(width / 4, 256));
    k_combine<<<combine_grid, 256, 0, ctx->stream>>>(
        (const float *)(ws + w.P), (const int *)(ws + w.where_), (const float *)weights, (const float *)(ws + w.gate),
        routed_rows, (float *)Y, tokens, topk, width, resid);
    if (int rc = launched(ctx)) return rc;
    return stage_mark(ctx, -1);
}

}  // namespace smi
