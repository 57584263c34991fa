// Certified batch router: the reference's routing (kernels/strata.cu:156-165
// router projection, :479-509 strata_router_batch) for many tokens without
// forming every logit in the reference's exact f32 order.
//
// The exact order (lane-strided sums of separately rounded products, then a
// 6-level tree; no FMA) makes the logits a VALU workload of 2 operations per
// weight and token. The expert IDs and their order only depend on which
// logits are largest, so:
//
//  1. k_route_prep_w copies W_r to fp16 (scaled by 2^8 so that its entries
//     sit in fp16's normal range) and forms the squared norms of its rows;
//     k_route_approx forms every logit approximately on fp16 MFMA (f32
//     accumulation) from that copy and the fp16 high halves of X that the
//     expert GEMMs use anyway, split over K so that small batches fill the
//     GPU.
//  2. k_route_certify, one block per token, bounds the error of every
//     approximate logit by delta (a worst-case bound from |x| |w_e|: fp16
//     rounding of both operands, subnormals flushed, the MFMA's f32
//     accumulation in any order, the reference's own rounding), takes the
//     candidates whose approximate logit lies within 2 delta + m of the K-th
//     largest, and forms their exact logits in the reference's order. Every
//     other expert's exact logit lies more than m below K of the candidates'.
//     The candidates are ranked by their exact exponentials; when adjacent
//     ones among the first K + 1 are either equal or separated by more than
//     rounding, the reference's probabilities order them the same way for any
//     value of 1 / sum, so the IDs and their order are the reference's. The
//     sum itself uses the approximate logits of the non-candidates, so the
//     routing weights agree with the reference's to a few ulp (their ratio
//     p_k / sum_k p_k barely depends on the sum).
//  3. k_route_fallback routes the tokens that failed any check (too many
//     candidates, exponentials within rounding of each other, underflow, NaN
//     or inf; about one random token in a thousand) with every logit exact
//     and the reference's selection, their 513 rows spread over 17 blocks
//     each, so that one such token costs a few microseconds, not a block
//     reading all of W_r alone.
//
// Per token, stats[t] = candidates | (1 << 16 when the token fell back).
#include <hip/hip_runtime.h>

#include <math.h>

#include <type_traits>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr float kApproxWScale = 256.0f;  // W_r scaled by 2^8 before the fp16 conversion
constexpr int kCertMaxCandidates = 64;
constexpr int kCertMaxSplits = 4;  // K splits of the approximate GEMM
constexpr int kCertMaxWidth = 2560;  // the widest router row (40 groups)
constexpr int kCertWideTokens = 1024;  // from here on, two waves per token
constexpr uint32_t kCertFallback = 1u << 16;

// Position q of a 64-wide group holds element 16 (q / 16) + (q / 2) % 8 +
// 8 (q % 2) of the group: the order of the expert GEMMs' split activations
// (moe_prefill.hip, k_split_hilo). Any order serves a dot product as long as
// both operands share it.
// Wh[e][64 g + q] = fp16(256 W_r[e][64 g + element(q)]); rn2[e] = sum of the
// row's squares. One block per row. The blocks also clear `nzero` words at
// `zero` (the fallback list's count and per-token counters) for the
// kernels after them.
// Blocks from `experts` on (when X is given) write X's fp16 hi/lo split
// instead (sm::split_hilo_chunk, 256 chunks per block): the two jobs are
// independent and share one launch.
__global__ void __launch_bounds__(256) k_route_prep_w(const float *__restrict__ Wr, _Float16 *__restrict__ Wh,
                                                      float *__restrict__ rn2, int width, int *__restrict__ zero,
                                                      int nzero, int experts, const float *__restrict__ X,
                                                      _Float16 *__restrict__ Xhl, int64_t groups) {
    __shared__ float s_part[4];
    const int e = blockIdx.x, tid = threadIdx.x;
    if (e >= experts) {
        sm::split_hilo_chunk(X, Xhl, (int64_t)(e - experts) * 256 + tid, groups);
        return;
    }
    for (int i = e * 256 + tid; i < nzero; i += experts * 256) zero[i] = 0;
    const float *row = Wr + (int64_t)e * width;
    _Float16 *out = Wh + (int64_t)e * width;
    float ss = 0.0f;
    for (int c = tid; c < width / 8; c += 256) {
        // chunk c: positions 8 (c % 8) .. + 7 of group c / 8, i.e. elements
        // 16 w + 4 h + {0, 8, 1, 9, 2, 10, 3, 11} (w = (c % 8) / 2, h = c % 2)
        const int g = c >> 3, ch = c & 7, src = 64 * g + 16 * (ch >> 1) + 4 * (ch & 1);
        const float4 a = *(const float4 *)(row + src), b = *(const float4 *)(row + src + 8);
        const float x[8] = {a.x, b.x, a.y, b.y, a.z, b.z, a.w, b.w};
        half8 h;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            h[u] = (_Float16)(x[u] * kApproxWScale);
            ss = ss + x[u] * x[u];
        }
        *(half8 *)(out + 8 * c) = h;
    }
    ss = sm::tree_sum64(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    if (tid == 0) rn2[e] = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
}

// ------------------------------------------------------------ approximate
// Block tile: 32 WM tokens x 32 (4 / WM) experts, four waves of one 32 x 32
// v_mfma_f32_32x32x16_f16 tile each; groups [ks GS, (ks + 1) GS) of K.
// P[ks][t][e] = sum over the range of fp16(x) * fp16(256 w) / 256, from the
// high halves of the split activations (Xhl: [t][group][hi, lo][64]) and Wh.
// One group per ring stage in LDS, filled by DMA (global_load_lds, 16 bytes
// per lane); three stages, so two groups are in flight while one is used. A
// row's eight 16-byte parts sit in slots part ^ ((row / 2) % 8), so the 32
// rows a half-wave reads fall on distinct banks. Each stage is an object of
// its own at namespace scope and the group loop is unrolled (GS is a
// template parameter): the compiler's waits then tell the DMA into one stage
// from the reads of another (after unrolling, every stage pointer is a
// constant). Rows past `tokens` / `experts` load clamped rows and are not
// written.
constexpr int kApproxStageRows = 160;  // the larger tile: 32 tokens + 128 experts
__shared__ __attribute__((aligned(16))) uint4 g_ap0[kApproxStageRows * 8], g_ap1[kApproxStageRows * 8],
    g_ap2[kApproxStageRows * 8];
template <int S>
__device__ __forceinline__ uint4 *approx_stage() {
    return S % 3 == 0 ? g_ap0 : S % 3 == 1 ? g_ap1 : g_ap2;
}
typedef __attribute__((address_space(3))) void lds_void_t;
// 16 bytes per lane from global memory into LDS (lane l's at base + 16 l).
__device__ __forceinline__ void approx_dma16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds_base, 16, 0, 0);
}
// Waits until at most N vector-memory operations of this wave are pending,
// then joins the block at a barrier; the memory clobbers keep LDS accesses
// on their side of it.
template <int N>
__device__ __forceinline__ void approx_sync() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int WM, int GS>
__global__ void __launch_bounds__(256) k_route_approx(const _Float16 *__restrict__ Xhl, const _Float16 *__restrict__ Wh,
                                                      float *__restrict__ P, int tokens, int width, int experts,
                                                      int xl_tiles_e, int xl_tiles_t, int xl_splits) {
    constexpr int WN = 4 / WM, TM = 32 * WM, TN = 32 * WN, ROWS = TM + TN;
    constexpr int PER = ROWS * 8 / 256;  // DMA parts per thread per group
    static_assert(ROWS * 8 % 256 == 0 && ROWS <= kApproxStageRows, "stage shape");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
    if (xl_tiles_e) {
        // One-dimensional grid in an XCD-aware order: block L runs on XCD
        // L % 8, and the xl_tiles_e expert tiles of one (token tile, split)
        // pair are consecutive blocks of one XCD, so that XCD's L2 fetches
        // the pair's activation rows once (the grid is padded to a multiple
        // of 8 pairs; blocks past the last pair return).
        const int L = blockIdx.x, slot = L >> 3;
        const int pair = (slot / xl_tiles_e) * 8 + (L & 7);
        if (pair >= xl_tiles_t * xl_splits) return;
        bx = slot % xl_tiles_e;
        by = pair % xl_tiles_t;
        bz = pair / xl_tiles_t;
    }
    const int e0 = bx * TN, t0 = by * TM, ks = bz;
    const int G = width / 64, g0 = ks * GS;

    // Part c = tid + 256 i lands in LDS slot c: row c / 8 (token rows first),
    // slot c % 8 holding part (c % 8) ^ ((row / 2) % 8).
    const _Float16 *src[PER];
    int step[PER];  // halves between consecutive groups of the row
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int c = tid + 256 * i, r = c >> 3, part = (c & 7) ^ ((r >> 1) & 7);
        if (r < TM) {
            const int64_t t = min(t0 + r, tokens - 1);
            src[i] = Xhl + ((t * G + g0) * 2) * 64 + 8 * part;
            step[i] = 128;
        } else {
            const int64_t e = min(e0 + r - TM, experts - 1);
            src[i] = Wh + (e * G + g0) * 64 + 8 * part;
            step[i] = 64;
        }
    }
    auto issue = [&](uint4 *stage, int g) {
#pragma unroll
        for (int i = 0; i < PER; i++)
            approx_dma16(src[i] + step[i] * g, &stage[256 * i + 64 * wave]);
    };
    float16v acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const int j = lane & 31, kh = lane >> 5;
    const int ar = wm * 32 + j, br = TM + wn * 32 + j;
    auto mfma4 = [&](const uint4 *stage) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // k-step k: halves 16 k + 8 kh .. + 7 = part 2 k + kh
            const int pa = (2 * k + kh) ^ ((ar >> 1) & 7), pb = (2 * k + kh) ^ ((br >> 1) & 7);
            const half8 a = __builtin_bit_cast(half8, stage[ar * 8 + pa]);
            const half8 b = __builtin_bit_cast(half8, stage[br * 8 + pb]);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc, 0, 0, 0);
        }
    };

    issue(approx_stage<0>(), 0);
    if (GS > 1) issue(approx_stage<1>(), 1);
    // Group g: wait for its parts (the parts of group g + 1 may stay in
    // flight), barrier (every wave's parts are in, and every wave is done
    // with group g - 1's stage), refill that stage with group g + 2, multiply.
#pragma unroll
    for (int g = 0; g < GS; g++) {
        if (g + 1 < GS) approx_sync<PER>();
        else approx_sync<0>();
        if (g + 2 < GS) {
            switch ((g + 2) % 3) {
            case 0: issue(approx_stage<0>(), g + 2); break;
            case 1: issue(approx_stage<1>(), g + 2); break;
            default: issue(approx_stage<2>(), g + 2); break;
            }
        }
        switch (g % 3) {
        case 0: mfma4(approx_stage<0>()); break;
        case 1: mfma4(approx_stage<1>()); break;
        default: mfma4(approx_stage<2>()); break;
        }
    }

    // acc[r] = D[i][j]: token i = 8 (r / 4) + 4 kh + r % 4, expert j.
    const int e = e0 + wn * 32 + j;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int t = t0 + wm * 32 + 8 * (r >> 2) + 4 * kh + (r & 3);
        if (t < tokens && e < experts) P[((int64_t)ks * tokens + t) * experts + e] = acc[r] * (1.0f / kApproxWScale);
    }
}

// -------------------------------------------------------------- certify
struct CertArgs {
    const float *X, *Wr, *bias, *Wsg, *P, *rn2;
    int *ids;
    float *weights, *gate_out;
    uint32_t *stats;
    // tokens left to the exact fallback: their count (zeroed by the prep
    // kernel), their indices, per listed token the row chunks done, and the
    // exact logits [listed][experts + 1] (the gate row last)
    int *fb_count, *fb_list, *fb_done;
    float *Lf;
    int tokens, width, experts, topk, ks, kspan;
};

struct CertScratch {
    float a[512];  // approximate logits (+ bias), the candidates' exact ones once formed; -FLT_MAX past `experts`
    int cand[kCertMaxCandidates + 1];
    float se[kCertMaxCandidates + 1];  // the candidates' exponentials, sorted (first topk + 1)
    int sid[kCertMaxCandidates + 1];   // their IDs, in that order
    int nc, mode;                      // candidate count; 0 certified so far, 1 fallback
};

// Exact rows of one token in the reference's order (lane l holds x[l + 64 j]:
// the lane's sequential sum of separately rounded products, then the tree):
// items [0, n) through row(i) -> (pointer, tag), put(tag, value) from lane 0.
// A wave handles items first, first + stride, ...; the next item's loads are
// in flight while the current one is summed, so a wave pays one load latency
// plus one summing chain per item. NJ = 0: a strided loop over any width.
template <int NJ, typename Row, typename Put>
__device__ __forceinline__ void exact_rows(const float (&xv)[NJ > 0 ? NJ : 1], const float *x, int width, int n,
                                           int first, int stride, Row &&row, Put &&put) {
    const int lane = threadIdx.x & 63;
    if (NJ == 0) {
        for (int i = first; i < n; i += stride) {
            int e;
            const float *w = row(i, e);
            float sum = 0.0f;
            for (int k = lane; k < width; k += 64) sum = sum + w[k] * x[k];
            put(e, sm::tree_sum64(sum));
        }
        return;
    }
    constexpr int J = NJ > 0 ? NJ : 1;
    float wa[J], wb[J];
    auto load = [&](float (&dst)[J], const float *w) {
#pragma unroll
        for (int j = 0; j < J; j++) dst[j] = w[lane + 64 * j];
    };
    auto dot = [&](const float (&w)[J]) {
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < J; j++) sum = sum + w[j] * xv[j];
        return sm::tree_sum64(sum);
    };
    int i = first, ea = 0, eb = 0;
    if (i >= n) return;
    load(wa, row(i, ea));
    while (true) {
        // wa holds item i; item i + stride goes to wb while wa is summed
        const int i1 = i + stride;
        if (i1 < n) load(wb, row(i1, eb));
        put(ea, dot(wa));
        if (i1 >= n) return;
        const int i2 = i1 + stride;
        if (i2 < n) load(wa, row(i2, ea));
        put(eb, dot(wb));
        if (i2 >= n) return;
        i = i2;
    }
}

// Upper bound of the approximate logits' error for a token: |x| = nx,
// sum |x| <= sx1, max_e |w_e| <= rnorm, sum_i |w_ei| <= sqrt(width) rnorm.
__device__ __forceinline__ float cert_delta(float nx, float sx1, float rnorm, float amax, float bmax, int width,
                                            int kspan, int ks) {
    const float S = nx * rnorm;                     // >= sum_i |x_i w_ei| (Cauchy-Schwarz)
    const float W1 = sqrtf((float)width) * rnorm;  // >= sum_i |w_ei|
    // fp16 rounding of x and 256 w (|h(v) - v| <= 2^-11 |v| + 2^-14 with
    // subnormals flushed), scaled back by 2^-8
    const float conv = 0.0009775f * S + 6.104e-5f * W1 + 2.385e-7f * sx1 + (float)width * 1.5e-11f;
    // f32 accumulation in any order: a chain of kspan products per split,
    // ks - 1 partial sums and the bias add (2^-23 per addition, truncation
    // included) over the magnitude of the products
    const float chain = (float)(kspan + ks + 2) * 1.1921e-7f * (1.01f * S + 1.2e-4f * W1 + 4.8e-7f * sx1);
    // the reference's own rounding (one product, 32 sums and 6 tree levels
    // per term) and its bias add; the sum of the split partials and bias
    const float ref = 48.0f * 5.97e-8f * S + (float)(ks + 2) * 1.1921e-7f * (1.01f * S + bmax + amax);
    return 1.01f * (conv + chain + ref) + 1e-30f;
}

// Timeline hook, compiled in only with -DSM_CERT_TRACE (profiling builds):
// lane 0 of the calling wave records the real-time clock (100 MHz) at mark k
// of its token in LDS; the block copies its marks out when it ends.
#ifdef SM_CERT_TRACE
__device__ uint64_t g_cert_trace[4096 * 16];
#define CERT_MARK(k) \
    do { if ((threadIdx.x & 63) == 0) s_marks[k] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define CERT_MARK_LOADED(k) \
    do { __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8)); CERT_MARK(k); } while (0)
#define CERT_FLUSH() \
    do { __syncthreads(); if (threadIdx.x < 16 && blockIdx.x < 4096) g_cert_trace[blockIdx.x * 16 + threadIdx.x] = s_marks[threadIdx.x]; } while (0)
#else
#define CERT_MARK(k) do { } while (0)
#define CERT_MARK_LOADED(k) do { } while (0)
#define CERT_FLUSH() do { } while (0)
#endif

// Lists token t for the exact fallback (k_route_fallback).
__device__ __forceinline__ void enqueue_fallback(const CertArgs &a, int t, int nc) {
    if ((threadIdx.x & 63) == 0) {
        const int f = atomicAdd(a.fb_count, 1);
        a.fb_list[f] = t;
        a.stats[t] = (uint32_t)nc | kCertFallback;
    }
}

// One block of WPT waves per token: 4 for batches whose blocks all fit on
// the GPU at once, 2 for large ones (2048 tokens then run in one round
// instead of two).
template <int NJ, int WPT>
__global__ void __launch_bounds__(64 * WPT) __attribute__((amdgpu_waves_per_eu(WPT == 2 && NJ <= 32 ? 4 : 2)))
k_route_certify(CertArgs a) {
    constexpr int NT = 64 * WPT;
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    __shared__ CertScratch s;
    __shared__ int s_ids[32];
    __shared__ __attribute__((aligned(16))) float s_x[kCertMaxWidth];
    __shared__ float s_norm[2 * WPT];
#ifdef SM_CERT_TRACE
    __shared__ uint64_t s_marks[16];
    if (threadIdx.x < 16) s_marks[threadIdx.x] = 0;
#endif
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t = blockIdx.x, E = a.experts, K = a.topk;
    if (wave == 0) CERT_MARK(0);
    const float *x = a.X + (int64_t)t * a.width;
    // Wave 0's loads of the approximate logits first (every split's partial
    // before any sum; one uniform branch on the split count, straight-line
    // loads inside it; the bias row, or any row when there is none, loaded
    // unconditionally), then the token's x row by every thread in 16-byte
    // loads (clamped, so that one wait covers them all), into LDS once for
    // the block (each wave reading it from memory would be WPT times the
    // traffic of the launch's first burst). The x norms are formed from the
    // same registers, every thread over its own elements. The exponential
    // table is written while the loads are in flight.
    float qp[8][kCertMaxSplits], r2v[8], bv[8];
    if (wave == 0) {
        const float *brow = a.bias ? a.bias : a.rn2;
        auto load = [&](auto nsplit) {
            constexpr int NS = decltype(nsplit)::value;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int e = min(lane + 64 * j, E - 1);
#pragma unroll
                for (int k = 0; k < NS; k++) qp[j][k] = a.P[((int64_t)k * a.tokens + t) * E + e];
#pragma unroll
                for (int k = NS; k < kCertMaxSplits; k++) qp[j][k] = 0.0f;
                r2v[j] = a.rn2[e];
                bv[j] = brow[e];
            }
        };
        if (a.ks == 1) load(std::integral_constant<int, 1>());
        else if (a.ks == 2) load(std::integral_constant<int, 2>());
        else if (a.ks == 3) load(std::integral_constant<int, 3>());
        else load(std::integral_constant<int, kCertMaxSplits>());
    }
#ifdef SM_CERT_TRACE
    if (wave == 0) CERT_MARK(12);
#endif
    constexpr int XV = (kCertMaxWidth / 4 + NT - 1) / NT;
    const int nx4 = a.width / 4;
    float4 xr[XV];
#pragma unroll
    for (int u = 0; u < XV; u++) xr[u] = ((const float4 *)x)[min(tid + NT * u, nx4 - 1)];
    sm::fill_exp_table(s_tab);
    {
        float ss = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int u = 0; u < XV; u++) {
            if (tid + NT * u < nx4) {
                const float4 v = xr[u];
                ss = ss + (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
                s1 = s1 + (fabsf(v.x) + fabsf(v.y)) + (fabsf(v.z) + fabsf(v.w));
                ((float4 *)s_x)[tid + NT * u] = v;
            }
        }
        ss = sm::tree_sum64(ss);
        s1 = sm::tree_sum64(s1);
        if (lane == 0) {
            s_norm[wave] = ss;
            s_norm[WPT + wave] = s1;
        }
    }
#ifdef SM_CERT_TRACE
    if (wave == 0) CERT_MARK_LOADED(13);
#endif
    __syncthreads();
    if (wave == 0) CERT_MARK(14);
    float xv[NJ > 0 ? NJ : 1];
    if (NJ > 0) {
#pragma unroll
        for (int j = 0; j < NJ; j++) xv[j] = s_x[lane + 64 * j];
    }

    // ---- wave 0: approximate logits, bound, threshold, candidates
    if (wave == 0) {
        float av[8], rn = 0.0f, amax = 0.0f, bmax = 0.0f;
        bool finite = true;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int e = lane + 64 * j;
            float v = -3.402823e38f;
            if (e < E) {
                const float b = a.bias ? bv[j] : 0.0f;
                float p = qp[j][0];
#pragma unroll
                for (int k = 1; k < kCertMaxSplits; k++)
                    if (k < a.ks) p = p + qp[j][k];
                v = a.bias ? p + b : p;
                finite = finite && isfinite(v) && isfinite(r2v[j]);
                rn = fmaxf(rn, r2v[j]);
                amax = fmaxf(amax, fabsf(v));
                bmax = fmaxf(bmax, fabsf(b));
            }
            av[j] = v;
            s.a[e] = v;
        }
        CERT_MARK_LOADED(1);
        float ss = s_norm[0], s1 = s_norm[WPT];
#pragma unroll
        for (int w = 1; w < WPT; w++) {
            ss = ss + s_norm[w];
            s1 = s1 + s_norm[WPT + w];
        }
        // sums in any order: the factors 1.002 below cover their rounding
        // (widths <= 2^13)
        rn = sm::wave_max(rn);
        amax = sm::wave_max(amax);
        bmax = sm::wave_max(bmax);
        const float nx = sqrtf(ss) * 1.002f, sx1 = s1 * 1.002f, rnorm = sqrtf(rn) * 1.002f;
        const float delta = cert_delta(nx, sx1, rnorm, amax, bmax, a.width, a.kspan, a.ks);
        finite = __ballot(!finite) == 0 && isfinite(delta) && isfinite(nx) && isfinite(sx1);
        int mode = finite ? 0 : 1, nc = 0;
        if (!mode) {
            // tau = the K-th largest approximate logit (lower ID first on ties)
            uint32_t kk[8], hk = 0;
            uint64_t Q[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                kk[j] = lane + 64 * j < E ? sm::logit_key(av[j]) : 0u;
                hk = max(hk, kk[j]);
                Q[j] = ((uint64_t)kk[j] << 9) | (uint64_t)(511 - (lane + 64 * j));
            }
            const uint32_t T = sm::logit_threshold(hk, K);
            bool in[8];
#pragma unroll
            for (int j = 0; j < 8; j++) in[j] = kk[j] != 0u && kk[j] >= T;
            if (T == 0u || !sm::rank_candidates(Q, in, K, s_router, s_ids, false)) mode = 1;
            sm::wave_lds_sync();  // s_ids written by other lanes
            if (!mode) {
                const float tau = s.a[s_ids[K - 1]];
                const float m = 2.44140625e-4f + 9.5367431640625e-7f * fabsf(tau);  // 2^-12 + 2^-20 |tau|
                const float lo = tau - 2.0f * delta - m;
                bool c[8];
                int cnt = 0, pos[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    c[j] = lane + 64 * j < E && av[j] >= lo;
                    pos[j] = cnt;
                    cnt += c[j] ? 1 : 0;
                }
                const int incl = sm::wave_scan_incl(cnt);
                nc = __builtin_amdgcn_readlane(incl, 63);
                if (nc > kCertMaxCandidates || nc < K) {
                    mode = 1;
                } else {
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        if (c[j]) s.cand[incl - cnt + pos[j]] = lane + 64 * j;
                }
            }
        }
        if (lane == 0) {
            s.nc = nc;
            s.mode = mode;
        }
        if (mode) enqueue_fallback(a, t, nc);
        CERT_MARK(2);
    }
    __syncthreads();
    if (s.mode) {
        CERT_FLUSH();
        return;
    }
    if (wave == 0) CERT_MARK(3);

    // ---- exact logits of the candidates (in place of their approximate
    // ones) and of the shared-expert gate row, all waves
    const int nc = s.nc;
    auto cand_row = [&](int i, int &e) -> const float * {
        if (i >= nc) {
            e = -1;
            return a.Wsg;
        }
        e = s.cand[i];
        return a.Wr + (int64_t)e * a.width;
    };
    auto cand_put = [&](int e, float v) {
        if (lane != 0) return;
        if (e < 0) a.gate_out[t] = v;
        else s.a[e] = a.bias ? v + a.bias[e] : v;
    };
    exact_rows<NJ>(xv, s_x, a.width, nc + (a.Wsg ? 1 : 0), wave, WPT, cand_row, cand_put);
    CERT_MARK(4 + wave);
    __syncthreads();
    if (wave == 0) CERT_MARK(8);

    // ---- every expert's exponential (exact logit for the candidates,
    // approximate for the rest: only the sum uses those), 512 / NT per
    // thread. The maximum over the candidates is the maximum of all exact
    // logits (the largest exact logit's expert is always a candidate).
    const bool mine = lane < nc;
    const int id = mine ? s.cand[lane] : 0;
    const float lc = mine ? s.a[id] : -3.402823e38f;
    const bool finite = __ballot(mine && !isfinite(lc)) == 0;
    const float mx = sm::wave_max(lc);
    {
        constexpr int PT = 512 / NT;
        float d[PT], ex[PT];
#pragma unroll
        for (int u = 0; u < PT; u++) d[u] = s.a[tid + NT * u] - mx;
        sm::wave_lds_sync();  // this wave's copy of the exp table is in LDS
        sm::expf_or_n<PT>(d, ex, s_tab);
#pragma unroll
        for (int u = 0; u < PT; u++) s_router.p[tid + NT * u] = tid + NT * u < E ? ex[u] : 0.0f;
    }
    if (wave == 0) CERT_MARK(9);
    __syncthreads();
#ifdef SM_CERT_TRACE
    if (wave == 0) CERT_MARK(10);
    const bool w0 = wave == 0;
    if (!w0) {
        __syncthreads();  // CERT_FLUSH's barrier, matched below
        if (threadIdx.x < 16 && blockIdx.x < 4096) g_cert_trace[blockIdx.x * 16 + threadIdx.x] = s_marks[threadIdx.x];
        return;
    }
#else
    if (wave != 0) return;
#endif

    // ---- wave 0: the reference's sum, the candidates ranked by (exp desc,
    // ID asc), certification, routing
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) sum = sum + s_router.p[lane + 64 * j];
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sm::tree_sum64(sum))));
    const float inv = 1.0f / sum;
    bool ok = finite && isfinite(sum) && sum > 0.0f && isfinite(inv);
    const float ec = mine ? s_router.p[id] : 0.0f;
    const uint64_t q = mine ? (((uint64_t)__builtin_bit_cast(uint32_t, ec) << 9) | (uint64_t)(511 - id)) : 0ull;
    const uint32_t qlo = (uint32_t)q, qhi = (uint32_t)(q >> 32);
    int rank = 0;
    for (int c = 0; c < nc; c++) {
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)qhi, c);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)qlo, c);
        rank += (hi > qhi || (hi == qhi && lo > qlo)) ? 1 : 0;
    }
    if (mine && rank <= K) {
        s.se[rank] = ec;
        s.sid[rank] = id;
    }
    sm::wave_lds_sync();
    // Adjacent pairs among the first min(K + 1, nc): equal, or apart by more
    // than 2^-21 relative. Then e_i / e_{i+1} > 1 + 2^-21, so
    // fl(e_i r) >= e_i r (1 - 2^-24) > e_{i+1} r (1 + 2^-24) >= fl(e_{i+1} r)
    // for any r = 1 / sum: p keeps their order. The difference is exact
    // (Sterbenz) when it matters, and the scaling by 2^-21 is exact. The K-th
    // must be clear of underflow.
    const int pairs = min(K, nc - 1);
    bool sep = true;
    if (lane < pairs) {
        const float hi = s.se[lane], lo2 = s.se[lane + 1];
        sep = hi == lo2 || hi - lo2 > hi * 4.76837158203125e-7f;
    }
    ok = ok && __ballot(!sep) == 0 && s.se[K - 1] >= 8.077935669463161e-28f;  // 2^-90
    if (!ok) {
        enqueue_fallback(a, t, nc);
    } else {
        const float pk = lane < K ? s.se[lane] * inv : 0.0f;
        if (lane < K) a.ids[(int64_t)t * K + lane] = s.sid[lane];
        sm::router_weights(pk, K, a.weights + (int64_t)t * K);
        if (lane == 0) a.stats[t] = (uint32_t)nc;
    }
#ifdef SM_CERT_TRACE
    CERT_MARK(11);
    __syncthreads();  // with the other waves' barrier above
    if (threadIdx.x < 16 && blockIdx.x < 4096) g_cert_trace[blockIdx.x * 16 + threadIdx.x] = s_marks[threadIdx.x];
#endif
}

// ------------------------------------------------------------- fallback
// Exact routing of the tokens the certification left: block (c, s) forms row
// chunk c (rows 32 c .. 32 c + 31 of the experts' rows and the gate row
// after them) for listed tokens s, s + gridDim.y, ...; the block that
// completes a token's last chunk (a device-scope counter per listed token,
// with release / acquire fences around it) runs the reference's selection
// on its exact logits. With nothing listed every block returns at once.
constexpr int kFallbackRows = 32, kFallbackSlots = 16;
template <int NJ>
__global__ void __launch_bounds__(256) k_route_fallback(CertArgs a) {
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    __shared__ int s_ids[32];
    __shared__ int s_last;
    const int count = *a.fb_count;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = a.experts, K = a.topk, rows = E + (a.Wsg ? 1 : 0);
    const int chunks = (rows + kFallbackRows - 1) / kFallbackRows, r0 = blockIdx.x * kFallbackRows;
    if (count == 0) return;
    sm::fill_exp_table(s_tab);
    for (int f = blockIdx.y; f < count; f += gridDim.y) {
        const int t = a.fb_list[f];
        const float *x = a.X + (int64_t)t * a.width;
        float *L = a.Lf + (int64_t)f * (E + 1);
        float xv[NJ > 0 ? NJ : 1];
        if (NJ > 0) {
#pragma unroll
            for (int j = 0; j < NJ; j++) xv[j] = x[lane + 64 * j];
        }
        const int n = min(kFallbackRows, rows - r0);
        exact_rows<NJ>(
            xv, x, a.width, n, wave, 4,
            [&](int i, int &e) -> const float * {
                e = r0 + i;
                return e < E ? a.Wr + (int64_t)e * a.width : a.Wsg;
            },
            [&](int e, float v) {
                if (lane == 0) L[e] = e < E && a.bias ? v + a.bias[e] : v;
            });
        __threadfence();  // this block's rows before its count
        __syncthreads();
        if (tid == 0) s_last = atomicAdd(a.fb_done + f, 1) == chunks - 1;
        __syncthreads();
        if (s_last) {
            __threadfence();  // every other chunk's rows after the count
            float l[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                l[j] = lane + 64 * j < E ? __hip_atomic_load(L + lane + 64 * j, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)
                                         : -3.402823e38f;
            sm::router_block(l, E, K, s_tab, s_router, s_ids);  // waves 1-3 skip the selection
            if (wave == 0) {
                if (lane < K) a.ids[(int64_t)t * K + lane] = s_ids[lane];
                sm::router_weights(lane < K ? s_router.val[lane] : 0.0f, K, a.weights + (int64_t)t * K);
                if (lane == 0 && a.Wsg)
                    a.gate_out[t] = __hip_atomic_load(L + E, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();  // s_last and the scratch before the next token
    }
}

// Splits of K and tile shapes: at least 512 blocks where the splits allow
// (two per CU), each split a group span the kernel is built for.
struct CertPlan {
    int wm, ks, gspan, tiles_e, tiles_t;
};
bool approx_span_built(int gs) { return gs == 8 || gs == 16 || gs == 10 || gs == 20; }
static_assert(kCertMaxWidth >= 64 * 40, "the widest built width");
CertPlan cert_plan(int tokens, int width, int experts) {
    CertPlan p;
    p.wm = tokens >= 1024 ? 2 : 1;
    const int tm = 32 * p.wm, tn = 128 / p.wm, G = width / 64;
    p.tiles_t = (tokens + tm - 1) / tm;
    p.tiles_e = (experts + tn - 1) / tn;
    const int blocks = p.tiles_t * p.tiles_e;
    p.ks = 0;
    for (int ks = 1; ks <= kCertMaxSplits; ks++) {
        if (G % ks || !approx_span_built(G / ks)) continue;
        p.ks = ks;
        if (blocks * ks >= 512) break;
    }
    p.gspan = p.ks ? G / p.ks : 0;
    return p;
}

constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct CertWs {
    uint64_t P, Wh, rn2, stats, fb, fb_list, Lf, end;  // fb: the count, then one counter per token
};
CertWs cert_ws(int tokens, int width, int experts) {
    const CertPlan p = cert_plan(tokens, width, experts);
    CertWs w;
    w.P = 0;
    w.Wh = up(w.P + (uint64_t)p.ks * tokens * experts * 4);
    w.rn2 = up(w.Wh + (uint64_t)experts * width * 2);
    w.stats = up(w.rn2 + (uint64_t)experts * 4);
    w.fb = up(w.stats + (uint64_t)tokens * 4);
    w.fb_list = up(w.fb + ((uint64_t)tokens + 1) * 4);
    w.Lf = up(w.fb_list + (uint64_t)tokens * 4);
    w.end = up(w.Lf + (uint64_t)tokens * (experts + 1) * 4);
    return w;
}

}  // namespace

namespace smi {

bool route_cert_applies(int tokens, int width, int experts, int topk) {
    return tokens >= kRouteCertMinTokens && width % 64 == 0 && width <= kCertMaxWidth &&
           cert_plan(tokens, width, experts).ks > 0 && experts <= 512 && topk <= 32;
}

uint64_t route_cert_workspace(int tokens, int width, int experts) { return cert_ws(tokens, width, experts).end; }

uint64_t route_cert_stats_offset(int tokens, int width, int experts) {
    return cert_ws(tokens, width, experts).stats;
}

int route_cert_prepare(sm_ctx *ctx, const float *Wr, int tokens, int width, int experts, char *ws, const float *X,
                       _Float16 *Xhl) {
    const CertWs w = cert_ws(tokens, width, experts);
    const int64_t groups = X ? (int64_t)tokens * (width / 64) : 0;
    const unsigned split_blocks = (unsigned)((groups * 8 + 255) / 256);
    k_route_prep_w<<<(unsigned)experts + split_blocks, 256, 0, ctx->stream>>>(
        Wr, (_Float16 *)(ws + w.Wh), (float *)(ws + w.rn2), width, (int *)(ws + w.fb), tokens + 1, experts, X, Xhl,
        groups);
    return launched(ctx);
}

int route_cert_launch(sm_ctx *ctx, const float *X, const _Float16 *Xhl, int tokens, int width, const float *Wr,
                      const float *bias, int experts, int topk, int *ids, float *weights, const float *gate_w,
                      float *gate_out, char *ws) {
    const CertPlan p = cert_plan(tokens, width, experts);
    const CertWs w = cert_ws(tokens, width, experts);
    float *P = (float *)(ws + w.P), *rn2 = (float *)(ws + w.rn2);
    const _Float16 *Wh = (const _Float16 *)(ws + w.Wh);
    // From 1,024 tokens on the activation rows outweigh W_r's copy: the
    // XCD-aware order keeps each token tile on one XCD (8 x W_r's 2 MiB
    // copy fetched into the eight L2s, instead of every token tile into up
    // to eight).
    const bool xlocal = p.wm == 2;
    const int pairs = p.tiles_t * p.ks, padded = (pairs + 7) / 8 * 8;
    const dim3 g1 = xlocal ? dim3((unsigned)(padded * p.tiles_e))
                           : dim3((unsigned)p.tiles_e, (unsigned)p.tiles_t, (unsigned)p.ks);
    using KA = void (*)(const _Float16 *, const _Float16 *, float *, int, int, int, int, int, int);
    const int gi = p.gspan == 8 ? 0 : p.gspan == 16 ? 1 : p.gspan == 10 ? 2 : 3;
    static const KA by_span[2][4] = {
        {k_route_approx<1, 8>, k_route_approx<1, 16>, k_route_approx<1, 10>, k_route_approx<1, 20>},
        {k_route_approx<2, 8>, k_route_approx<2, 16>, k_route_approx<2, 10>, k_route_approx<2, 20>}};
    by_span[p.wm - 1][gi]<<<g1, 256, 0, ctx->stream>>>(Xhl, Wh, P, tokens, width, experts, xlocal ? p.tiles_e : 0,
                                                       p.tiles_t, p.ks);
    if (int rc = launched(ctx)) return rc;
    CertArgs a;
    a.X = X;
    a.Wr = Wr;
    a.bias = bias;
    a.Wsg = gate_w;
    a.P = P;
    a.rn2 = rn2;
    a.ids = ids;
    a.weights = weights;
    a.gate_out = gate_out;
    a.stats = (uint32_t *)(ws + w.stats);
    a.tokens = tokens;
    a.width = width;
    a.experts = experts;
    a.topk = topk;
    a.ks = p.ks;
    a.kspan = p.gspan * 64;
    a.fb_count = (int *)(ws + w.fb);
    a.fb_done = a.fb_count + 1;
    a.fb_list = (int *)(ws + w.fb_list);
    a.Lf = (float *)(ws + w.Lf);
    const int nj = width == 2048 ? 32 : width == 2560 ? 40 : 0;
    using KC = void (*)(CertArgs);
    // 2 waves per token from kCertWideTokens tokens on (all blocks resident
    // at once), 4 below
    const int wi = tokens >= kCertWideTokens ? 1 : 0;
    static const KC by_width[3][2] = {{k_route_certify<32, 4>, k_route_certify<32, 2>},
                                      {k_route_certify<40, 4>, k_route_certify<40, 2>},
                                      {k_route_certify<0, 4>, k_route_certify<0, 2>}};
    by_width[nj == 32 ? 0 : nj == 40 ? 1 : 2][wi]<<<(unsigned)tokens, wi ? 128 : 256, 0, ctx->stream>>>(a);
    if (int rc = launched(ctx)) return rc;
    const dim3 g3((unsigned)ceil_div(experts + (gate_w ? 1 : 0), kFallbackRows), (unsigned)kFallbackSlots);
    if (nj == 32)
        k_route_fallback<32><<<g3, 256, 0, ctx->stream>>>(a);
    else if (nj == 40)
        k_route_fallback<40><<<g3, 256, 0, ctx->stream>>>(a);
    else
        k_route_fallback<0><<<g3, 256, 0, ctx->stream>>>(a);
    return launched(ctx);
}

}  // namespace smi

#ifdef SM_CERT_TRACE
extern "C" int sm_cert_trace_read(uint64_t *out, int n) {
    if (n < 4096 * 16) return SM_E_ARG;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_cert_trace), sizeof(uint64_t) * 4096 * 16) == hipSuccess ? SM_OK
                                                                                                            : SM_E_HIP;
}
#endif
