// Router logits, softmax top-k and expert-contiguous dispatch on the device.
//
// Router logits follow the reference's f32 operation order exactly
// (kernels/strata.cu:156-165: lane l sums columns l, l+64, ... in order, then
// the tree s = 32..1), so selected expert IDs and their order are bit-exact
// with the reference's CPU path; the top-k is router_wave (strata.cu:240-270).
//
//  * tokens == 1: one wave per router row (all of a lane's loads issued
//    before its sequential sum), then a one-wave top-k kernel. The kernel
//    boundary orders the two; a per-block completion counter with device-
//    scope fences measured an order of magnitude slower on MI355X.
//  * tokens > 1: register-tiled exact GEMM. Each wave owns 8 tokens x 8 rows
//    and keeps, per lane l, the 64 partial sums of "lane l" of the reference
//    workgroup for all 64 outputs. A transpose (butterfly) reduction then
//    forms the reference tree for every output: at level s each lane keeps
//    half of its outputs and adds its partner's (lane ^ s) copy, which yields
//    exactly partial[l] + partial[l+s] of the reference (f32 addition is
//    commutative), and after six levels lane l holds output l.
//
// Dispatch (replacing the host grouping of src/prefill.js:56-61): per block of
// 64 tokens a 64-bit token mask per expert, an exclusive scan over
// (expert, block) in expert-major order, and the rank of a token inside its
// expert = base + popcount of the lower mask bits. Integer-only, so the
// permutation (experts ascending, tokens ascending within an expert) is
// deterministic.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

// ---------------------------------------------------- route, few tokens
// One 64-thread block per (row, token): rows [0, experts) are router rows,
// row `experts` is the shared-expert gate (when gate_w != 0); blocks past the
// last row (grid.x is padded to a multiple of 8, so a row's blocks run on one
// XCD for every token) return. NJ = width / 64 loads per lane, all issued
// before the (sequential, reference-order) sum.
template <int NJ>
__global__ void __launch_bounds__(64) k_route_rows(const float *__restrict__ X, const float *__restrict__ Wr,
                                                   const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                   float *__restrict__ logits, float *__restrict__ gate_out, int width,
                                                   int experts, int rows) {
    const int row = blockIdx.x, lane = threadIdx.x, t = blockIdx.y;
    if (row >= rows) return;
    X += (int64_t)t * width;
    logits += (int64_t)t * experts;
    gate_out += t;
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

// -------------------------------------------------------- T > 1 route GEMM
// Tiles of TT tokens x TR rows per wave: 8 x 8 for large batches, 4 x 4 (four
// times the waves) for small ones.
constexpr int kRouteSmallTileMaxTokens = 128;

// One level of the reference's tree (lanes l and l ^ D added) over the N
// outputs each lane still holds; lanes with bit D set keep the upper half.
template <int N, int D>
__device__ __forceinline__ void butterfly_level(float *a, int lane) {
    constexpr int H = N / 2;
    const bool upper = (lane & D) != 0;
#pragma unroll
    for (int i = 0; i < H; i++) {
        float send = upper ? a[i] : a[i + H];
        float keep = upper ? a[i + H] : a[i];
        a[i] = keep + __shfl_xor(send, D, 64);
    }
}

// Grid: x = groups of four row tiles (ceil((experts+1)/TR) tiles), y = token
// tiles (ceil(T/TT)). Row `experts` is the shared-expert gate. Rows/tokens
// past the end are computed on clamped (valid) addresses and discarded.
template <int TT, int TR>
__global__ void __launch_bounds__(256) k_route_gemm(const float *__restrict__ X, const float *__restrict__ Wr,
                                                    const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                    float *__restrict__ logits, float *__restrict__ gate_out,
                                                    int tokens, int width, int experts, int with_gate) {
    constexpr int NO = TT * TR;  // outputs per wave
    static_assert(NO == 64 || NO == 16, "64 or 16 outputs per wave");
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nrows = experts + (with_gate ? 1 : 0);
    const int row_tiles = (nrows + TR - 1) / TR;
    const int tile = blockIdx.x * 4 + wave;
    if (tile >= row_tiles) return;
    const int r0 = tile * TR, t0 = blockIdx.y * TT;
    // Row and token bases are the same for the whole wave (scalar registers);
    // lanes differ only by a 32-bit byte offset.
    const char *wp[TR];
    const char *xp[TT];
#pragma unroll
    for (int r = 0; r < TR; r++) {
        int row = min(r0 + r, nrows - 1);
        wp[r] = (const char *)(row < experts ? Wr + (int64_t)row * width : Wsg);
    }
#pragma unroll
    for (int t = 0; t < TT; t++) xp[t] = (const char *)(X + (int64_t)min(t0 + t, tokens - 1) * width);
    float a[NO];
#pragma unroll
    for (int o = 0; o < NO; o++) a[o] = 0.0f;
    float xv[TT], wv[TR];
    auto load = [&](uint32_t off, float *xd, float *wd) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; t++) xd[t] = *(const float *)(xp[t] + off);
#pragma unroll
        for (int r = 0; r < TR; r++) wd[r] = *(const float *)(wp[r] + off);
    };
    auto madd = [&](const float *xs, const float *ws) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < TR; r++) a[t * TR + r] = a[t * TR + r] + ws[r] * xs[t];
    };
    constexpr int PD = 8;  // positions in flight for the 4 x 4 tiles
    if (NO == 16 && width % (64 * PD) == 0) {
        // Few products per position: PD positions' values are in flight while
        // one is used (a ring of PD buffers, refilled as each is consumed;
        // loads past the end repeat the last position and are not used).
        const int steps = width / 64;
        const uint32_t first = (uint32_t)lane * 4u, last = first + (uint32_t)(steps - 1) * 256u;
        float xb[PD][TT], wb[PD][TR];
#pragma unroll
        for (int p = 0; p < PD; p++) load(first + (uint32_t)p * 256u, xb[p], wb[p]);
        for (int k = 0; k < steps; k += PD) {
#pragma unroll
            for (int p = 0; p < PD; p++) {
                madd(xb[p], wb[p]);
                load(min(first + (uint32_t)(k + p + PD) * 256u, last), xb[p], wb[p]);
            }
        }
    } else if (width % 64 == 0) {
        // Each lane sums its positions lane, lane + 64, ... in order; the next
        // position's values are loaded while the current ones are used. The
        // loads are unconditional (past the end they repeat the last
        // position), so the compiler's waits only cover the buffer in use.
        const int steps = width / 64;
        const uint32_t first = (uint32_t)lane * 4u, last = first + (uint32_t)(steps - 1) * 256u;
        uint32_t off = first;
        float xn[TT], wn[TR];
        load(off, xv, wv);
        for (int k = 0;; k += 2, off += 512u) {
            load(min(off + 256u, last), xn, wn);
            madd(xv, wv);
            if (k + 1 >= steps) break;
            load(min(off + 512u, last), xv, wv);
            madd(xn, wn);
            if (k + 2 >= steps) break;
        }
    } else {
        for (int i = lane; i < width; i += 64) {
            load((uint32_t)i * 4u, xv, wv);
            madd(xv, wv);
        }
    }
    // The reference's tree pairs lanes at distances 32, 16, 8, 4, 2, 1.
    int o;
    if (NO == 64) {
        butterfly_level<64, 32>(a, lane);
        butterfly_level<32, 16>(a, lane);
        butterfly_level<16, 8>(a, lane);
        butterfly_level<8, 4>(a, lane);
        butterfly_level<4, 2>(a, lane);
        butterfly_level<2, 1>(a, lane);
        o = lane;  // lane l holds output l
    } else {
        butterfly_level<16, 32>(a, lane);
        butterfly_level<8, 16>(a, lane);
        butterfly_level<4, 8>(a, lane);
        butterfly_level<2, 4>(a, lane);
        // lanes 4o .. 4o + 3 hold parts of output o: the last two levels
        a[0] = a[0] + __shfl_xor(a[0], 2, 64);
        a[0] = a[0] + __shfl_xor(a[0], 1, 64);
        o = (lane & 3) == 0 ? lane >> 2 : NO;  // one writer per output
    }
    const int t = t0 + o / TR, row = r0 + o % TR;
    if (o < NO && t < tokens && row < nrows) {
        if (row < experts) logits[(int64_t)t * experts + row] = bias ? a[0] + bias[row] : a[0];
        else gate_out[t] = a[0];
    }
}

// Top-k of every token's logits (kernels/strata.cu:479-509 strata_router_batch
// results): one 256-thread block per token (router_block: the exponentials
// over four waves, the ranked selection in wave 0). Needs experts <= 512.
__global__ void __launch_bounds__(256) k_topk(const float *__restrict__ logits, int *__restrict__ ids,
                                              float *__restrict__ weights, int experts, int topk) {
    __shared__ uint64_t s_tab[32];
    __shared__ sm::RouterScratch s_router;
    __shared__ int s_ids[32];
    const int t = blockIdx.x;
    float lg[8];
    sm::router_load(logits + (int64_t)t * experts, experts, lg);
    sm::fill_exp_table(s_tab);
    sm::router_block(lg, experts, topk, s_tab, s_router, s_ids);  // waves 1-3 return inside
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    if (lane < topk) ids[(int64_t)t * topk + lane] = s_ids[lane];
    sm::router_weights(lane < topk ? s_router.val[lane] : 0.0f, topk, weights + (int64_t)t * topk);
}

// ---------------------------------------------------------------- dispatch
// Block b covers tokens [64b, 64b+64). masks[b*E + e] = tokens of the block
// routed to e; counts[b*E + e] = popcount; flags[b] bit 0: an ID outside
// [0, experts) (left out, marked by k_dispatch_place), bit 1: an ID repeated
// within one token. k_dispatch_scan folds the flags into the status word.
__global__ void __launch_bounds__(256) k_dispatch_masks(const int *__restrict__ ids, int tokens, int topk, int experts,
                                                        int nb, unsigned long long *__restrict__ masks,
                                                        int *__restrict__ counts, uint32_t *__restrict__ flags) {
    __shared__ unsigned long long m[512];
    __shared__ uint32_t s_flags;
    const int b = blockIdx.x;
    for (int e = threadIdx.x; e < experts; e += blockDim.x) m[e] = 0ull;
    if (threadIdx.x == 0) s_flags = 0;
    __syncthreads();
    const int t0 = b * 64, nt = min(64, tokens - t0);
    for (int a = threadIdx.x; a < nt * topk; a += blockDim.x) {
        int tl = a / topk, e = ids[(int64_t)(t0 + tl) * topk + a % topk];
        if (e < 0 || e >= experts) {
            atomicOr(&s_flags, 1u);
            continue;
        }
        const unsigned long long bit = 1ull << tl;
        if (atomicOr(&m[e], bit) & bit) atomicOr(&s_flags, 2u);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < experts; e += blockDim.x) {
        masks[(int64_t)b * experts + e] = m[e];
        counts[(int64_t)b * experts + e] = __popcll(m[e]);
    }
    if (threadIdx.x == 0) flags[b] = s_flags;
}

// Inclusive prefix sum over one block of SCAN_THREADS threads (wave scans,
// then the wave totals). s_wave holds SCAN_THREADS / 64 ints.
constexpr int SCAN_THREADS = 1024;
__device__ __forceinline__ int block_inclusive_scan(int v, int *s_wave) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int u = __shfl_up(v, d, 64);
        if (lane >= d) v += u;
    }
    if (lane == 63) s_wave[wave] = v;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; w++) before += s_wave[w];
    __syncthreads();  // s_wave may be reused by the next scan
    return v + before;
}

// Single block, one thread per expert: the expert's total over the token
// blocks (counts[b*E + e]: each step reads one contiguous row), the exclusive scan of the totals in expert order (offsets[E];
// offsets[E+1] = offsets[E] + extra for the shared-expert segment), the
// per-block bases (base[b*E + e] = offsets[e] + counts of e in blocks < b),
// and the m-tile bases of the grouped GEMMs over the E+1 segments: a segment
// with at least `split` rows is tiled by mt_big rows in tile_big and is
// absent from tile_small, a shorter one the other way round (tile_x[s] =
// tiles of the segments before s; tile_x[E+1] = the total). experts < 1024.
__global__ void __launch_bounds__(SCAN_THREADS) k_dispatch_scan(const int *__restrict__ counts, int *__restrict__ base,
                                                                int *__restrict__ offsets, int *__restrict__ tile_small,
                                                                int *__restrict__ tile_big, int experts, int nb, int extra,
                                                                int split, int mt_small, int mt_big,
                                                                const uint32_t *__restrict__ flags,
                                                                uint32_t *__restrict__ status,
                                                                int4 *__restrict__ info_small,
                                                                int4 *__restrict__ info_big) {
    __shared__ int s_wave[SCAN_THREADS / 64];
    __shared__ uint32_t s_status;
    const int e = threadIdx.x;
    if (e == 0) s_status = 0;
    __syncthreads();
    for (int b = e; b < nb; b += SCAN_THREADS)
        if (flags[b]) atomicOr(&s_status, flags[b]);
    // The column is read in batches of SCAN_BATCH independent loads (one
    // batch up to 2048 tokens); a batch is kept for the base pass when it is
    // the only one.
    constexpr int SCAN_BATCH = 32;
    const int ec = min(e, experts - 1);  // threads past the experts read a valid column
    int v[SCAN_BATCH];
    int tot = 0;
    for (int b0 = 0; b0 < nb; b0 += SCAN_BATCH) {
#pragma unroll
        for (int u = 0; u < SCAN_BATCH; u++) v[u] = counts[(int64_t)min(b0 + u, nb - 1) * experts + ec];
#pragma unroll
        for (int u = 0; u < SCAN_BATCH; u++) tot += b0 + u < nb ? v[u] : 0;
    }
    if (e >= experts) tot = 0;
    const int incl = block_inclusive_scan(tot, s_wave), excl = incl - tot;
    if (e < experts) {
        offsets[e] = excl;
        int run = excl;
        for (int b0 = 0; b0 < nb; b0 += SCAN_BATCH) {
            if (nb > SCAN_BATCH) {
#pragma unroll
                for (int u = 0; u < SCAN_BATCH; u++) v[u] = counts[(int64_t)min(b0 + u, nb - 1) * experts + e];
            }
#pragma unroll
            for (int u = 0; u < SCAN_BATCH; u++)
                if (b0 + u < nb) {
                    base[(int64_t)(b0 + u) * experts + e] = run;
                    run += v[u];
                }
        }
        if (e == experts - 1) {
            offsets[experts] = incl;
            offsets[experts + 1] = incl + extra;
        }
    }
    // Tiles per segment (experts + 1 segments; the last holds the extra rows
    // and may be empty), then an inclusive scan of each kind.
    const int cnt = e < experts ? tot : e == experts ? extra : 0;
    int ns = 0, nbg = 0;
    if (cnt >= split) nbg = (cnt + mt_big - 1) / mt_big;
    else ns = (cnt + mt_small - 1) / mt_small;
    // Both kinds in one scan while the counts fit 16 and 15 bits (at most
    // rows / 16 + segments small and rows / 64 + segments big tiles, rows <=
    // 64 nb x 32 + extra), else one scan each.
    int ts, tb;
    if ((int64_t)nb * 128 + extra / 16 + experts + 1 < 32768) {
        const int both = block_inclusive_scan(ns | (nbg << 16), s_wave);
        ts = both & 0xffff;
        tb = both >> 16;
    } else {
        ts = block_inclusive_scan(ns, s_wave);
        tb = block_inclusive_scan(nbg, s_wave);
    }
    if (e == 0) *status = s_status;  // block scans above synchronised the block
    // Tile records of the segment (excl is the segment's first row, also for
    // the shared-expert segment, whose total is 0 here).
    if (e <= experts) {
        int4 *info = ns ? info_small : info_big;
        const int n = ns ? ns : nbg, mt = ns ? mt_small : mt_big, first = (ns ? ts : tb) - n;
        if (info)
            for (int j = 0; j < n; j++) info[first + j] = make_int4(e, excl + j * mt, excl + cnt, excl);
    }
    if (e <= experts) {
        if (tile_small) tile_small[e + 1] = ts;
        if (tile_big) tile_big[e + 1] = tb;
        if (e == 0) {
            if (tile_small) tile_small[0] = 0;
            if (tile_big) tile_big[0] = 0;
        }
    }
}

// The whole dispatch for up to kDispatchOneMaxBlocks token blocks (64
// tokens each) in one block of SCAN_THREADS threads: the token masks of
// every token block per expert in LDS, expert offsets by a block scan, the
// tilings and tile records, then the placement (same results as masks +
// scan + place). experts <= 512, tokens x topk + extra <= kDispatchOneRows.
// Up to 512 tokens (A/B on one GPU, graph replays against masks + scan +
// place: 128 tokens 154 -> 145 us per stack block, 256 tokens 191 -> 184,
// T=512 unchanged). The rows and parts lists are built in LDS (token |
// assignment << 16 per position) and written out in order: written
// straight from each assignment, the stores scatter over the lists and the
// block's single address unit took ~5.8 of the kernel's ~12.3 us at 512
// tokens (timeline marks, -DSM_DISPATCH_TRACE). A row's first position in
// its token block's part of the segment is the segment start plus the
// expert's tokens in the blocks before (popcounts of their masks).
constexpr int kDispatchOneMaxBlocks = 8;
constexpr int kDispatchOnePerThread = 8;  // assignments per thread: tokens x topk <= SCAN_THREADS x 8
constexpr int kDispatchOneRows = 7168;    // positions staged in LDS (512 tokens x top-13 + 512 shared)
#ifdef SM_DISPATCH_TRACE
// Timeline hook (profiling builds): thread 0 writes s_memrealtime (100 MHz) at mark k.
__device__ uint64_t g_dispatch_trace[16];
#define DISPATCH_MARK(k)                                                                   \
    do {                                                                                   \
        if (threadIdx.x == 0) g_dispatch_trace[k] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define DISPATCH_MARK(k) \
    do {                 \
    } while (0)
#endif
__global__ void __launch_bounds__(SCAN_THREADS) k_dispatch_one(const int *__restrict__ ids, int tokens, int topk,
                                                               int experts, int *__restrict__ offsets,
                                                               int *__restrict__ rows, int *__restrict__ parts,
                                                               int *__restrict__ where_, int extra,
                                                               int *__restrict__ tile_small,
                                                               int *__restrict__ tile_big, int split, int mt_small,
                                                               int mt_big, uint32_t *__restrict__ status,
                                                               int4 *__restrict__ info_small,
                                                               int4 *__restrict__ info_big) {
    __shared__ unsigned long long m[kDispatchOneMaxBlocks][512];  // [token block][expert] token masks
    __shared__ uint32_t s_stage[kDispatchOneRows];                // position -> token | assignment << 16
    __shared__ int s_off[513];
    __shared__ int s_wave[SCAN_THREADS / 64];
    __shared__ uint32_t s_flags;
    const int tid = threadIdx.x, n = tokens * topk, nb = (tokens + 63) >> 6;
    DISPATCH_MARK(0);
    // The thread's assignments a = tid + SCAN_THREADS u: IDs loaded once, all
    // at once (the placement uses them again).
    int my_e[kDispatchOnePerThread];
#pragma unroll
    for (int u = 0; u < kDispatchOnePerThread; u++) {
        const int a = tid + SCAN_THREADS * u;
        my_e[u] = a < n ? ids[a] : -1;
    }
    for (int i = tid; i < nb * 512; i += SCAN_THREADS) m[i >> 9][i & 511] = 0ull;
    if (tid == 0) s_flags = 0;
    __syncthreads();
    DISPATCH_MARK(1);
#pragma unroll
    for (int u = 0; u < kDispatchOnePerThread; u++) {
        const int a = tid + SCAN_THREADS * u, e = my_e[u];
        if (a >= n) continue;
        if (e < 0 || e >= experts) {
            atomicOr(&s_flags, 1u);
            continue;
        }
        const int t = a / topk;
        const unsigned long long bit = 1ull << (t & 63);
        if (atomicOr(&m[t >> 6][e], bit) & bit) atomicOr(&s_flags, 2u);
    }
    __syncthreads();
    DISPATCH_MARK(2);
    const int e = tid;
    int tot = 0;
    if (e < experts)
        for (int b = 0; b < nb; b++) tot += __popcll(m[b][e]);
    const int incl = block_inclusive_scan(tot, s_wave), excl = incl - tot;
    DISPATCH_MARK(3);
    if (e < experts) {
        offsets[e] = excl;
        s_off[e] = excl;
        if (e == experts - 1) {
            offsets[experts] = incl;
            offsets[experts + 1] = incl + extra;
            s_off[experts] = incl;
        }
    }
    // Tiles per segment, both kinds in one scan (small tiles in the low 16
    // bits: at most kDispatchOneRows of them).
    const int cnt = e < experts ? tot : e == experts ? extra : 0;
    int ns = 0, nbg = 0;
    if (cnt >= split) nbg = (cnt + mt_big - 1) / mt_big;
    else ns = (cnt + mt_small - 1) / mt_small;
    const int both = block_inclusive_scan(ns | (nbg << 16), s_wave);
    const int ts = both & 0xffff, tb = both >> 16;
    DISPATCH_MARK(4);
    if (e == 0) *status = s_flags;  // the block scans above synchronised the block
    if (e <= experts) {
        tile_small[e + 1] = ts;
        tile_big[e + 1] = tb;
        if (e == 0) tile_small[0] = tile_big[0] = 0;
        int4 *info = ns ? info_small : info_big;
        const int cnt_t = ns ? ns : nbg, mt = ns ? mt_small : mt_big, first = (ns ? ts : tb) - cnt_t;
        if (info)
            for (int j = 0; j < cnt_t; j++) info[first + j] = make_int4(e, excl + j * mt, excl + cnt, excl);
    }
    __syncthreads();  // s_off complete
    DISPATCH_MARK(5);
#pragma unroll
    for (int u = 0; u < kDispatchOnePerThread; u++) {
        const int a = tid + SCAN_THREADS * u, ex = my_e[u];
        if (a >= n) continue;
        if (ex < 0 || ex >= experts) {
            where_[a] = -1;
            continue;
        }
        const int t = a / topk, tb6 = t >> 6, tl = t & 63;
        int pos = s_off[ex] + (tl ? __popcll(m[tb6][ex] & ((1ull << tl) - 1ull)) : 0);
        for (int b = 0; b < tb6; b++) pos += __popcll(m[b][ex]);
        s_stage[pos] = (uint32_t)t | ((uint32_t)a << 16);
        where_[a] = pos;
    }
    if (extra)
        for (int t = tid; t < tokens; t += SCAN_THREADS) s_stage[s_off[experts] + t] = (uint32_t)t | 0xffff0000u;
    __syncthreads();
    DISPATCH_MARK(6);
    const int total = s_off[experts] + (extra ? tokens : 0);
    for (int p = tid; p < total; p += SCAN_THREADS) {
        const uint32_t v = s_stage[p];
        rows[p] = (int)(v & 0xffffu);
        parts[p] = (v >> 16) == 0xffffu ? -1 : (int)(v >> 16);
    }
#ifdef SM_DISPATCH_TRACE
    __syncthreads();
    DISPATCH_MARK(7);
#endif
}

__global__ void k_dispatch_place(const int *__restrict__ ids, int tokens, int topk, int experts, int nb,
                                 const unsigned long long *__restrict__ masks, const int *__restrict__ base,
                                 int *__restrict__ rows, int *__restrict__ parts, int *__restrict__ where_,
                                 int extra, const int *__restrict__ offsets) {
    const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)tokens * topk;
    if (a < n) {
        int t = (int)(a / topk), e = ids[a];
        if (e < 0 || e >= experts) {
            where_[a] = -1;
            return;
        }
        int b = t >> 6, tl = t & 63;
        unsigned long long below = tl ? (masks[(int64_t)b * experts + e] & ((1ull << tl) - 1ull)) : 0ull;
        int pos = base[(int64_t)b * experts + e] + __popcll(below);
        rows[pos] = t;
        parts[pos] = (int)a;
        where_[a] = pos;
    } else if (extra && a < n + tokens) {
        // The shared-expert segment follows the routed rows (offsets[experts]).
        int t = (int)(a - n), at = offsets[experts] + t;
        rows[at] = t;
        parts[at] = -1;
    }
}

// ---------------------------------------------------------- workspace
constexpr uint64_t kAlign = 256;
inline uint64_t up(uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct DispatchWs {
    uint64_t status, flags, masks, counts, base, tile_small, tile_big, end;
};
DispatchWs dispatch_ws(int tokens, int experts) {
    const uint64_t nb = (uint64_t)(tokens + 63) / 64;
    DispatchWs w;
    w.status = 0;  // uint32: bit 0 an ID out of range, bit 1 an ID repeated within a token
    w.flags = up(w.status + 64);
    w.masks = up(w.flags + (uint64_t)nb * 4);
    w.counts = up(w.masks + nb * experts * 8);
    w.base = up(w.counts + nb * experts * 4);
    w.tile_small = up(w.base + nb * experts * 4);
    w.tile_big = up(w.tile_small + ((uint64_t)experts + 2) * 4);
    w.end = up(w.tile_big + ((uint64_t)experts + 2) * 4);
    return w;
}

}  // namespace

namespace smi {

uint64_t dispatch_workspace(int tokens, int experts) { return dispatch_ws(tokens, experts).end; }

int topk_launch(sm_ctx *ctx, const float *logits, int *ids, float *weights, int tokens, int experts, int topk) {
    k_topk<<<(unsigned)tokens, 256, 0, ctx->stream>>>(logits, ids, weights, experts, topk);
    return launched(ctx);
}

int route_launch(sm_ctx *ctx, const float *X, int tokens, int width, const float *Wr, const float *bias, int experts,
                 int topk, float *logits, int *ids, float *weights, const float *gate_w, float *gate_out) {
    if (tokens <= kRouteRowsMaxTokens) {
        // Few tokens: one wave per (row, token), latency-bound anyway.
        const int total = experts + (gate_w ? 1 : 0);
        const dim3 grid((unsigned)((total + 7) / 8 * 8), (unsigned)tokens);
        if (width == 2048)
            k_route_rows<32><<<grid, 64, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, width, experts,
                                                          total);
        else
            k_route_rows<0><<<grid, 64, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, width, experts,
                                                         total);
        if (int rc = launched(ctx)) return rc;
        return topk_launch(ctx, logits, ids, weights, tokens, experts, topk);
    }
    const int nrows = experts + (gate_w ? 1 : 0);
    if (tokens <= kRouteSmallTileMaxTokens) {
        const dim3 grid((unsigned)ceil_div(ceil_div(nrows, 4), 4), (unsigned)ceil_div(tokens, 4));
        k_route_gemm<4, 4><<<grid, 256, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, tokens, width,
                                                          experts, gate_w ? 1 : 0);
    } else {
        const dim3 grid((unsigned)ceil_div(ceil_div(nrows, 8), 4), (unsigned)ceil_div(tokens, 8));
        k_route_gemm<8, 8><<<grid, 256, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, tokens, width,
                                                          experts, gate_w ? 1 : 0);
    }
    if (int rc = launched(ctx)) return rc;
    k_topk<<<(unsigned)tokens, 256, 0, ctx->stream>>>(logits, ids, weights, experts, topk);
    return launched(ctx);
}

int route(sm_ctx *ctx, uint64_t X, int tokens, int width, uint64_t Wr, uint64_t bias, int experts, int topk,
          uint64_t logits, uint64_t ids, uint64_t weights, uint64_t gate_w, uint64_t gate_out) {
    if (int rc = need(ctx, X, (uint64_t)tokens * width * 4, "X")) return rc;
    if (int rc = need(ctx, Wr, (uint64_t)experts * width * 4, "router weights")) return rc;
    if (bias)
        if (int rc = need(ctx, bias, (uint64_t)experts * 4, "router bias")) return rc;
    if (int rc = need(ctx, ids, (uint64_t)tokens * topk * 4, "ids")) return rc;
    if (int rc = need(ctx, weights, (uint64_t)tokens * topk * 4, "weights")) return rc;
    if (gate_w) {
        if (int rc = need(ctx, gate_w, (uint64_t)width * 4, "shared gate weights")) return rc;
        if (int rc = need(ctx, gate_out, (uint64_t)tokens * 4, "shared gate output")) return rc;
    }
    uint64_t L = logits;
    bool own = false;
    if (!L) {  // the caller does not keep the logits: use a temporary
        if (int rc = sm_alloc(ctx, (uint64_t)tokens * experts * 4, 0, &L)) return rc;
        own = true;
    } else if (int rc = need(ctx, L, (uint64_t)tokens * experts * 4, "logits")) {
        return rc;
    }
    int rc = route_launch(ctx, (const float *)X, tokens, width, (const float *)Wr, (const float *)bias, experts, topk,
                          (float *)L, (int *)ids, (float *)weights, (const float *)gate_w, (float *)gate_out);
    if (own) {
        int rc2 = sm_free(ctx, L);
        if (!rc) rc = rc2;
    }
    return rc;
}

int dispatch_launch(sm_ctx *ctx, const int *ids, int tokens, int topk, int experts, int *offsets, int *rows, int *parts,
                    int *where_, char *ws, int extra_rows, const GemmTiling *tiling) {
    const int nb = ceil_div(tokens, 64);
    DispatchWs w = dispatch_ws(tokens, experts);
    const uint64_t n = (uint64_t)tokens * topk, extra = extra_rows ? (uint64_t)tokens : 0;
    GemmTiling none = {(int *)(ws + w.tile_small), (int *)(ws + w.tile_big), 64, 32, 128};
    const GemmTiling &tl = tiling ? *tiling : none;
    if (nb <= kDispatchOneMaxBlocks && experts <= 512 && n <= (uint64_t)SCAN_THREADS * kDispatchOnePerThread &&
        n + extra <= (uint64_t)kDispatchOneRows) {
        k_dispatch_one<<<1, SCAN_THREADS, 0, ctx->stream>>>(ids, tokens, topk, experts, offsets, rows, parts, where_,
                                                            (int)extra, tl.small, tl.big, tl.split, tl.mt_small,
                                                            tl.mt_big, (uint32_t *)(ws + w.status),
                                                            (int4 *)tl.info_small, (int4 *)tl.info_big);
        return launched(ctx);
    }
    k_dispatch_masks<<<nb, 256, 0, ctx->stream>>>(ids, tokens, topk, experts, nb, (unsigned long long *)(ws + w.masks),
                                                  (int *)(ws + w.counts), (uint32_t *)(ws + w.flags));
    if (int rc = launched(ctx)) return rc;
    k_dispatch_scan<<<1, SCAN_THREADS, 0, ctx->stream>>>((const int *)(ws + w.counts), (int *)(ws + w.base), offsets,
                                                 tl.small, tl.big, experts, nb, (int)extra, tl.split, tl.mt_small,
                                                 tl.mt_big, (const uint32_t *)(ws + w.flags),
                                                 (uint32_t *)(ws + w.status), (int4 *)tl.info_small,
                                                 (int4 *)tl.info_big);
    if (int rc = launched(ctx)) return rc;
    const uint64_t threads = n + extra;
    k_dispatch_place<<<(unsigned)((threads + 255) / 256), 256, 0, ctx->stream>>>(
        ids, tokens, topk, experts, nb, (const unsigned long long *)(ws + w.masks), (const int *)(ws + w.base), rows,
        parts, where_, (int)extra, offsets);
    return launched(ctx);
}

int dispatch(sm_ctx *ctx, uint64_t ids, int tokens, int topk, int experts, uint64_t offsets, uint64_t rows,
             uint64_t parts, uint64_t where_, uint64_t workspace, uint64_t workspace_bytes, int extra_rows) {
    DispatchWs w = dispatch_ws(tokens, experts);
    const uint64_t n = (uint64_t)tokens * topk, extra = extra_rows ? (uint64_t)tokens : 0;
    if (workspace_bytes < w.end) return fail(ctx, SM_E_ARG, "dispatch workspace too small");
    if (int rc = need(ctx, workspace, w.end, "dispatch workspace")) return rc;
    if (int rc = need(ctx, ids, n * 4, "ids")) return rc;
    if (int rc = need(ctx, offsets, ((uint64_t)experts + 2) * 4, "offsets")) return rc;
    if (int rc = need(ctx, rows, (n + extra) * 4, "rows")) return rc;
    if (int rc = need(ctx, parts, (n + extra) * 4, "parts")) return rc;
    if (int rc = need(ctx, where_, n * 4, "where")) return rc;
    return dispatch_launch(ctx, (const int *)ids, tokens, topk, experts, (int *)offsets, (int *)rows, (int *)parts,
                           (int *)where_, (char *)workspace, extra_rows, nullptr);
}

}  // namespace smi

#ifdef SM_DISPATCH_TRACE
extern "C" int sm_dispatch_trace_read(uint64_t *out, int n) {
    if (n < 16) return SM_E_ARG;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_dispatch_trace), sizeof(uint64_t) * 16) == hipSuccess ? SM_OK
                                                                                                      : SM_E_HIP;
}
#endif
