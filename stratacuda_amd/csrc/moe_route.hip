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

// ------------------------------------------------------------ T = 1 route
// One 64-thread block per row: rows [0, experts) are router rows, row
// `experts` is the shared-expert gate (when gate_w != 0). NJ = width / 64
// loads per lane, all issued before the (sequential, reference-order) sum.
template <int NJ>
__global__ void __launch_bounds__(64) k_route_rows(const float *__restrict__ X, const float *__restrict__ Wr,
                                                   const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                   float *__restrict__ logits, float *__restrict__ gate_out, int width,
                                                   int experts) {
    const int row = blockIdx.x, lane = threadIdx.x;
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
constexpr int TT = 8, TR = 8;  // tokens x rows per wave

template <int N>
__device__ __forceinline__ void butterfly_level(float (&a)[64], int lane) {
    // N = number of outputs still held; keeps N/2.
    constexpr int H = N / 2;
    const bool upper = (lane & H) != 0;
#pragma unroll
    for (int i = 0; i < H; i++) {
        float send = upper ? a[i] : a[i + H];
        float keep = upper ? a[i + H] : a[i];
        a[i] = keep + __shfl_xor(send, H, 64);
    }
}

// Grid: x = row tiles (ceil((experts+1)/8)), y = token tiles (ceil(T/8)).
// Row `experts` is the shared-expert gate. Rows/tokens past the end are
// computed on clamped (valid) addresses and discarded.
__global__ void __launch_bounds__(256) k_route_gemm(const float *__restrict__ X, const float *__restrict__ Wr,
                                                    const float *__restrict__ bias, const float *__restrict__ Wsg,
                                                    float *__restrict__ logits, float *__restrict__ gate_out,
                                                    int tokens, int width, int experts, int with_gate) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nrows = experts + (with_gate ? 1 : 0);
    const int row_tiles = (nrows + TR - 1) / TR;
    const int tile = blockIdx.x * 4 + wave;
    if (tile >= row_tiles) return;
    const int r0 = tile * TR, t0 = blockIdx.y * TT;
    const float *wp[TR];
    const float *xp[TT];
#pragma unroll
    for (int r = 0; r < TR; r++) {
        int row = min(r0 + r, nrows - 1);
        wp[r] = row < experts ? Wr + (int64_t)row * width : Wsg;
    }
#pragma unroll
    for (int t = 0; t < TT; t++) xp[t] = X + (int64_t)min(t0 + t, tokens - 1) * width;
    float a[64];
#pragma unroll
    for (int o = 0; o < 64; o++) a[o] = 0.0f;
    for (int i = lane; i < width; i += 64) {
        float xv[TT], wv[TR];
#pragma unroll
        for (int t = 0; t < TT; t++) xv[t] = xp[t][i];
#pragma unroll
        for (int r = 0; r < TR; r++) wv[r] = wp[r][i];
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int r = 0; r < TR; r++) a[t * TR + r] = a[t * TR + r] + wv[r] * xv[t];
    }
    butterfly_level<64>(a, lane);
    butterfly_level<32>(a, lane);
    butterfly_level<16>(a, lane);
    butterfly_level<8>(a, lane);
    butterfly_level<4>(a, lane);
    butterfly_level<2>(a, lane);
    // lane l now holds output o = l: token t0 + l/8, row r0 + l%8.
    const int t = t0 + lane / TR, row = r0 + lane % TR;
    if (t < tokens && row < nrows) {
        if (row < experts) logits[(int64_t)t * experts + row] = bias ? a[0] + bias[row] : a[0];
        else gate_out[t] = a[0];
    }
}

__global__ void __launch_bounds__(256) k_topk(const float *__restrict__ logits, int *__restrict__ ids,
                                              float *__restrict__ weights, int tokens, int experts, int topk) {
    __shared__ uint64_t s_tab[32];
    sm::fill_exp_table(s_tab);
    __syncthreads();
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= tokens) return;
    sm::router_wave(logits + (int64_t)t * experts, ids + (int64_t)t * topk, weights + (int64_t)t * topk, experts, topk,
                    s_tab);
}

// ---------------------------------------------------------------- dispatch
// Block b covers tokens [64b, 64b+64). masks[b*E + e] = tokens of the block
// routed to e; counts[e*nb + b] = popcount. status bit 0: an ID outside
// [0, experts); bit 1: an ID repeated within one token.
__global__ void __launch_bounds__(256) k_dispatch_masks(const int *__restrict__ ids, int tokens, int topk, int experts,
                                                        int nb, unsigned long long *__restrict__ masks,
                                                        int *__restrict__ counts, uint32_t *status) {
    __shared__ unsigned long long m[512];
    const int b = blockIdx.x;
    for (int e = threadIdx.x; e < experts; e += blockDim.x) m[e] = 0ull;
    __syncthreads();
    const int t0 = b * 64, nt = min(64, tokens - t0);
    for (int a = threadIdx.x; a < nt * topk; a += blockDim.x) {
        int tl = a / topk, e = ids[(int64_t)(t0 + tl) * topk + a % topk];
        if (e < 0 || e >= experts) {
            atomicOr(status, 1u);
            continue;
        }
        unsigned long long bit = 1ull << tl;
        unsigned long long old = atomicOr(&m[e], bit);
        if (old & bit) atomicOr(status, 2u);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < experts; e += blockDim.x) {
        masks[(int64_t)b * experts + e] = m[e];
        counts[(int64_t)e * nb + b] = __popcll(m[e]);
    }
}

// Single block: exclusive scan of counts (expert-major) into base, per-expert
// offsets[E+1] (+ offsets[E+1] = offsets[E] + extra for the shared-expert
// segment), and the m-tile bases of the grouped GEMMs over the E+1 segments:
// a segment with at least `split` rows is tiled by mt_big rows in tile_big
// and is absent from tile_small, a shorter one the other way round
// (tile_x[s] = tiles of the segments before s; tile_x[E+1] = the total).
__global__ void __launch_bounds__(1024) k_dispatch_scan(const int *__restrict__ counts, int *__restrict__ base,
                                                        int *__restrict__ offsets, int *__restrict__ tile_small,
                                                        int *__restrict__ tile_big, int experts, int nb, int extra,
                                                        int split, int mt_small, int mt_big) {
    __shared__ int part[1024];
    __shared__ int tsm[1024], tbg[1024];
    const int n = experts * nb, tid = threadIdx.x;
    const int chunk = (n + 1023) / 1024, lo = min(n, tid * chunk), hi = min(n, lo + chunk);
    int s = 0;
    for (int b0 = lo; b0 < hi; b0 += 8) {  // 8 loads in flight at a time
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = b0 + u < hi ? counts[b0 + u] : 0;
#pragma unroll
        for (int u = 0; u < 8; u++) s += v[u];
    }
    part[tid] = s;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        int v = tid >= d ? part[tid - d] : 0;
        __syncthreads();
        part[tid] += v;
        __syncthreads();
    }
    int run = tid ? part[tid - 1] : 0;
    for (int b0 = lo; b0 < hi; b0 += 8) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = b0 + u < hi ? counts[b0 + u] : 0;
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (b0 + u < hi) base[b0 + u] = run;
            run += v[u];
        }
    }
    __syncthreads();
    const int total = part[1023];
    for (int e = tid; e < experts; e += 1024) offsets[e] = base[(int64_t)e * nb];
    if (tid == 0) {
        offsets[experts] = total;
        offsets[experts + 1] = total + extra;
    }
    __syncthreads();
    // Tiles per segment (experts + 1 segments, the last may be empty), then an
    // inclusive scan of each kind; experts + 1 <= 513 < 1024.
    int ns = 0, nbg = 0;
    if (tid <= experts) {
        const int cnt = offsets[tid + 1] - offsets[tid];
        if (cnt >= split) nbg = (cnt + mt_big - 1) / mt_big;
        else ns = (cnt + mt_small - 1) / mt_small;
    }
    tsm[tid] = ns;
    tbg[tid] = nbg;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        int vs = tid >= d ? tsm[tid - d] : 0, vb = tid >= d ? tbg[tid - d] : 0;
        __syncthreads();
        tsm[tid] += vs;
        tbg[tid] += vb;
        __syncthreads();
    }
    if (tid <= experts + 1) {
        if (tile_small) tile_small[tid] = tid ? tsm[tid - 1] : 0;
        if (tile_big) tile_big[tid] = tid ? tbg[tid - 1] : 0;
    }
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
        int pos = base[(int64_t)e * nb + b] + __popcll(below);
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
    uint64_t status, masks, counts, base, tile_small, tile_big, end;
};
DispatchWs dispatch_ws(int tokens, int experts) {
    const uint64_t nb = (uint64_t)(tokens + 63) / 64;
    DispatchWs w;
    w.status = 0;
    w.masks = up(w.status + 64);
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

int route_launch(sm_ctx *ctx, const float *X, int tokens, int width, const float *Wr, const float *bias, int experts,
                 int topk, float *logits, int *ids, float *weights, const float *gate_w, float *gate_out) {
    if (tokens == 1) {
        const int total = experts + (gate_w ? 1 : 0);
        if (width == 2048)
            k_route_rows<32><<<total, 64, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, width, experts);
        else
            k_route_rows<0><<<total, 64, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, width, experts);
        if (int rc = launched(ctx)) return rc;
        k_topk<<<1, 64, 0, ctx->stream>>>(logits, ids, weights, 1, experts, topk);
        return launched(ctx);
    }
    const int nrows = experts + (gate_w ? 1 : 0);
    dim3 grid((unsigned)ceil_div(ceil_div(nrows, TR), 4), (unsigned)ceil_div(tokens, TT));
    k_route_gemm<<<grid, 256, 0, ctx->stream>>>(X, Wr, bias, gate_w, logits, gate_out, tokens, width, experts,
                                                gate_w ? 1 : 0);
    if (int rc = launched(ctx)) return rc;
    k_topk<<<ceil_div(tokens, 4), 256, 0, ctx->stream>>>(logits, ids, weights, tokens, experts, topk);
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
    if (int rc = zero_words(ctx, ws + w.status, 16)) return rc;
    k_dispatch_masks<<<nb, 256, 0, ctx->stream>>>(ids, tokens, topk, experts, nb, (unsigned long long *)(ws + w.masks),
                                                  (int *)(ws + w.counts), (uint32_t *)(ws + w.status));
    if (int rc = launched(ctx)) return rc;
    GemmTiling none = {(int *)(ws + w.tile_small), (int *)(ws + w.tile_big), 64, 32, 128};
    const GemmTiling &tl = tiling ? *tiling : none;
    k_dispatch_scan<<<1, 1024, 0, ctx->stream>>>((const int *)(ws + w.counts), (int *)(ws + w.base), offsets,
                                                 tl.small, tl.big, experts, nb, (int)extra, tl.split, tl.mt_small,
                                                 tl.mt_big);
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
