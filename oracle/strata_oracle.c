/*
 * CPU oracle for the StrataCuda mixture-of-experts path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the timed CPU baseline; the product path never calls it.
 *
 * Each function restates one kernel of the reference's kernels/strata.cu in
 * plain C with the reference's exact f32 operation order: a workgroup of 64
 * lanes, lane l accumulating elements l, l+64, ... in order, followed by the
 * shared-memory tree reduction s = 32, 16, ..., 1 (lane l adds lane l+s).
 * Build with -ffp-contract=off: the reference's CPU path is WebAssembly, which
 * has no fused multiply-add, so every product and every sum rounds separately.
 *
 * Threads: workgroups are independent in every kernel restated here, so the
 * OpenMP loops over workgroups change neither results nor their bits.
 *
 * Parity pins (what each function is checked against, see tests/):
 *   or_half_bits       exhaustive 65,536 patterns vs numpy float16 and the
 *                      reference's own fp16_to_fp32 (dequant.hpp) built in oracle/_ref
 *   or_expf            exhaustive over [-104, 0] vs glibc expf (1 input differs)
 *   or_q2 decode       reference dequantize_q2_0 KAT (256 blocks) and the
 *                      gate/up interleave KAT (tests/model.test.mjs:32-50)
 *   or_router          "ties" / "spread" KATs (tests/conformance.js:35-39),
 *                      F64 router (tests/reference.mjs:173-177), brute force sort
 *   or_project etc.    F64 numpy dot products within 2e-5 (tests/conformance.js:7-10)
 *   or_dispatch        brute-force stable grouping (src/prefill.js:56-61)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#include <omp.h>

#define LANES 64

/* ---------------------------------------------------------------- fp16 --- */
/* kernels/strata.cu:13-18 strata_half_bits */
/* Thread count of the OpenMP loops below (the CPU baseline times the oracle
 * at the reference pool's default of 4 threads and its limit of 8,
 * vendor/webcuda/src/wasm/thread-pool.hpp:49-50). */
void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int or_max_threads(void) { return omp_get_max_threads(); }

float or_half_bits(uint32_t h) {
    uint32_t sign = (h & 32768u) << 16, exponent = (h >> 10) & 31u, fraction = h & 1023u, bits;
    float out;
    if (exponent == 0u) {
        if (fraction == 0u) { memcpy(&out, &sign, 4); return out; }
        float v = (float)fraction * 0.000000059604644775390625f;
        return sign != 0u ? -v : v;
    }
    if (exponent == 31u) bits = sign | 2139095040u | (fraction << 13);
    else bits = sign | ((exponent + 112u) << 23) | (fraction << 13);
    memcpy(&out, &bits, 4);
    return out;
}

/* ---------------------------------------------------------------- expf --- */
/* libm expf as the reference's WebAssembly build evaluates it: musl's expf is
 * the ARM optimized-routines design (N = 32 table of 2^(i/32), cubic
 * polynomial for 2^(r/32), double arithmetic), and wasm32 has no FMA, so each
 * double operation rounds separately. The table is 2^(i/32) rounded to double
 * with i<<47 subtracted from its bits; it is filled at first use. */
static uint64_t or_exp2_tab[32];
static int or_exp2_ready = 0;
static uint64_t u64_of(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static double dbl_of(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static void or_exp_init(void) {
    if (or_exp2_ready) return;
    for (int i = 0; i < 32; i++) {
        long double v = powl(2.0L, (long double)i / 32.0L);
        or_exp2_tab[i] = u64_of((double)v) - ((uint64_t)i << 47);
    }
    or_exp2_ready = 1;
}
float or_expf(float x) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double Shift = 0x1.8p+52;
    uint32_t ux; memcpy(&ux, &x, 4);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) { /* |x| >= 88 or NaN/inf (top12 of 88.0f = 0x42b) */
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;          /* overflow */
        if (x < -0x1.9fe368p6f) return 0.0f;             /* underflow */
    }
    or_exp_init();
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + Shift;
    uint64_t ki = u64_of(kd);
    kd -= Shift;
    double r = z - kd;
    uint64_t t = or_exp2_tab[ki % 32];
    t += ki << 47;
    double s = dbl_of(t);
    double zz = C0 * r;
    zz = zz + C1;
    double r2 = r * r;
    double y = C2 * r;
    y = y + 1.0;
    double q = zz * r2;
    y = q + y;
    y = y * s;
    return (float)y;
}
/* kernels/strata.cu:7-8 */
float or_sigmoid(float x) { return 1.0f / (1.0f + or_expf(-x)); }
float or_silu(float x) { return x * or_sigmoid(x); }

/* tree reduction of 64 lane partials, kernels/strata.cu:53,66,128,163 */
static float tree_sum(float *p) {
    for (int s = 32; s > 0; s >>= 1)
        for (int l = 0; l < s; l++) p[l] += p[l + s];
    return p[0];
}

static inline uint32_t q2_code_word(const uint32_t *blob, int64_t index, int64_t word_base) {
    return (blob[word_base + index / 16] >> ((index % 16) * 2)) & 3u;
}
static inline float blob_half(const uint32_t *blob, int64_t s) {
    return or_half_bits((blob[s / 2] >> ((s % 2) * 16)) & 65535u);
}

/* ------------------------------------------------------------ kernels --- */
/* kernels/strata.cu:19-21 strata_unpack_half */
void or_unpack_half(const uint32_t *packed, float *values, int count) {
    for (int i = 0; i < count; i++) values[i] = or_half_bits((packed[i / 2] >> ((i % 2) * 16)) & 65535u);
}
/* kernels/strata.cu:35-37 strata_expert_scales */
void or_expert_scales(const uint32_t *blob, float *scales, int offset, int count) {
    for (int i = 0; i < count; i++) scales[i] = blob_half(blob, (int64_t)offset + i);
}

/* kernels/strata.cu:156-165 strata_project; also strata_gemv :121-130 with
 * outputStride = rows, outputOffset = 0. Grid [rows, tokens]. */
void or_project(const float *X, const float *W, float *Y, int cols, int rows, int tokens,
                int outputStride, int outputOffset) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < rows; row++) {
            float p[LANES];
            const float *w = W + (int64_t)row * cols, *x = X + (int64_t)token * cols;
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int i = l; i < cols; i += LANES) sum += w[i] * x[i];
                p[l] = sum;
            }
            Y[(int64_t)token * outputStride + outputOffset + row] = tree_sum(p);
        }
}

/* kernels/strata.cu:38-55 strata_q2_gate_up. Grid [ff, tokens]. */
void or_q2_gate_up(const float *X, const uint32_t *Blob, const float *Scales, const int *Mapping,
                   float *Hidden, int width, int ff, int tokens, int mapped, int expanded,
                   int codeOffset, int scaleOffset) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < ff; row++) {
            int inputRow = mapped ? Mapping[2 * token] : token;
            float gp[LANES], up[LANES];
            for (int l = 0; l < LANES; l++) {
                float g = 0.0f, u = 0.0f;
                for (int i = l; i < width; i += LANES) {
                    int64_t gi = (int64_t)row * 2 * width + i, ui = gi + width;
                    int gc = (int)q2_code_word(Blob, gi, codeOffset) - 1;
                    int uc = (int)q2_code_word(Blob, ui, codeOffset) - 1;
                    int64_t gs = scaleOffset + gi / 64, us = scaleOffset + ui / 64;
                    float gw = (float)gc * (expanded ? Scales[gs] : blob_half(Blob, gs));
                    float uw = (float)uc * (expanded ? Scales[us] : blob_half(Blob, us));
                    float x = X[(int64_t)inputRow * width + i];
                    g += gw * x;
                    u += uw * x;
                }
                gp[l] = g; up[l] = u;
            }
            /* both trees advance level by level in the reference; the two
             * reductions are independent so their order does not matter */
            float gs = tree_sum(gp), us = tree_sum(up);
            Hidden[(int64_t)token * ff + row] = or_silu(gs) * us;
        }
}

/* kernels/strata.cu:56-69 strata_q2_down. Grid [width, tokens]. */
void or_q2_down(const float *Hidden, const uint32_t *Blob, const float *Scales, const int *Mapping,
                float *Y, int width, int ff, int tokens, int mapped, int expanded,
                int outputOffset, int codeOffset, int scaleOffset) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < width; row++) {
            float p[LANES];
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int i = l; i < ff; i += LANES) {
                    int64_t index = (int64_t)row * ff + i;
                    int code = (int)q2_code_word(Blob, index, codeOffset) - 1;
                    int64_t si = scaleOffset + index / 64;
                    float w = (float)code * (expanded ? Scales[si] : blob_half(Blob, si));
                    sum += w * Hidden[(int64_t)token * ff + i];
                }
                p[l] = sum;
            }
            int destination = mapped ? Mapping[2 * token + 1] : token;
            Y[(int64_t)outputOffset + (int64_t)destination * width + row] = tree_sum(p);
        }
}

/* kernels/strata.cu:179-192 strata_q2_project. Grid [rows, tokens]. */
void or_q2_project(const float *X, const uint32_t *Blob, float *Y, int cols, int rows, int tokens,
                   int outputStride, int outputOffset, int codeOffset, int scaleOffset,
                   int weightRow, int rowStride) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < rows; row++) {
            float p[LANES];
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int i = l; i < cols; i += LANES) {
                    int64_t ix = (int64_t)(weightRow + row * rowStride) * cols + i;
                    int code = (int)q2_code_word(Blob, ix, codeOffset) - 1;
                    float weight = (float)code * blob_half(Blob, scaleOffset + ix / 64);
                    sum += weight * X[(int64_t)token * cols + i];
                }
                p[l] = sum;
            }
            Y[(int64_t)token * outputStride + outputOffset + row] = tree_sum(p);
        }
}

/* kernels/strata.cu:22-31 */
static float or_iq4(int c) {
    static const float t[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    return t[c & 15];
}
/* kernels/strata.cu:9-12 */
static int or_group(int index, int size) { return index / size; }

/* kernels/strata.cu:193-211 strata_quant_project. Grid [rows, tokens]. */
void or_quant_project(const float *X, const uint32_t *Codes, const float *Scales, const float *Offsets,
                      float *Y, int cols, int rows, int tokens, int outputStride, int outputOffset,
                      int bits, int groupSize, int bias, int codebook, int hasOffset) {
    #pragma omp parallel for collapse(2) schedule(static)
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < rows; row++) {
            float p[LANES];
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int i = l; i < cols; i += LANES) {
                    int index = row * cols + i, bit = index * bits;
                    int code = (int)((Codes[bit / 32] >> (bit % 32)) & ((1u << bits) - 1u));
                    float value = codebook == 1 ? or_iq4(code) : (float)(code + bias);
                    int group = or_group(index, groupSize);
                    float weight = value * Scales[group];
                    if (hasOffset) weight += Offsets[group];
                    sum += weight * X[(int64_t)token * cols + i];
                }
                p[l] = sum;
            }
            Y[(int64_t)token * outputStride + outputOffset + row] = tree_sum(p);
        }
}

/* kernels/strata.cu:214-227 strata_norm. Grid [rows]. */
void or_norm(const float *X, const float *W, float *Y, int cols, int rows, int weightRows, int mode,
             float epsilon, float scale) {
    #pragma omp parallel for schedule(static)
    for (int row = 0; row < rows; row++) {
        float p[LANES];
        for (int l = 0; l < LANES; l++) {
            float ss = 0.0f;
            for (int i = l; i < cols; i += LANES) { float v = X[(int64_t)row * cols + i]; ss += v * v; }
            p[l] = ss;
        }
        float total = tree_sum(p);
        float inv = scale / sqrtf((mode == 0 ? total / (float)cols : total) + epsilon);
        for (int i = 0; i < cols; i++) {
            float w = mode == 0 ? W[(int64_t)(row % weightRows) * cols + i] : 1.0f;
            Y[(int64_t)row * cols + i] = X[(int64_t)row * cols + i] * inv * w;
        }
    }
}

/* kernels/strata.cu:230-236 strata_elementwise */
void or_elementwise(const float *A, const float *B, float *Y, int n, int mode, float scale) {
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < n; i++) {
        float a = A[i] * scale, v = a;
        if (mode == 1) v = or_silu(a);
        if (mode == 2) v = or_sigmoid(a);
        if (mode == 3) v = or_silu(a) * B[i];
        if (mode == 4) v = a * or_sigmoid(B[i]);
        if (mode == 5) v = a + B[i];
        Y[i] = v;
    }
}

/* kernels/strata.cu:240-270 strata_router and :479-509 strata_router_batch
 * (identical per token). One 64-lane workgroup per token. */
static void router_one(const float *Logits, int *Ids, float *Weights, int experts, int topK) {
    float prob[512], reduce[LANES], selected[32];
    int winner[LANES];
    for (int l = 0; l < LANES; l++) {
        float mx = -3.402823e38f;
        for (int e = l; e < experts; e += LANES) mx = fmaxf(mx, Logits[e]);
        reduce[l] = mx;
    }
    for (int s = 32; s > 0; s >>= 1)
        for (int l = 0; l < s; l++) reduce[l] = fmaxf(reduce[l], reduce[l + s]);
    float mx = reduce[0];
    for (int l = 0; l < LANES; l++) {
        float sum = 0.0f;
        for (int e = l; e < experts; e += LANES) { prob[e] = or_expf(Logits[e] - mx); sum += prob[e]; }
        reduce[l] = sum;
    }
    float inv = 1.0f / tree_sum(reduce);
    for (int e = 0; e < experts; e++) prob[e] *= inv;
    for (int k = 0; k < topK; k++) {
        for (int l = 0; l < LANES; l++) {
            float best = -1.0f; int id = experts;
            for (int e = l; e < experts; e += LANES)
                if (prob[e] > best || (prob[e] == best && e < id)) { best = prob[e]; id = e; }
            reduce[l] = best; winner[l] = id;
        }
        for (int s = 32; s > 0; s >>= 1)
            for (int l = 0; l < s; l++) {
                float v = reduce[l + s]; int j = winner[l + s];
                if (v > reduce[l] || (v == reduce[l] && j < winner[l])) { reduce[l] = v; winner[l] = j; }
            }
        Ids[k] = winner[0]; selected[k] = reduce[0];
        /* the reference writes prob[winner] = -1; a winner of `experts`
         * cannot occur for topK <= experts */
        if (winner[0] < experts) prob[winner[0]] = -1.0f;
    }
    float denom = 0.0f;
    for (int k = 0; k < topK; k++) denom += selected[k];
    denom = fmaxf(denom, 0.00006103515625f);
    for (int k = 0; k < topK; k++) Weights[k] = selected[k] / denom;
}
void or_router_batch(const float *Logits, int *Ids, float *Weights, int experts, int topK, int tokens) {
    #pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; t++)
        router_one(Logits + (int64_t)t * experts, Ids + (int64_t)t * topK, Weights + (int64_t)t * topK,
                   experts, topK);
}

/* kernels/strata.cu:360-365 strata_moe_combine and :470-476 _batch */
void or_moe_combine_batch(const float *Parts, const float *Weights, const float *Shared,
                          const float *SharedGate, float *Y, int width, int count, int tokens) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)width * tokens; i++) {
        int64_t token = i / width, d = i % width;
        float value = Shared[i] * or_sigmoid(SharedGate[token]);
        for (int k = 0; k < count; k++)
            value += Parts[(token * count + k) * width + d] * Weights[token * count + k];
        Y[i] = value;
    }
}

/* kernels/strata.cu:464-469 */
void or_gather_rows(const float *X, const int *Indices, float *Y, int width, int rows) {
    for (int64_t i = 0; i < (int64_t)width * rows; i++) Y[i] = X[(int64_t)Indices[i / width] * width + i % width];
}
void or_scatter_rows(const float *X, const int *Indices, float *Y, int width, int rows) {
    for (int64_t i = 0; i < (int64_t)width * rows; i++) Y[(int64_t)Indices[i / width] * width + i % width] = X[i];
}

/* ----------------------------------------------------------- dispatch --- */
/* Expert-contiguous dispatch. src/prefill.js:56-61 groups the routed
 * (token, k) pairs per expert, each expert's jobs in ascending token order,
 * with part = token*topK + k. Experts here are ordered by ascending ID (the
 * reference orders them by first appearance; the within-expert order, which
 * alone fixes every arithmetic result, is the same).
 * Outputs: offsets[experts+1] (exclusive scan of per-expert counts),
 * rows[pos] = token, parts[pos] = token*topK + k, where_[token*topK + k] = pos. */
int or_dispatch(const int *Ids, int tokens, int topK, int experts, int *offsets, int *rows,
                int *parts, int *where_) {
    int *count = (int *)calloc((size_t)experts + 1, sizeof(int));
    if (!count) return -1;
    for (int64_t a = 0; a < (int64_t)tokens * topK; a++) {
        int e = Ids[a];
        if (e < 0 || e >= experts) { free(count); return -2; }
        count[e]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < experts; e++) offsets[e + 1] = offsets[e] + count[e];
    for (int e = 0; e < experts; e++) count[e] = offsets[e];
    for (int t = 0; t < tokens; t++)
        for (int k = 0; k < topK; k++) {
            int e = Ids[(int64_t)t * topK + k], pos = count[e]++;
            rows[pos] = t; parts[pos] = t * topK + k; where_[(int64_t)t * topK + k] = pos;
        }
    free(count);
    return 0;
}

/* ------------------------------------------------------ MoE layer ------ */
/* Blob layout (vendor/strata/tools/pack_layer.py:54-65,99-105): gate/up codes
 * (2F rows interleaved g0,u0,...; W/4 bytes each), down codes (W rows of
 * F/4 bytes), gate/up fp16 scales (2F x W/64), down fp16 scales (W x F/64). */
typedef struct {
    int64_t gate_up_codes, down_codes, gate_up_scales, down_scales, blob_bytes;
} or_blob_layout;
or_blob_layout or_layout(int width, int ff) {
    or_blob_layout L;
    L.gate_up_codes = 0;
    L.down_codes = (int64_t)2 * ff * width / 4;
    L.gate_up_scales = L.down_codes + (int64_t)width * ff / 4;
    L.down_scales = L.gate_up_scales + (int64_t)2 * ff * (width / 64) * 2;
    L.blob_bytes = L.down_scales + (int64_t)width * (ff / 64) * 2;
    return L;
}

/* Ops.packedExpert (src/ops.js:56-72) on a resident blob: gate_up then down,
 * writing rows of Y at outputOffset + Mapping[2t+1]*width (mapped) or t*width. */
void or_packed_expert(const float *X, const uint32_t *blob, const int *mapping, float *hidden,
                      float *Y, int width, int ff, int tokens, int outputOffset) {
    or_blob_layout L = or_layout(width, ff);
    int mapped = mapping != NULL;
    or_q2_gate_up(X, blob, NULL, mapping, hidden, width, ff, tokens, mapped, 0,
                  (int)(L.gate_up_codes / 4), (int)(L.gate_up_scales / 2));
    or_q2_down(hidden, blob, NULL, mapping, Y, width, ff, tokens, mapped, 0, outputOffset,
               (int)(L.down_codes / 4), (int)(L.down_scales / 2));
}

/* One MoE layer over `tokens` rows in the reference stage order
 * (src/engine.js:133-156 for one token, src/prefill.js:52-78 for a batch):
 *   router projection -> (+ optional per-expert logit bias, an elementwise
 *   add before the router) -> router -> per-expert gate_up/down into part
 *   slots t*topK+k -> shared expert -> shared-gate projection -> combine.
 * Outputs: Y [tokens x width]; Ids/Weights [tokens x topK]; Logits
 * [tokens x experts] (optional). Scratch is allocated here. */
int or_moe_layer(const float *X, int tokens, const float *Wr, const float *bias, const uint8_t *arena,
                 int64_t blob_stride, const uint8_t *shared_blob, const float *Wsg, int width, int ff,
                 int experts, int topK, float *Y, int *Ids, float *Weights, float *LogitsOut) {
    float *logits = (float *)malloc(sizeof(float) * (size_t)tokens * experts);
    float *parts = (float *)malloc(sizeof(float) * (size_t)tokens * topK * width);
    float *shared = (float *)malloc(sizeof(float) * (size_t)tokens * width);
    float *hidden = (float *)malloc(sizeof(float) * (size_t)tokens * (topK > 1 ? topK : 1) * ff);
    float *gate = (float *)malloc(sizeof(float) * (size_t)tokens);
    int *offsets = (int *)malloc(sizeof(int) * ((size_t)experts + 1));
    int *rows = (int *)malloc(sizeof(int) * (size_t)tokens * topK);
    int *partIdx = (int *)malloc(sizeof(int) * (size_t)tokens * topK);
    int *where_ = (int *)malloc(sizeof(int) * (size_t)tokens * topK);
    int *mapping = (int *)malloc(sizeof(int) * 2 * (size_t)tokens * topK);
    int rc = 0;
    if (!logits || !parts || !shared || !hidden || !gate || !offsets || !rows || !partIdx || !where_ || !mapping) { rc = -1; goto done; }
    or_project(X, Wr, logits, width, experts, tokens, experts, 0);
    if (bias) {
        for (int t = 0; t < tokens; t++)
            for (int e = 0; e < experts; e++) {
                float a = logits[(int64_t)t * experts + e] * 1.0f;
                logits[(int64_t)t * experts + e] = a + bias[e];
            }
    }
    if (LogitsOut) memcpy(LogitsOut, logits, sizeof(float) * (size_t)tokens * experts);
    or_router_batch(logits, Ids, Weights, experts, topK, tokens);
    rc = or_dispatch(Ids, tokens, topK, experts, offsets, rows, partIdx, where_);
    if (rc) goto done;
    for (int e = 0; e < experts; e++) {
        int n = offsets[e + 1] - offsets[e];
        if (!n) continue;
        for (int j = 0; j < n; j++) {
            mapping[2 * j] = rows[offsets[e] + j];
            mapping[2 * j + 1] = partIdx[offsets[e] + j];
        }
        or_packed_expert(X, (const uint32_t *)(arena + (int64_t)e * blob_stride), mapping, hidden, parts,
                         width, ff, n, 0);
    }
    or_packed_expert(X, (const uint32_t *)shared_blob, NULL, hidden, shared, width, ff, tokens, 0);
    or_project(X, Wsg, gate, width, 1, tokens, 1, 0);
    or_moe_combine_batch(parts, Weights, shared, gate, Y, width, topK, tokens);
done:
    free(logits); free(parts); free(shared); free(hidden); free(gate); free(offsets);
    free(rows); free(partIdx); free(where_); free(mapping);
    return rc;
}

/* Stacked decode glue (48-layer MoE stack): h' = h + MoE(RMSNorm(h; gamma)),
 * as strata_norm mode 0 (eps 1e-6, src/ops.js:116) then strata_elementwise
 * mode 5. One layer; the caller chains layers. */
int or_moe_block(const float *H, float *Hout, int tokens, const float *gamma, const float *Wr,
                 const uint8_t *arena, int64_t blob_stride, const uint8_t *shared_blob,
                 const float *Wsg, int width, int ff, int experts, int topK, int *Ids, float *Weights) {
    float *xn = (float *)malloc(sizeof(float) * (size_t)tokens * width);
    float *y = (float *)malloc(sizeof(float) * (size_t)tokens * width);
    int rc = -1;
    if (xn && y) {
        or_norm(H, gamma, xn, width, tokens, 1, 0, 1e-6f, 1.0f);
        rc = or_moe_layer(xn, tokens, Wr, NULL, arena, blob_stride, shared_blob, Wsg, width, ff, experts,
                          topK, y, Ids, Weights, NULL);
        if (!rc) or_elementwise(H, y, Hout, tokens * width, 5, 1.0f);
    }
    free(xn); free(y);
    return rc;
}

/* ---------------------------------------------------- synthetic inputs --- */
/* Counter-based generator for the seeded synthetic workloads. Host and device
 * draw identical bits because every step is integer arithmetic or one IEEE
 * double multiply rounded to float:
 *   rand(seed, stream, i) = mix(mix(seed + G*(stream+1)) + i), mix = SplitMix64
 *   uniform u32 pair      = low / high halves of rand
 *   normal(i)             = Irwin-Hall: sum of 12 uniform u32 from rand(6i..6i+5),
 *                           times 2^-32, minus 6 (mean 0, variance 1, |n| <= 6)
 * Blob codes are raw random bytes (uniform 2-bit codes); blob scales are
 * fp16(|sigma * normal|) rounded to nearest even. */
static uint64_t or_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t or_rand(uint64_t seed, uint64_t stream, uint64_t i) {
    return or_mix(or_mix(seed + 0x9E3779B97F4A7C15ull * (stream + 1)) + i);
}
double or_normal(uint64_t seed, uint64_t stream, uint64_t i) {
    uint64_t s = 0;
    for (int j = 0; j < 6; j++) {
        uint64_t r = or_rand(seed, stream, 6 * i + j);
        s += (r & 0xffffffffull) + (r >> 32);
    }
    return (double)s * 0x1p-32 - 6.0;
}
/* float -> binary16, round to nearest even (IEEE 754 conversion). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t half = m >> shift, rem = m & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)(sign | half);
}
/* f32 values sigma * normal, rounded once to float. */
void or_synth_normal(float *out, int64_t n, uint64_t seed, uint64_t stream, double sigma) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = (float)(or_normal(seed, stream, (uint64_t)i) * sigma);
}
/* f32 values 1 + amp * U(-1, 1), U from the low 32 bits of rand. */
void or_synth_uniform_pm(float *out, int64_t n, uint64_t seed, uint64_t stream, double amp) {
    for (int64_t i = 0; i < n; i++) {
        double u = (double)(or_rand(seed, stream, (uint64_t)i) & 0xffffffffull) * 0x1p-31 - 1.0;
        out[i] = (float)(1.0 + amp * u);
    }
}
/* One Q2 expert blob: code bytes (u32 word w = low half of rand(stream, w)),
 * then fp16 scales |sigma * normal(scale stream)|. */
void or_synth_blob(uint8_t *blob, int width, int ff, uint64_t seed, uint64_t stream, double sigma) {
    or_blob_layout L = or_layout(width, ff);
    uint32_t *words = (uint32_t *)blob;
    int64_t code_words = L.gate_up_scales / 4, halves = (L.blob_bytes - L.gate_up_scales) / 2;
    #pragma omp parallel for schedule(static)
    for (int64_t w = 0; w < code_words; w++) words[w] = (uint32_t)(or_rand(seed, stream, (uint64_t)w) & 0xffffffffull);
    uint16_t *scales = (uint16_t *)(blob + L.gate_up_scales);
    #pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < halves; j++)
        scales[j] = or_f32_to_f16((float)fabs(sigma * or_normal(seed, stream + (1ull << 32), (uint64_t)j)));
}

/* ------------------------------------------------------- self checks --- */
/* Counts, over float bit patterns u = start, start+step, ... < end, the inputs
 * where or_expf differs from this platform's libm expf (out[0]) and from
 * (float)exp((double)x) (out[1]). Used to pin or_expf against libm. */
void or_expf_survey(uint32_t start, uint32_t end, uint32_t step, uint64_t *out) {
    uint64_t d_libm = 0, d_dbl = 0;
    #pragma omp parallel for reduction(+ : d_libm, d_dbl) schedule(static)
    for (int64_t u = start; u < (int64_t)end; u += step) {
        uint32_t bits = (uint32_t)u;
        float x; memcpy(&x, &bits, 4);
        float a = or_expf(x), b = expf(x), c = (float)exp((double)x);
        uint32_t ua, ub, uc; memcpy(&ua, &a, 4); memcpy(&ub, &b, 4); memcpy(&uc, &c, 4);
        d_libm += ua != ub;
        d_dbl += ua != uc;
    }
    out[0] = d_libm; out[1] = d_dbl;
}
