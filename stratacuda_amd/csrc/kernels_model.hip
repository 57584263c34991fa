// The untrained fixture model's kernels outside the MoE path, by reference
// name for sm_run (backend.run(name, args, groups)): what StrataEngine.step
// (src/engine.js:76-196) launches besides the router, the projections, the
// norm, the elementwise modes and the combine.
//
// Each kernel computes what the kernels/strata.cu entry of the same name
// computes, in the same f32 (and, for RoPE, f64) operation order, so results
// are bit-identical to the CPU oracle. Kernels of one work item per lane use
// 256-thread blocks over the items the 64-lane grid covers; the three
// reductions (attention, PLE gate, argmax) run one reference workgroup as one
// 64-lane wavefront, the reference's shared-memory trees becoming cross-lane
// shuffles in the same order.
//
// Launchers check the reference's validateDispatch conditions
// (src/backend.js:33-55) and then every buffer access of the requested grid
// against the recorded allocation sizes before anything runs; work items the
// reference computes but never stores (attention and PLE-gate groups beyond
// `heads` / `streams`) are skipped.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <string>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

constexpr float kNegBig = -3.402823e38f;  // the reference's initial maximum (kernels/strata.cu:337,388)

// IQ4_NL codebook (kernels/strata.cu:22-31).
__constant__ float kIq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
__device__ __forceinline__ float iq4_value(int c) { return kIq4[c & 15]; }
__device__ __forceinline__ int item() { return (int)(blockIdx.x * blockDim.x + threadIdx.x); }

// kernels/strata.cu:72-80
__global__ void k_embedding(const float *Values, const uint32_t *Codes, const float *Scales, const float *Offsets,
                            float *Residual, int width, int streams, int outputOffset, int format, int bits,
                            int groupSize, int bias, int codebook, int hasOffset, int n) {
    int i = item();
    if (i >= n) return;
    float value = 0.0f;
    if (format == 0) {
        value = Values[i];
    } else if (format == 1) {
        value = __uint_as_float(((Codes[i / 2] >> ((i % 2) * 16)) & 65535u) << 16);
    } else {
        int bit = i * bits, group = i / groupSize;
        int code = (int)((Codes[bit / 32] >> (bit % 32)) & ((1u << bits) - 1u));
        value = (codebook == 1 ? iq4_value(code) : (float)(code + bias)) * Scales[group];
        if (hasOffset != 0) value = value + Offsets[group];
    }
    for (int s = 0; s < streams; ++s) Residual[outputOffset + s * width + i] = value;
}

// kernels/strata.cu:90-104: ln(base) by the atanh series (25 odd terms) after
// halving base below 2, the power split into whole multiples of ln 2 and a
// remainder, 2^remainder-ish by a 20-term exp series, scaled by halvings.
__global__ void k_rope_frequencies(float *High, float *Low, int rotary, float base, int n) {
    int i = item();
    if (i >= n) return;
    const double ln2 = 0.693147180559945309417232121458176568;
    double m = (double)base;
    int ex = 0;
    while (m >= 2.0) {
        m = m * 0.5;
        ex += 1;
    }
    double y = (m - 1.0) / (m + 1.0), term = y, lg = 0.0;
    for (int k = 1; k <= 49; k += 2) {
        lg = lg + term / (double)k;
        term = term * y * y;
    }
    lg = 2.0 * lg + (double)ex * ln2;
    double power = -lg * (double)(2 * i) / (double)rotary;
    int whole = (int)(float)(power / ln2);
    double rem = power - (double)whole * ln2, result = 1.0;
    term = 1.0;
    for (int k = 1; k <= 20; ++k) {
        term = term * rem / (double)k;
        result = result + term;
    }
    for (; whole < 0; whole++) result = result * 0.5;
    High[i] = (float)result;
    Low[i] = (float)(result - (double)High[i]);
}

// kernels/strata.cu:105-111
__global__ void k_rope_table(const float *High, const float *Low, float *Cos, float *Sin, int half, int n) {
    int i = item();
    if (i >= n) return;
    const double turn = 6.283185307179586476925286766559005768;
    int pair = i % half;
    double angle = (double)(i / half) * ((double)High[pair] + (double)Low[pair]);
    int wraps = (int)(float)(angle / turn + 0.5);
    float reduced = (float)(angle - (double)wraps * turn), s, c;
    sm::sincos_or(reduced, s, c);
    Cos[i] = c;
    Sin[i] = s;
}

// kernels/strata.cu:113-120
__global__ void k_rope_position(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int heads,
                                int rotary, int position, int n) {
    int i = item();
    if (i >= n) return;
    int d = i % dim;
    if (d >= rotary) {
        Y[i] = X[i];
        return;
    }
    int half = rotary / 2, pair = d % half, row = i - d;
    int angle = (position + i / (dim * heads)) * half + pair;
    float c = Cos[angle], s = Sin[angle], a = X[row + pair], b = X[row + pair + half];
    Y[i] = d < half ? a * c - b * s : b * c + a * s;
}

// kernels/strata.cu:273-277
__global__ void k_hc_mix(const float *Norm, const float *Gate, float *Mixed, int width, int streams, int n) {
    int i = item();
    if (i >= n) return;
    float v = 0.0f;
    for (int c = 0; c < streams; ++c) v = v + Norm[c * width + i] * sm::sigmoid(Gate[c * width + i]);
    Mixed[i] = v / (float)streams;
}
// kernels/strata.cu:278-281
__global__ void k_hc_write(float *Residual, const float *Output, const float *Inject, int width, int streams, int n) {
    int i = item();
    if (i >= n) return;
    Residual[i] = Residual[i] + Output[i % width] * (2.0f * sm::sigmoid(Inject[i / width] / (float)streams));
}

// kernels/strata.cu:287-295: one channel per lane; the channel's history
// shifts by one after the output is formed.
__global__ void k_conv(float *History, const float *X, const float *W, float *Y, int taps, int dilation,
                       int activation, int n) {
    int c = item();
    if (c >= n) return;
    int span = (taps - 1) * dilation;
    float *h = History + (int64_t)c * span;
    float sum = 0.0f;
    for (int t = 0; t < taps - 1; ++t) sum = sum + h[t * dilation] * W[c * taps + t];
    sum = sum + X[c] * W[c * taps + taps - 1];
    Y[c] = activation == 1 ? sm::silu(sum) : sum;
    for (int t = 0; t < span - 1; ++t) h[t] = h[t + 1];
    if (span > 0) h[span - 1] = X[c];
}

// kernels/strata.cu:296-302
__global__ void k_gdn_gates(const float *Alpha, const float *Beta, const float *A, const float *Dt, float *Decay,
                            float *Strength, int n) {
    int h = item();
    if (h >= n) return;
    float a = Alpha[h] + Dt[h];
    float sp = a > 20.0f ? a : sm::logf_or(1.0f + sm::expf_or(a));
    Decay[h] = sm::expf_or(A[h] * sp);
    Strength[h] = sm::sigmoid(Beta[h]);
}

// kernels/strata.cu:304-313: one (value head, value component) per lane;
// state [key dim][value head][value dim], so lanes of one key index read
// consecutive words.
__global__ void k_gdn_step(float *State, const float *Q, const float *K, const float *V, const float *Decay,
                           const float *Beta, float *Y, int dim, int keyHeads, int valueHeads, int n) {
    int jh = item();
    if (jh >= n) return;
    int h = jh / dim, kh = h % keyHeads, stride = valueHeads * dim;
    float decay = Decay[h], prediction = 0.0f;
    for (int i = 0; i < dim; ++i) {
        int ix = i * stride + jh;
        float s = State[ix] * decay;
        State[ix] = s;
        prediction = prediction + s * K[kh * dim + i];
    }
    float delta = (V[jh] - prediction) * Beta[h], result = 0.0f;
    for (int i = 0; i < dim; ++i) {
        int ix = i * stride + jh;
        float s = State[ix] + K[kh * dim + i] * delta;
        State[ix] = s;
        result = result + s * Q[kh * dim + i];
    }
    Y[jh] = result;
}

// kernels/strata.cu:314-316
__global__ void k_slice(const float *X, float *Y, int width, int stride, int offset, int n) {
    int i = item();
    if (i < n) Y[i] = X[(i / width) * stride + offset + i % width];
}
// kernels/strata.cu:328-330
__global__ void k_kv_append(const float *K, const float *V, float *Keys, float *Values, int width, int position,
                            int n) {
    int i = item();
    if (i >= n) return;
    Keys[position * width + i] = K[i];
    Values[position * width + i] = V[i];
}

// kernels/strata.cu:334-356: one 64-lane block per (head, 64-component
// tile). Lane-strided scores (sequential dot over the head dimension), the
// reference's maximum tree, exponentials with the lane-strided sum and its
// tree, then per component the sequential weighted sum over the cells.
__global__ __launch_bounds__(64) void k_attention(const float *Q, const float *Keys, const float *Values,
                                                  const int *Cells, float *Y, int dim, int heads, int kvHeads,
                                                  int count, float scale) {
    __shared__ float scores[2048];
    const int lane = threadIdx.x, h = blockIdx.x, d = blockIdx.y * 64 + lane;
    const int kh = h / (heads / kvHeads);
    const float *q = Q + h * dim;
    float mx = kNegBig;
    for (int t = lane; t < count; t += 64) {
        const float *k = Keys + (int64_t)(Cells[t] * kvHeads + kh) * dim;
        float score = 0.0f;
        for (int j = 0; j < dim; ++j) score = score + q[j] * k[j];
        score = score * scale;
        scores[t] = score;
        mx = fmaxf(mx, score);
    }
    for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_down(mx, s, 64));
    mx = __shfl(mx, 0, 64);
    float sum = 0.0f;
    for (int t = lane; t < count; t += 64) {
        float p = sm::expf_or(scores[t] - mx);
        scores[t] = p;
        sum = sum + p;
    }
    float total = __shfl(sm::tree_sum64(sum), 0, 64);
    __syncthreads();
    if (d >= dim) return;
    float value = 0.0f;
    for (int t = 0; t < count; ++t) value = value + scores[t] * Values[(int64_t)(Cells[t] * kvHeads + kh) * dim + d];
    Y[h * dim + d] = value / total;
}

// kernels/strata.cu:357-359
__global__ void k_attention_gate(const float *Attention, const float *FullQ, float *Y, int dim, int n) {
    int i = item();
    if (i < n) Y[i] = Attention[i] * sm::sigmoid(FullQ[(i / dim) * dim * 2 + dim + i % dim]);
}

// kernels/strata.cu:367-377: one 64-lane block per stream.
__global__ __launch_bounds__(64) void k_ple_gate(const float *Key, const float *Query, float *Gate, int width) {
    const int lane = threadIdx.x, c = blockIdx.x;
    float dot = 0.0f;
    for (int d = lane; d < width; d += 64) dot = dot + Key[c * width + d] * Query[c * width + d];
    dot = sm::tree_sum64(dot);
    if (lane != 0) return;
    float v = dot / sqrtf((float)width);
    float sign = v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
    Gate[c] = sm::sigmoid(sign * sqrtf(fmaxf(fabsf(v), 0.000001f)));
}
// kernels/strata.cu:378-380
__global__ void k_ple_broadcast(const float *Value, const float *Gate, float *Y, int width, int n) {
    int i = item();
    if (i < n) Y[i] = Value[i % width] * Gate[i / width];
}
// kernels/strata.cu:381-383
__global__ void k_ple_add(float *Residual, const float *Gated, const float *Conv, int n) {
    int i = item();
    if (i < n) Residual[i] = Residual[i] + (Gated[i] + Conv[i]);
}

// kernels/strata.cu:386-396: lane-strided best (lowest index on ties), then
// the reference's tree with the same rule.
__global__ __launch_bounds__(64) void k_argmax(const float *Logits, int *Token, int count) {
    const int lane = threadIdx.x;
    float best = kNegBig;
    int id = count;
    for (int i = lane; i < count; i += 64) {
        float v = Logits[i];
        if (v > best || (v == best && i < id)) {
            best = v;
            id = i;
        }
    }
    for (int s = 32; s > 0; s >>= 1) {
        float ov = __shfl_down(best, s, 64);
        int oi = __shfl_down(id, s, 64);
        if (lane < s && (ov > best || (ov == best && oi < id))) {
            best = ov;
            id = oi;
        }
    }
    if (lane == 0) Token[0] = id;
}

// kernels/strata.cu:81-89: IQ4_NL blocks of 18 bytes, an fp16 scale then 16
// bytes of 32 codes (low nibbles first).
__global__ void k_ple_decode(const uint32_t *Packed, float *Values, int n) {
    int i = item();
    if (i >= n) return;
    int block = i / 32, scaleByte = block * 18, codeByte = scaleByte + 2 + i % 16;
    uint32_t halfBits = (Packed[scaleByte / 4] >> ((scaleByte % 4) * 8)) & 65535u;
    int code = (int)((Packed[codeByte / 4] >> ((codeByte % 4) * 8 + (i % 32 < 16 ? 0 : 4))) & 15u);
    Values[i] = sm::half_bits(halfBits) * iq4_value(code);
}
// kernels/strata.cu:282-285
__global__ void k_embed(const float *Row, float *Residual, int width, int n) {
    int i = item();
    if (i < n) Residual[i] = Row[i % width];
}
// kernels/strata.cu:319-327
__global__ void k_rope(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int rotary, int n) {
    int i = item();
    if (i >= n) return;
    int d = i % dim, base = i - d;
    if (d >= rotary) {
        Y[i] = X[i];
        return;
    }
    int half = rotary / 2, pair = d % half;
    float a = X[base + pair], b = X[base + pair + half];
    Y[i] = d < half ? a * Cos[pair] - b * Sin[pair] : b * Cos[pair] + a * Sin[pair];
}

// ------------------------------------------------ prompt (batch) kernels
// kernels/strata.cu:399-402
__global__ void k_embed_batch(const float *Rows, float *Residual, int width, int hc, int n) {
    int i = item();
    if (i < n) Residual[i] = Rows[(i / hc) * width + i % width];
}
// kernels/strata.cu:403-408
__global__ void k_hc_mix_batch(const float *Norm, const float *Gate, float *Mixed, int width, int streams, int n) {
    int i = item();
    if (i >= n) return;
    int token = i / width, d = i % width;
    float v = 0.0f;
    for (int c = 0; c < streams; ++c) {
        int p = (token * streams + c) * width + d;
        v = v + Norm[p] * sm::sigmoid(Gate[p]);
    }
    Mixed[i] = v / (float)streams;
}
// kernels/strata.cu:409-412
__global__ void k_hc_write_batch(float *Residual, const float *Output, const float *Inject, int width, int streams,
                                 int n) {
    int i = item();
    if (i >= n) return;
    int hc = width * streams;
    Residual[i] = Residual[i] +
                  Output[(i / hc) * width + i % width] * (2.0f * sm::sigmoid(Inject[i / width] / (float)streams));
}
// kernels/strata.cu:413-424: one channel per lane, its tokens in order.
__global__ void k_conv_batch(float *History, const float *X, const float *W, float *Y, int channels, int taps,
                             int dilation, int activation, int tokens, int n) {
    int c = item();
    if (c >= n) return;
    int span = (taps - 1) * dilation;
    float *h = History + (int64_t)c * span;
    for (int token = 0; token < tokens; ++token) {
        float sum = 0.0f;
        for (int t = 0; t < taps - 1; ++t) sum = sum + h[t * dilation] * W[c * taps + t];
        const float x = X[token * channels + c];
        sum = sum + x * W[c * taps + taps - 1];
        Y[token * channels + c] = activation == 1 ? sm::silu(sum) : sum;
        for (int t = 0; t < span - 1; ++t) h[t] = h[t + 1];
        if (span > 0) h[span - 1] = x;
    }
}
// kernels/strata.cu:425-431
__global__ void k_gdn_gates_batch(const float *Alpha, const float *Beta, const float *A, const float *Dt,
                                  float *Decay, float *Strength, int heads, int n) {
    int i = item();
    if (i >= n) return;
    float x = Alpha[i] + Dt[i % heads];
    float sp = x > 20.0f ? x : sm::logf_or(1.0f + sm::expf_or(x));
    Decay[i] = sm::expf_or(A[i % heads] * sp);
    Strength[i] = sm::sigmoid(Beta[i]);
}
// kernels/strata.cu:432-445: one (value head, component) per lane, its tokens in order.
__global__ void k_gdn_batch(float *State, const float *Q, const float *K, const float *V, const float *Decay,
                            const float *Beta, float *Y, int dim, int keyHeads, int valueHeads, int tokens, int n) {
    int jh = item();
    if (jh >= n) return;
    int h = jh / dim, kh = h % keyHeads, stride = valueHeads * dim;
    for (int token = 0; token < tokens; ++token) {
        const int qbase = (token * keyHeads + kh) * dim, gh = token * valueHeads + h;
        const float decay = Decay[gh];
        float prediction = 0.0f;
        for (int i = 0; i < dim; ++i) {
            int ix = i * stride + jh;
            float s = State[ix] * decay;
            State[ix] = s;
            prediction = prediction + s * K[qbase + i];
        }
        float delta = (V[token * stride + jh] - prediction) * Beta[gh], result = 0.0f;
        for (int i = 0; i < dim; ++i) {
            int ix = i * stride + jh;
            float s = State[ix] + K[qbase + i] * delta;
            State[ix] = s;
            result = result + s * Q[qbase + i];
        }
        Y[token * stride + jh] = result;
    }
}
// kernels/strata.cu:446-453: token t rotated by table row t.
__global__ void k_rope_batch(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int heads,
                             int rotary, int n) {
    int i = item();
    if (i >= n) return;
    int d = i % dim;
    if (d >= rotary) {
        Y[i] = X[i];
        return;
    }
    int half = rotary / 2, pair = d % half, base = i - d, angle = (i / (dim * heads)) * half + pair;
    float a = X[base + pair], b = X[base + pair + half];
    Y[i] = d < half ? a * Cos[angle] - b * Sin[angle] : b * Cos[angle] + a * Sin[angle];
}
// kernels/strata.cu:454-457
__global__ void k_kv_append_batch(const float *K, const float *V, float *Keys, float *Values, int width, int position,
                                  int n) {
    int i = item();
    if (i >= n) return;
    Keys[position * width + i] = K[i];
    Values[position * width + i] = V[i];
}
// kernels/strata.cu:461-464
__global__ void k_ple_broadcast_batch(const float *Value, const float *Gate, float *Y, int width, int hc, int n) {
    int i = item();
    if (i < n) Y[i] = Value[(i / hc) * width + i % width] * Gate[i / width];
}
// The two longest prompt kernels with their memory round trips taken out and
// the reference's arithmetic unchanged:
//
// k_gdn_batch_reg: k_gdn_batch with the thread's state column (dim <= 128
// values) held in registers across the chunk's tokens instead of reread and
// rewritten in memory twice per token; the products and sums are the same
// operations in the same order, and the column is stored once at the end.
constexpr int GDN_REG_MAX_DIM = 128;
__global__ void __launch_bounds__(256) k_gdn_batch_reg(float *__restrict__ State, const float *__restrict__ Q,
                                                       const float *__restrict__ K, const float *__restrict__ V,
                                                       const float *__restrict__ Decay, const float *__restrict__ Beta,
                                                       float *__restrict__ Y, int dim, int keyHeads, int valueHeads,
                                                       int tokens, int n) {
    int jh = item();
    if (jh >= n) return;
    const int h = jh / dim, kh = h % keyHeads, stride = valueHeads * dim;
    float st[GDN_REG_MAX_DIM];
#pragma unroll
    for (int i = 0; i < GDN_REG_MAX_DIM; ++i)
        if (i < dim) st[i] = State[i * stride + jh];
    for (int token = 0; token < tokens; ++token) {
        const int qbase = (token * keyHeads + kh) * dim, gh = token * valueHeads + h;
        const float decay = Decay[gh];
        float prediction = 0.0f;
#pragma unroll
        for (int i = 0; i < GDN_REG_MAX_DIM; ++i)
            if (i < dim) {
                st[i] = st[i] * decay;
                prediction = prediction + st[i] * K[qbase + i];
            }
        const float delta = (V[token * stride + jh] - prediction) * Beta[gh];
        float result = 0.0f;
#pragma unroll
        for (int i = 0; i < GDN_REG_MAX_DIM; ++i)
            if (i < dim) {
                st[i] = st[i] + K[qbase + i] * delta;
                result = result + st[i] * Q[qbase + i];
            }
        Y[token * stride + jh] = result;
    }
#pragma unroll
    for (int i = 0; i < GDN_REG_MAX_DIM; ++i)
        if (i < dim) State[i * stride + jh] = st[i];
}

// k_attention_batch4 (kernels/strata.cu:512-534: cells 0 .. position + t for
// prompt token t): one 256-thread block per (head, token) and four
// 64-component tiles. The reference's 64-lane blocks of one (head, token)
// all compute the same scores; here the four waves compute each score once
// (cell t by wave (t / 64) % 4, same sequential dot over the head
// dimension, loads issued eight at a time), then every wave forms the
// maximum, the exponentials and their sum in the reference's lane order
// (lane l: cells l, l + 64, ...; the same trees) and each wave runs the
// weighted sum of its own tile, sequential over the cells.
__global__ __launch_bounds__(256) void k_attention_batch4(const float *__restrict__ Q, const float *__restrict__ Keys,
                                                          const float *__restrict__ Values, float *__restrict__ Y,
                                                          int dim, int heads, int kvHeads, int position, float scale,
                                                          int tiles) {
    __shared__ float s_score[2048], s_prob[2048];
    const int token = blockIdx.z, count = position + token + 1, h = blockIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, kh = h / (heads / kvHeads);
    const float *q = Q + (int64_t)(token * heads + h) * dim;
    for (int t = threadIdx.x; t < count; t += 256) {
        const float *k = Keys + (int64_t)(t * kvHeads + kh) * dim;
        float score = 0.0f;
        for (int j0 = 0; j0 < dim; j0 += 8) {
            float kv[8], qv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = min(j0 + u, dim - 1);
                kv[u] = k[j];
                qv[u] = q[j];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (j0 + u < dim) score = score + qv[u] * kv[u];
        }
        s_score[t] = score * scale;
    }
    __syncthreads();
    float mx = kNegBig;
    for (int t = lane; t < count; t += 64) mx = fmaxf(mx, s_score[t]);
    for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_down(mx, s, 64));
    mx = __shfl(mx, 0, 64);
    float sum = 0.0f;
    for (int t = lane; t < count; t += 64) {
        const float p = sm::expf_or(s_score[t] - mx);
        if (w == 0) s_prob[t] = p;
        sum = sum + p;
    }
    const float total = __shfl(sm::tree_sum64(sum), 0, 64);
    __syncthreads();
    const int tile = blockIdx.y * 4 + w, d = tile * 64 + lane;
    if (tile >= tiles || d >= dim) return;
    float value = 0.0f;
    for (int t0 = 0; t0 < count; t0 += 8) {
        float vv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) vv[u] = Values[(int64_t)(min(t0 + u, count - 1) * kvHeads + kh) * dim + d];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (t0 + u < count) value = value + s_prob[t0 + u] * vv[u];
    }
    Y[(int64_t)(token * heads + h) * dim + d] = value / total;
}

// The batched prompt attention in two launches, the same operations in the
// same order as k_attention_batch4 (kernels/strata.cu:512-534), with the
// work spread over the GPU:
//  k_attn_scores: one block per (64-cell tile, KV head, token). The tile's
//    keys (64 rows) go to LDS with 16-byte loads, the query rows of the KV
//    head's query heads too; lane l of wave w forms cell c0 + l's score for
//    query heads w, w + 4, ... (HPW of them side by side, each the
//    sequential dot over the head dimension), times `scale`, into
//    S[token][head][cell].
//  k_attn_values: below.
// A row of keys in LDS is padded by 4 floats so that the 64 lanes' 16-byte
// reads of one offset spread over the banks.
template <int D, int HPW>
__global__ __launch_bounds__(256) void k_attn_scores(const float *__restrict__ Q, const float *__restrict__ Keys,
                                                     float *__restrict__ S, int heads, int kvHeads, int position,
                                                     float scale, int hu) {
    constexpr int P = D + 4;
    __shared__ __attribute__((aligned(16))) float s_k[64 * P];
    __shared__ __attribute__((aligned(16))) float s_q[4 * HPW][D];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int token = blockIdx.z, kh = blockIdx.y, c0 = blockIdx.x * 64, count = position + token + 1;
    if (c0 >= count) return;
    const int group = heads / kvHeads, h0 = kh * group;
    for (int idx = tid; idx < 64 * (D / 4); idx += 256) {
        const int r = idx / (D / 4), i4 = idx - r * (D / 4), cell = min(c0 + r, count - 1);
        *(float4 *)&s_k[r * P + 4 * i4] = ((const float4 *)(Keys + ((int64_t)cell * kvHeads + kh) * D))[i4];
    }
    for (int idx = tid; idx < group * (D / 4); idx += 256) {
        const int g = idx / (D / 4), i4 = idx - g * (D / 4);
        *(float4 *)&s_q[g][4 * i4] = ((const float4 *)(Q + ((int64_t)token * heads + h0 + g) * D))[i4];
    }
    __syncthreads();
    float score[HPW];
#pragma unroll
    for (int u = 0; u < HPW; u++) score[u] = 0.0f;
    const float *kr = &s_k[lane * P];
    for (int j = 0; j < D; j += 4) {
        const float4 k4 = *(const float4 *)&kr[j];
#pragma unroll
        for (int u = 0; u < HPW; u++) {
            const int g = min(w + 4 * u, group - 1);
            const float4 q4 = *(const float4 *)&s_q[g][j];
            float v = score[u];
            v = v + q4.x * k4.x;
            v = v + q4.y * k4.y;
            v = v + q4.z * k4.z;
            v = v + q4.w * k4.w;
            score[u] = v;
        }
    }
    const int cell = c0 + lane;
#pragma unroll
    for (int u = 0; u < HPW; u++) {
        const int g = w + 4 * u, h = h0 + g;
        if (g < group && h < hu && cell < count) S[((int64_t)token * heads + h) * 2048 + cell] = score[u] * scale;
    }
}

// k_attn_values: one block per (64-component tile, group of up to HPW query
// heads of one KV head, token); wave w handles head w of the group. First
// the reference's softmax of its scores: the maximum, the exponentials and
// their sum in the reference's lane order (lane l: cells l, l + 64, ...; the
// tree), the probabilities in LDS. Then the weighted sum over the cells of
// the tile's 64 components: the block's waves share the values, staged
// through LDS 16 HPW cells at a time by all threads (double-buffered: the
// next chunk's loads are in flight while this one is summed, and the
// barriers order LDS only, so they do not wait for them); each lane's sum
// runs over the cells in order.
template <int D, int HPW>
__global__ __launch_bounds__(64 * HPW) void k_attn_values(const float *__restrict__ S, const float *__restrict__ Values,
                                                         float *__restrict__ Y, int heads, int kvHeads, int position,
                                                         int hu, int tiles) {
    constexpr int CH = 16 * HPW;  // cells per chunk: four 16-byte loads per thread
    __shared__ __attribute__((aligned(16))) float s_p[HPW][2048];
    __shared__ __attribute__((aligned(16))) float s_v[2][CH][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int token = blockIdx.z, count = position + token + 1, group = heads / kvHeads;
    const int groups_per_kv = (group + HPW - 1) / HPW;
    const int kh = blockIdx.y / groups_per_kv, g = (blockIdx.y - kh * groups_per_kv) * HPW + w;
    const int h = kh * group + g;
    const bool live = g < group && h < hu;
    // (all 32 of the lane's scores loaded at once, clamped past the count)
    const float *sc = S + ((int64_t)token * heads + min(h, heads - 1)) * 2048;
    float sv[32];
#pragma unroll
    for (int i = 0; i < 32; i++) sv[i] = sc[min(lane + 64 * i, count - 1)];
    float mx = kNegBig;
#pragma unroll
    for (int i = 0; i < 32; i++)
        if (lane + 64 * i < count) mx = fmaxf(mx, sv[i]);
    for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_down(mx, s, 64));
    mx = __shfl(mx, 0, 64);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        if (lane + 64 * i < count) {
            const float p = sm::expf_or(sv[i] - mx);
            s_p[w][lane + 64 * i] = p;
            sum = sum + p;
        }
    }
    const float total = __shfl(sm::tree_sum64(sum), 0, 64);
    const int d = blockIdx.x * 64 + lane;
    const int64_t vstride = (int64_t)kvHeads * D;
    const float *vtile = Values + (int64_t)kh * D + blockIdx.x * 64;
    const int nch = (count + CH - 1) / CH;
    // (four named registers, not an array: the compiler can place a small
    // private array in LDS, and then waits for the loads at once)
    const int row = threadIdx.x / 16, col = 4 * (threadIdx.x & 15);  // 16 threads per cell row
    constexpr int RS = 4 * HPW;  // cell rows between a thread's four loads
    auto vload = [&](int cell) -> float4 {
        return *(const float4 *)(vtile + (int64_t)min(cell, count - 1) * vstride + col);
    };
    float4 l0 = vload(row), l1 = vload(row + RS), l2 = vload(row + 2 * RS), l3 = vload(row + 3 * RS);
    *(float4 *)&s_v[0][row][col] = l0;
    *(float4 *)&s_v[0][row + RS][col] = l1;
    *(float4 *)&s_v[0][row + 2 * RS][col] = l2;
    *(float4 *)&s_v[0][row + 3 * RS][col] = l3;
    float value = 0.0f;
    for (int c = 0; c < nch; c++) {
        if (c + 1 < nch) {
            const int c1 = (c + 1) * CH + row;
            l0 = vload(c1);
            l1 = vload(c1 + RS);
            l2 = vload(c1 + 2 * RS);
            l3 = vload(c1 + 3 * RS);
        }
        // (the next chunk's loads are issued here, not sunk to their use)
        asm volatile("" ::: "memory");
        sm::lds_barrier();  // chunk c is in LDS (and the probabilities); chunk c - 1's buffer is free
        const int t0 = c * CH, n = min(CH, count - t0), buf = c & 1;
        // 16 cells at a time: their values and probabilities read from LDS
        // into registers, then the 16 steps of the sum
        for (int gg = 0; gg < n; gg += 16) {
            float vv[16], pp[16];
#pragma unroll
            for (int u = 0; u < 16; u++) vv[u] = s_v[buf][min(gg + u, CH - 1)][lane];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 p4 = *(const float4 *)&s_p[w][min(t0 + gg + 4 * i, 2044)];
                pp[4 * i] = p4.x;
                pp[4 * i + 1] = p4.y;
                pp[4 * i + 2] = p4.z;
                pp[4 * i + 3] = p4.w;
            }
            if (gg + 16 <= n) {
#pragma unroll
                for (int u = 0; u < 16; u++) value = value + pp[u] * vv[u];
            } else {
                for (int u = 0; u < n - gg; u++) {
                    float a = pp[0], b = vv[0];
#pragma unroll
                    for (int i = 1; i < 16; i++) {
                        a = u == i ? pp[i] : a;
                        b = u == i ? vv[i] : b;
                    }
                    value = value + a * b;
                }
            }
        }
        // the next chunk goes to LDS only after this one is summed (its loads
        // were in flight meanwhile)
        asm volatile("" ::: "memory");
        if (c + 1 < nch) {
            const int nb = (c + 1) & 1;
            *(float4 *)&s_v[nb][row][col] = l0;
            *(float4 *)&s_v[nb][row + RS][col] = l1;
            *(float4 *)&s_v[nb][row + 2 * RS][col] = l2;
            *(float4 *)&s_v[nb][row + 3 * RS][col] = l3;
        }
    }
    if (live && blockIdx.x < (unsigned)tiles && d < D) Y[((int64_t)token * heads + h) * D + d] = value / total;
}

// k_gdn_batch_reg with the key and query rows of the block's key head staged
// in LDS (16 tokens at a time) and one 64-thread block per 64 state columns
// (all of one value head: D is a multiple of 64), so that each of the
// column's two sequential sums per token reads its K / Q values from LDS
// instead of waiting on global loads, and the columns spread over the CUs.
// The K / Q rows arrive by DMA, Decay and Beta of the staged tokens with
// them, and each token's V value one token ahead. The same operations in the
// same order as the reference (kernels/strata.cu:432-445). At the
// production shape (6,144 columns: 96 waves) each wave runs two dependent
// 128-step sums per token; the kernel is bound by that latency.
constexpr int kGdnStage = 16;
// 16 bytes per lane from global memory into LDS (lane l's at base + 16 l).
__device__ __forceinline__ void gdn_dma16(const void *src, void *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
}
template <int D>
__global__ void __launch_bounds__(64) k_gdn_batch_lds(float *__restrict__ State, const float *__restrict__ Q,
                                                      const float *__restrict__ K, const float *__restrict__ V,
                                                      const float *__restrict__ Decay, const float *__restrict__ Beta,
                                                      float *__restrict__ Y, int keyHeads, int valueHeads, int tokens,
                                                      int n) {
    static_assert(D % 64 == 0 && D <= GDN_REG_MAX_DIM, "whole value heads per block group");
    __shared__ __attribute__((aligned(16))) float s_k[kGdnStage][D], s_q[kGdnStage][D];
    __shared__ float s_decay[kGdnStage], s_beta[kGdnStage];
    const int jh = blockIdx.x * 64 + threadIdx.x;
    const int h = (int)(blockIdx.x * 64) / D, kh = h % keyHeads, stride = valueHeads * D;
    const bool live = jh < n;
    const int col = min(jh, n - 1);
    float st[D];
#pragma unroll
    for (int i = 0; i < D; ++i) st[i] = State[(int64_t)i * stride + col];
    for (int t0 = 0; t0 < tokens; t0 += kGdnStage) {
        const int nt = min(kGdnStage, tokens - t0);
        __syncthreads();  // the previous stage's readers are done
        // K and Q rows of the stage's tokens by DMA into LDS (16 bytes per
        // lane, a kilobyte per instruction: 1,024 / (4 D) rows; rows past
        // the stage's tokens reload its last token and are never read)
        constexpr int RPI = 256 / D;  // rows per instruction
        const int lr = threadIdx.x / (D / 4), lo = 4 * (threadIdx.x % (D / 4));
#pragma unroll
        for (int i = 0; i < kGdnStage / RPI; i++) {
            const int tt = min(RPI * i + lr, nt - 1);
            const int64_t qbase = ((int64_t)(t0 + tt) * keyHeads + kh) * D + lo;
            gdn_dma16(K + qbase, &s_k[RPI * i][0]);
            gdn_dma16(Q + qbase, &s_q[RPI * i][0]);
        }
        if (threadIdx.x < nt) {
            s_decay[threadIdx.x] = Decay[(t0 + threadIdx.x) * valueHeads + h];
            s_beta[threadIdx.x] = Beta[(t0 + threadIdx.x) * valueHeads + h];
        }
        __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));  // vmcnt(0): the DMA is in LDS
        __syncthreads();
        // the token's V value, loaded one token ahead (one register, not a
        // register per staged token)
        float vnext = V[(int64_t)t0 * stride + col];
        for (int tt = 0; tt < nt; tt++) {
            const float vt = vnext;
            vnext = V[(int64_t)(t0 + min(tt + 1, nt - 1)) * stride + col];
            const float decay = s_decay[tt];
            float prediction = 0.0f;
#pragma unroll
            for (int i = 0; i < D; ++i) {
                st[i] = st[i] * decay;
                prediction = prediction + st[i] * s_k[tt][i];
            }
            const float delta = (vt - prediction) * s_beta[tt];
            float result = 0.0f;
#pragma unroll
            for (int i = 0; i < D; ++i) {
                st[i] = st[i] + s_k[tt][i] * delta;
                result = result + st[i] * s_q[tt][i];
            }
            if (live) Y[(int64_t)(t0 + tt) * stride + jh] = result;
        }
    }
    if (live) {
#pragma unroll
        for (int i = 0; i < D; ++i) State[(int64_t)i * stride + jh] = st[i];
    }
}

// ------------------------------------------------------------- launchers
int bad(sm_ctx *ctx, const std::string &m) { return fail(ctx, SM_E_ARG, m); }
unsigned blocks256(int64_t n) { return (unsigned)((n + 255) / 256); }
// Items a 64-lane grid of G[0] workgroups covers.
int64_t covered(const uint32_t *G, int64_t n) { return std::min<int64_t>(n, (int64_t)G[0] * 64); }
const float *F(Args a, int i) { return (const float *)a.ptr(i); }
float *Fw(Args a, int i) { return (float *)a.ptr(i); }

int L_embedding(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(5), streams = a.i32(6), off = a.i32(7), format = a.i32(8), bits = a.i32(9), group = a.i32(10);
    int bias = a.i32(11), codebook = a.i32(12), hasOffset = a.i32(13);
    if (width < 1 || streams < 1) return bad(ctx, "strata_embedding: width and streams must be >= 1");
    if (off < 0) return bad(ctx, "embedding output offset must be >= 0");
    int64_t rlen = buf_len(ctx, a.ptr(4));
    if (format < 0 || format > 2 || (rlen >= 0 && off + (int64_t)width * streams > rlen / 4))
        return fail(ctx, SM_E_ARG, "Embedding exceeds buffer layout");
    if (format == 2 && ((bits != 2 && bits != 4 && bits != 8) || group < 1 || width % group))
        return fail(ctx, SM_E_ARG, "Invalid packed embedding layout");
    int64_t n = covered(G, width);
    if (int rc = need(ctx, a.ptr(4), (uint64_t)(off + (int64_t)(streams - 1) * width + n) * 4, "Residual")) return rc;
    if (format == 0) {
        if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "Values")) return rc;
    } else if (format == 1) {
        if (int rc = need(ctx, a.ptr(1), (uint64_t)(n + 1) / 2 * 4, "Codes")) return rc;
    } else {
        if (int rc = need(ctx, a.ptr(1), (uint64_t)(n * bits + 31) / 32 * 4, "Codes")) return rc;
        uint64_t groups = (uint64_t)((n - 1) / group + 1);
        if (int rc = need(ctx, a.ptr(2), groups * 4, "Scales")) return rc;
        if (hasOffset)
            if (int rc = need(ctx, a.ptr(3), groups * 4, "Offsets")) return rc;
    }
    k_embedding<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), (const uint32_t *)a.ptr(1), F(a, 2), F(a, 3), Fw(a, 4),
                                                       width, streams, off, format, bits, group, bias, codebook,
                                                       hasOffset, (int)n);
    return launched(ctx);
}

int L_rope_frequencies(sm_ctx *ctx, const uint32_t *G, Args a) {
    int rotary = a.i32(2);
    float base = a.f32(3);
    if (!std::isfinite(base) || base <= 1.0f || rotary < 1 || rotary % 2)
        return fail(ctx, SM_E_ARG, "Invalid RoPE frequencies");
    int64_t n = covered(G, rotary / 2);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "High")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "Low")) return rc;
    k_rope_frequencies<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), Fw(a, 1), rotary, base, (int)n);
    return launched(ctx);
}

int L_rope_table(sm_ctx *ctx, const uint32_t *G, Args a) {
    int rotary = a.i32(4), context = a.i32(5);
    if (rotary < 2 || rotary % 2 || context < 1) return bad(ctx, "strata_rope_table: rotary >= 2 even, context >= 1");
    int half = rotary / 2;
    int64_t n = covered(G, (int64_t)context * half);
    uint64_t pairs = (uint64_t)std::min<int64_t>(n, half);
    if (int rc = need(ctx, a.ptr(0), pairs * 4, "High")) return rc;
    if (int rc = need(ctx, a.ptr(1), pairs * 4, "Low")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Cos")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)n * 4, "Sin")) return rc;
    k_rope_table<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), Fw(a, 3), half, (int)n);
    return launched(ctx);
}

int L_rope_position(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(4), heads = a.i32(5), rotary = a.i32(6), position = a.i32(7), tokens = a.i32(8);
    if (position < 0 || position > 2047) return bad(ctx, "RoPE position must be an integer in [0, 2047]");
    if (dim < 1 || heads < 1 || rotary < 1 || tokens < 1)
        return bad(ctx, "strata_rope_position: dim, heads, rotary, tokens must be >= 1");
    int64_t xlen = buf_len(ctx, a.ptr(0)), clen = buf_len(ctx, a.ptr(1)), slen = buf_len(ctx, a.ptr(2)),
            ylen = buf_len(ctx, a.ptr(3)), total = (int64_t)dim * heads * tokens;
    if (rotary % 2 || rotary > dim || position + tokens > 2048 || clen < (int64_t)(position + tokens) * rotary / 2 * 4 ||
        slen != clen || xlen != total * 4 || ylen != xlen)
        return fail(ctx, SM_E_ARG, "Invalid RoPE layout");
    int64_t n = covered(G, total);
    k_rope_position<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), Fw(a, 3), dim, heads, rotary,
                                                           position, (int)n);
    return launched(ctx);
}

int L_hc_mix(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4);
    if (width < 1 || streams < 1) return bad(ctx, "strata_hc_mix: width and streams must be >= 1");
    int64_t n = covered(G, width);
    uint64_t span = (uint64_t)((int64_t)(streams - 1) * width + n) * 4;
    if (int rc = need(ctx, a.ptr(0), span, "Norm")) return rc;
    if (int rc = need(ctx, a.ptr(1), span, "Gate")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Mixed")) return rc;
    k_hc_mix<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), width, streams, (int)n);
    return launched(ctx);
}

int L_hc_write(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4);
    if (width < 1 || streams < 1) return bad(ctx, "strata_hc_write: width and streams must be >= 1");
    int64_t n = covered(G, (int64_t)width * streams);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "Residual")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)std::min<int64_t>(n, width) * 4, "Output")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)((n - 1) / width + 1) * 4, "Inject")) return rc;
    k_hc_write<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), width, streams, (int)n);
    return launched(ctx);
}

int L_conv(sm_ctx *ctx, const uint32_t *G, Args a) {
    int channels = a.i32(4), taps = a.i32(5), dilation = a.i32(6), activation = a.i32(7);
    if (channels < 1 || taps < 1 || dilation < 1)
        return bad(ctx, "strata_conv: channels, taps and dilation must be >= 1");
    int64_t n = covered(G, channels), span = (int64_t)(taps - 1) * dilation;
    if (span > 0)
        if (int rc = need(ctx, a.ptr(0), (uint64_t)(n * span) * 4, "History")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "X")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)(n * taps) * 4, "W")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)n * 4, "Y")) return rc;
    k_conv<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), Fw(a, 3), taps, dilation, activation,
                                                  (int)n);
    return launched(ctx);
}

int L_gdn_gates(sm_ctx *ctx, const uint32_t *G, Args a) {
    int heads = a.i32(6);
    if (heads < 1) return bad(ctx, "strata_gdn_gates: heads must be >= 1");
    int64_t n = covered(G, heads);
    const char *names[6] = {"Alpha", "Beta", "A", "Dt", "Decay", "Strength"};
    for (int i = 0; i < 6; i++)
        if (int rc = need(ctx, a.ptr(i), (uint64_t)n * 4, names[i])) return rc;
    k_gdn_gates<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), F(a, 3), Fw(a, 4), Fw(a, 5),
                                                       (int)n);
    return launched(ctx);
}

int L_gdn_step(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(7), keyHeads = a.i32(8), valueHeads = a.i32(9);
    if (dim < 1 || keyHeads < 1 || valueHeads < 1)
        return bad(ctx, "strata_gdn_step: dim, keyHeads, valueHeads must be >= 1");
    int64_t n = covered(G, (int64_t)dim * valueHeads), heads = (n - 1) / dim + 1;
    int64_t keyRows = std::min<int64_t>(keyHeads, heads);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)((int64_t)(dim - 1) * valueHeads * dim + n) * 4, "State")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)(keyRows * dim) * 4, "Q")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)(keyRows * dim) * 4, "K")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)n * 4, "V")) return rc;
    if (int rc = need(ctx, a.ptr(4), (uint64_t)heads * 4, "Decay")) return rc;
    if (int rc = need(ctx, a.ptr(5), (uint64_t)heads * 4, "Beta")) return rc;
    if (int rc = need(ctx, a.ptr(6), (uint64_t)n * 4, "Y")) return rc;
    k_gdn_step<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), F(a, 3), F(a, 4), F(a, 5), Fw(a, 6),
                                                      dim, keyHeads, valueHeads, (int)n);
    return launched(ctx);
}

int L_slice(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(2), rows = a.i32(3), stride = a.i32(4), offset = a.i32(5);
    if (width < 1 || rows < 1) return bad(ctx, "slice width and rows must be >= 1");
    if (stride < 0 || offset < 0) return bad(ctx, "strata_slice: stride and offset must be >= 0");
    int64_t n = covered(G, (int64_t)width * rows), last = n - 1;
    // Largest source index: the last item, or the end of the row before it.
    int64_t top = (last / width) * stride + offset + last % width;
    if (last >= width) top = std::max<int64_t>(top, (last / width - 1) * stride + offset + width - 1);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)(top + 1) * 4, "X")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "Y")) return rc;
    k_slice<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), Fw(a, 1), width, stride, offset, (int)n);
    return launched(ctx);
}

int L_kv_append(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(4), position = a.i32(5);
    if (width < 1 || position < 0) return bad(ctx, "strata_kv_append: width >= 1 and position >= 0");
    int64_t n = covered(G, width);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "K")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "V")) return rc;
    uint64_t end = (uint64_t)((int64_t)position * width + n) * 4;
    if (int rc = need(ctx, a.ptr(2), end, "Keys")) return rc;
    if (int rc = need(ctx, a.ptr(3), end, "Values")) return rc;
    k_kv_append<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), Fw(a, 3), width, position, (int)n);
    return launched(ctx);
}

int L_attention(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(5), heads = a.i32(6), kvHeads = a.i32(7), count = a.i32(8);
    float scale = a.f32(9);
    if (dim < 1 || heads < 1 || kvHeads < 1) return bad(ctx, "strata_attention: dim, heads, kvHeads must be >= 1");
    if (heads % kvHeads) return bad(ctx, "Attention heads must be divisible by KV heads");
    if (count < 1 || count > 2048) return bad(ctx, "attention selected cells must be an integer in [1, 2048]");
    int hu = (int)std::min<int64_t>(G[0], heads), tiles = (int)std::min<int64_t>(G[1], (dim + 63) / 64);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)hu * dim * 4, "Q")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)count * 4, "Cells")) return rc;
    int64_t written = (int64_t)(hu - 1) * dim + std::min<int64_t>(dim, (int64_t)tiles * 64);
    if (int rc = need(ctx, a.ptr(4), (uint64_t)written * 4, "Y")) return rc;
    // Cells index rows of kvHeads * dim values in Keys and Values.
    int64_t klen = buf_len(ctx, a.ptr(1)), vlen = buf_len(ctx, a.ptr(2));
    if (klen < 0) return need(ctx, a.ptr(1), 0, "Keys");
    if (vlen < 0) return need(ctx, a.ptr(2), 0, "Values");
    int64_t rowsAvail = std::min(klen, vlen) / 4 / ((int64_t)kvHeads * dim);
    if (int rc = check_indices(ctx, a.ptr(3), count, 1, 0, 0, (int)std::min<int64_t>(rowsAvail, 0x7fffffff),
                               "Attention cells"))
        return rc;
    k_attention<<<dim3(hu, tiles), 64, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), (const int *)a.ptr(3), Fw(a, 4),
                                                          dim, heads, kvHeads, count, scale);
    return launched(ctx);
}

int L_attention_gate(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(3), heads = a.i32(4);
    if (dim < 1 || heads < 1) return bad(ctx, "strata_attention_gate: dim and heads must be >= 1");
    int64_t n = covered(G, (int64_t)dim * heads), last = n - 1;
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "Attention")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)((last / dim) * dim * 2 + dim + last % dim + 1) * 4, "FullQ"))
        return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Y")) return rc;
    k_attention_gate<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), dim, (int)n);
    return launched(ctx);
}

int L_ple_gate(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4);
    if (width < 1 || streams < 1) return bad(ctx, "strata_ple_gate: width and streams must be >= 1");
    int cu = (int)std::min<int64_t>(G[0], streams);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)cu * width * 4, "Key")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)cu * width * 4, "Query")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)cu * 4, "Gate")) return rc;
    k_ple_gate<<<cu, 64, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), width);
    return launched(ctx);
}

int L_ple_broadcast(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4);
    if (width < 1 || streams < 1) return bad(ctx, "strata_ple_broadcast: width and streams must be >= 1");
    int64_t n = covered(G, (int64_t)width * streams);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)std::min<int64_t>(n, width) * 4, "Value")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)((n - 1) / width + 1) * 4, "Gate")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Y")) return rc;
    k_ple_broadcast<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), width, (int)n);
    return launched(ctx);
}

int L_ple_add(sm_ctx *ctx, const uint32_t *G, Args a) {
    int count = a.i32(3);
    if (count < 0) return bad(ctx, "strata_ple_add: n must be >= 0");
    int64_t n = covered(G, count);
    if (n == 0) return SM_OK;
    const char *names[3] = {"Residual", "Gated", "Conv"};
    for (int i = 0; i < 3; i++)
        if (int rc = need(ctx, a.ptr(i), (uint64_t)n * 4, names[i])) return rc;
    k_ple_add<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), (int)n);
    return launched(ctx);
}

int L_argmax(sm_ctx *ctx, const uint32_t *G, Args a) {
    int count = a.i32(2);
    if (count < 0) return bad(ctx, "strata_argmax: count must be >= 0");
    if (int rc = need(ctx, a.ptr(0), (uint64_t)count * 4, "Logits")) return rc;
    if (int rc = need(ctx, a.ptr(1), 4, "Token")) return rc;
    // Every workgroup of the reference computes the same winner; one suffices.
    k_argmax<<<1, 64, 0, ctx->stream>>>(F(a, 0), (int *)a.ptr(1), count);
    return launched(ctx);
}

int L_ple_decode(sm_ctx *ctx, const uint32_t *G, Args a) {
    int count = a.i32(2);
    int64_t plen = buf_len(ctx, a.ptr(0)), vlen = buf_len(ctx, a.ptr(1));
    if (count < 1) return bad(ctx, "strata_ple_decode.count must be an integer in [1, 2147483647]");
    if (count % 32 || (plen >= 0 && ((int64_t)count / 32 * 18 + 3) / 4 * 4 > plen) || (vlen >= 0 && count * 4LL > vlen))
        return fail(ctx, SM_E_ARG, "Invalid packed PLE layout");
    int64_t n = covered(G, count);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)(((n - 1) / 32 * 18 + 18 + 3) / 4 * 4), "Packed")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "Values")) return rc;
    k_ple_decode<<<blocks256(n), 256, 0, ctx->stream>>>((const uint32_t *)a.ptr(0), Fw(a, 1), (int)n);
    return launched(ctx);
}

int L_embed(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(2), streams = a.i32(3);
    if (width < 1 || streams < 1) return bad(ctx, "strata_embed: width and streams must be >= 1");
    int64_t n = covered(G, (int64_t)width * streams);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)std::min<int64_t>(n, width) * 4, "Row")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "Residual")) return rc;
    k_embed<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), Fw(a, 1), width, (int)n);
    return launched(ctx);
}

int L_rope(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(4), heads = a.i32(5), rotary = a.i32(6);
    if (dim < 1 || heads < 1 || rotary < 1) return bad(ctx, "strata_rope: dim, heads, rotary must be >= 1");
    if (rotary % 2 || rotary > dim) return bad(ctx, "Rotary width must be even and <= head dimension");
    int64_t n = covered(G, (int64_t)dim * heads);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)((n - 1) / dim + 1) * dim * 4, "X")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)(rotary / 2) * 4, "Cos")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)(rotary / 2) * 4, "Sin")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)n * 4, "Y")) return rc;
    k_rope<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), Fw(a, 3), dim, rotary, (int)n);
    return launched(ctx);
}

// Largest index + 1 of Rows[(i / hc) * width + i % width] over i < n.
int64_t row_span(int64_t n, int width, int64_t hc) {
    const int64_t tl = (n - 1) / hc;
    return tl * width + std::min<int64_t>(width, n - tl * hc);
}

int L_embed_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(2), streams = a.i32(3), tokens = a.i32(4);
    if (width < 1 || streams < 1 || tokens < 1) return bad(ctx, "strata_embed_batch: width, streams, tokens >= 1");
    const int64_t hc = (int64_t)width * streams, n = covered(G, hc * tokens);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)row_span(n, width, hc) * 4, "Rows")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "Residual")) return rc;
    k_embed_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), Fw(a, 1), width, (int)hc, (int)n);
    return launched(ctx);
}

int L_hc_mix_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4), tokens = a.i32(5);
    if (width < 1 || streams < 1 || tokens < 1) return bad(ctx, "strata_hc_mix_batch: width, streams, tokens >= 1");
    const int64_t n = covered(G, (int64_t)width * tokens), tl = (n - 1) / width;
    const uint64_t span = (uint64_t)((tl * streams + streams - 1) * width + (n - tl * width)) * 4;
    if (int rc = need(ctx, a.ptr(0), span, "Norm")) return rc;
    if (int rc = need(ctx, a.ptr(1), span, "Gate")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Mixed")) return rc;
    k_hc_mix_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), width, streams, (int)n);
    return launched(ctx);
}

int L_hc_write_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4), tokens = a.i32(5);
    if (width < 1 || streams < 1 || tokens < 1) return bad(ctx, "strata_hc_write_batch: width, streams, tokens >= 1");
    const int64_t hc = (int64_t)width * streams, n = covered(G, hc * tokens);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "Residual")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)row_span(n, width, hc) * 4, "Output")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)((n - 1) / width + 1) * 4, "Inject")) return rc;
    k_hc_write_batch<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), width, streams, (int)n);
    return launched(ctx);
}

int L_conv_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int channels = a.i32(4), taps = a.i32(5), dilation = a.i32(6), activation = a.i32(7), tokens = a.i32(8);
    if (channels < 1 || taps < 1 || dilation < 1 || tokens < 1)
        return bad(ctx, "strata_conv_batch: channels, taps, dilation and tokens must be >= 1");
    const int64_t n = covered(G, channels), span = (int64_t)(taps - 1) * dilation;
    const uint64_t xy = (uint64_t)((int64_t)(tokens - 1) * channels + n) * 4;
    if (span > 0)
        if (int rc = need(ctx, a.ptr(0), (uint64_t)(n * span) * 4, "History")) return rc;
    if (int rc = need(ctx, a.ptr(1), xy, "X")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)(n * taps) * 4, "W")) return rc;
    if (int rc = need(ctx, a.ptr(3), xy, "Y")) return rc;
    k_conv_batch<<<blocks256(n), 256, 0, ctx->stream>>>(Fw(a, 0), F(a, 1), F(a, 2), Fw(a, 3), channels, taps, dilation,
                                                        activation, tokens, (int)n);
    return launched(ctx);
}

int L_gdn_gates_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int heads = a.i32(6), tokens = a.i32(7);
    if (heads < 1 || tokens < 1) return bad(ctx, "strata_gdn_gates_batch: heads and tokens must be >= 1");
    const int64_t n = covered(G, (int64_t)heads * tokens), per = std::min<int64_t>(n, heads);
    const int idx[6] = {0, 1, 2, 3, 4, 5};
    const char *names[6] = {"Alpha", "Beta", "A", "Dt", "Decay", "Strength"};
    for (int i : idx)
        if (int rc = need(ctx, a.ptr(i), (uint64_t)(i == 2 || i == 3 ? per : n) * 4, names[i])) return rc;
    k_gdn_gates_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), F(a, 3), Fw(a, 4), Fw(a, 5),
                                                             heads, (int)n);
    return launched(ctx);
}

int L_gdn_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(7), keyHeads = a.i32(8), valueHeads = a.i32(9), tokens = a.i32(10);
    if (dim < 1 || keyHeads < 1 || valueHeads < 1 || tokens < 1)
        return bad(ctx, "strata_gdn_batch: dim, keyHeads, valueHeads and tokens must be >= 1");
    const int64_t stride = (int64_t)valueHeads * dim, n = covered(G, stride), heads = (n - 1) / dim + 1;
    const int64_t khs = std::min<int64_t>(keyHeads, heads);
    const uint64_t qk = (uint64_t)(((int64_t)(tokens - 1) * keyHeads + khs) * dim) * 4;
    const uint64_t vy = (uint64_t)((int64_t)(tokens - 1) * stride + n) * 4;
    const uint64_t gb = (uint64_t)((int64_t)(tokens - 1) * valueHeads + heads) * 4;
    if (int rc = need(ctx, a.ptr(0), (uint64_t)((int64_t)(dim - 1) * stride + n) * 4, "State")) return rc;
    if (int rc = need(ctx, a.ptr(1), qk, "Q")) return rc;
    if (int rc = need(ctx, a.ptr(2), qk, "K")) return rc;
    if (int rc = need(ctx, a.ptr(3), vy, "V")) return rc;
    if (int rc = need(ctx, a.ptr(4), gb, "Decay")) return rc;
    if (int rc = need(ctx, a.ptr(5), gb, "Beta")) return rc;
    if (int rc = need(ctx, a.ptr(6), vy, "Y")) return rc;
    // The register-resident variant needs a column of at most 128 values and
    // a State that no other argument aliases (the same handle twice).
    bool distinct = true;
    for (int i = 1; i < 7; i++) distinct = distinct && a.ptr(i) != a.ptr(0);
    if (distinct && (dim == 64 || dim == 128)) {
        // whole value heads of 64-column blocks, K / Q staged in LDS
        (dim == 64 ? k_gdn_batch_lds<64> : k_gdn_batch_lds<128>)<<<(unsigned)((n + 63) / 64), 64, 0, ctx->stream>>>(
            Fw(a, 0), F(a, 1), F(a, 2), F(a, 3), F(a, 4), F(a, 5), Fw(a, 6), keyHeads, valueHeads, tokens, (int)n);
        return launched(ctx);
    }
    (dim <= GDN_REG_MAX_DIM && distinct ? k_gdn_batch_reg : k_gdn_batch)<<<blocks256(n), 256, 0, ctx->stream>>>(
        Fw(a, 0), F(a, 1), F(a, 2), F(a, 3), F(a, 4), F(a, 5), Fw(a, 6), dim, keyHeads, valueHeads, tokens, (int)n);
    return launched(ctx);
}

int L_rope_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(4), heads = a.i32(5), rotary = a.i32(6), tokens = a.i32(7);
    if (dim < 1 || heads < 1 || rotary < 1 || tokens < 1) return bad(ctx, "strata_rope_batch: dim, heads, rotary, tokens >= 1");
    if (rotary % 2 || rotary > dim) return bad(ctx, "Rotary width must be even and <= head dimension");
    const int64_t n = covered(G, (int64_t)dim * heads * tokens);
    const uint64_t table = (uint64_t)(((n - 1) / ((int64_t)dim * heads) + 1) * (rotary / 2)) * 4;
    if (int rc = need(ctx, a.ptr(0), (uint64_t)((n - 1) / dim + 1) * dim * 4, "X")) return rc;
    if (int rc = need(ctx, a.ptr(1), table, "Cos")) return rc;
    if (int rc = need(ctx, a.ptr(2), table, "Sin")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)n * 4, "Y")) return rc;
    k_rope_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), Fw(a, 3), dim, heads, rotary, (int)n);
    return launched(ctx);
}

int L_kv_append_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(4), position = a.i32(5), tokens = a.i32(6);
    if (width < 1 || position < 0 || tokens < 1)
        return bad(ctx, "strata_kv_append_batch: width >= 1, position >= 0, tokens >= 1");
    const int64_t n = covered(G, (int64_t)width * tokens);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "K")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "V")) return rc;
    const uint64_t end = (uint64_t)((int64_t)position * width + n) * 4;
    if (int rc = need(ctx, a.ptr(2), end, "Keys")) return rc;
    if (int rc = need(ctx, a.ptr(3), end, "Values")) return rc;
    k_kv_append_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), Fw(a, 3), width, position,
                                                             (int)n);
    return launched(ctx);
}

int L_attention_gate_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(3), heads = a.i32(4), tokens = a.i32(5);
    if (dim < 1 || heads < 1 || tokens < 1) return bad(ctx, "strata_attention_gate_batch: dim, heads, tokens >= 1");
    const int64_t n = covered(G, (int64_t)dim * heads * tokens), last = n - 1;
    if (int rc = need(ctx, a.ptr(0), (uint64_t)n * 4, "Attention")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)((last / dim) * dim * 2 + dim + last % dim + 1) * 4, "FullQ"))
        return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Y")) return rc;
    k_attention_gate<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), dim, (int)n);
    return launched(ctx);
}

int L_ple_broadcast_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int width = a.i32(3), streams = a.i32(4), tokens = a.i32(5);
    if (width < 1 || streams < 1 || tokens < 1) return bad(ctx, "strata_ple_broadcast_batch: width, streams, tokens >= 1");
    const int64_t hc = (int64_t)width * streams, n = covered(G, hc * tokens);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)row_span(n, width, hc) * 4, "Value")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)((n - 1) / width + 1) * 4, "Gate")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Y")) return rc;
    k_ple_broadcast_batch<<<blocks256(n), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), Fw(a, 2), width, (int)hc, (int)n);
    return launched(ctx);
}

// src/backend.js:44-49: the prompt's token count is Q's length over heads x dim.
int L_attention_batch(sm_ctx *ctx, const uint32_t *G, Args a) {
    int dim = a.i32(4), heads = a.i32(5), kvHeads = a.i32(6), position = a.i32(7);
    float scale = a.f32(8);
    if (dim < 1 || heads < 1 || kvHeads < 1) return bad(ctx, "strata_attention_batch: dim, heads, kvHeads >= 1");
    if (heads % kvHeads) return fail(ctx, SM_E_ARG, "Attention heads must be divisible by KV heads");
    if (position < 0 || position > 2047) return bad(ctx, "attention position must be an integer in [0, 2047]");
    const int64_t qlen = buf_len(ctx, a.ptr(0)), row = (int64_t)heads * dim * 4;
    if (qlen < 0) return need(ctx, a.ptr(0), 0, "Q");
    if (qlen % row || position + qlen / row > 2048) return fail(ctx, SM_E_ARG, "Batched attention exceeds 2048 cells");
    const int tokens = (int)(qlen / row);
    const int tu = (int)std::min<int64_t>(G[2], tokens), hu = (int)std::min<int64_t>(G[0], heads);
    const int tiles = (int)std::min<int64_t>(G[1], (dim + 63) / 64);
    if (tu < 1) return SM_OK;
    const uint64_t kv = (uint64_t)(position + tu) * kvHeads * dim * 4;
    if (int rc = need(ctx, a.ptr(1), kv, "Keys")) return rc;
    if (int rc = need(ctx, a.ptr(2), kv, "Values")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)((int64_t)(tu - 1) * heads + hu) * dim * 4, "Y")) return rc;
    // Two launches over the whole GPU (k_attn_scores, k_attn_values) for the
    // production head sizes; one otherwise.
    const int group = heads / kvHeads;
    if ((dim == 64 || dim == 128 || dim == 256) && group <= 16 && (uint64_t)tu * heads * 2048 * 4 <= kAttnScoresBytes) {
        using KS = void (*)(const float *, const float *, float *, int, int, int, float, int);
        const int di = dim == 64 ? 0 : dim == 128 ? 1 : 2, hpw = (group + 3) / 4;
        static const KS ks[3][4] = {{k_attn_scores<64, 1>, k_attn_scores<64, 2>, k_attn_scores<64, 3>, k_attn_scores<64, 4>},
                                    {k_attn_scores<128, 1>, k_attn_scores<128, 2>, k_attn_scores<128, 3>,
                                     k_attn_scores<128, 4>},
                                    {k_attn_scores<256, 1>, k_attn_scores<256, 2>, k_attn_scores<256, 3>,
                                     k_attn_scores<256, 4>}};
        using KV = void (*)(const float *, const float *, float *, int, int, int, int, int);
        const int vh = group >= 4 ? 4 : group >= 2 ? 2 : 1, vi = vh == 4 ? 2 : vh == 2 ? 1 : 0;
        static const KV kv[3][3] = {{k_attn_values<64, 1>, k_attn_values<64, 2>, k_attn_values<64, 4>},
                                    {k_attn_values<128, 1>, k_attn_values<128, 2>, k_attn_values<128, 4>},
                                    {k_attn_values<256, 1>, k_attn_values<256, 2>, k_attn_values<256, 4>}};
        const int kvu = std::min(kvHeads, (hu - 1) / group + 1), cells = position + tu;
        ks[di][hpw - 1]<<<dim3((cells + 63) / 64, kvu, tu), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), ctx->attn_scores,
                                                                                    heads, kvHeads, position, scale, hu);
        if (int rc = launched(ctx)) return rc;
        const int gpk = (group + vh - 1) / vh;
        kv[di][vi]<<<dim3(tiles, kvu * gpk, tu), 64 * vh, 0, ctx->stream>>>(ctx->attn_scores, F(a, 2), Fw(a, 3), heads,
                                                                            kvHeads, position, hu, tiles);
        return launched(ctx);
    }
    k_attention_batch4<<<dim3(hu, (tiles + 3) / 4, tu), 256, 0, ctx->stream>>>(F(a, 0), F(a, 1), F(a, 2), Fw(a, 3),
                                                                                 dim, heads, kvHeads, position, scale,
                                                                                 tiles);
    return launched(ctx);
}

// Parameter lists in the reference's order (kernels/strata.cu).
const Entry kModelEntries[] = {
    {"strata_embedding",
     "Values:f32*,Codes:u32*,Scales:f32*,Offsets:f32*,Residual:f32*,width:i32,streams:i32,outputOffset:i32,format:i32,"
     "bits:i32,groupSize:i32,bias:i32,codebook:i32,hasOffset:i32",
     14, L_embedding},
    {"strata_rope_frequencies", "High:f32*,Low:f32*,rotary:i32,base:f32", 4, L_rope_frequencies},
    {"strata_rope_table", "High:f32*,Low:f32*,Cos:f32*,Sin:f32*,rotary:i32,context:i32", 6, L_rope_table},
    {"strata_rope_position", "X:f32*,Cos:f32*,Sin:f32*,Y:f32*,dim:i32,heads:i32,rotary:i32,position:i32,tokens:i32", 9,
     L_rope_position},
    {"strata_hc_mix", "Norm:f32*,Gate:f32*,Mixed:f32*,width:i32,streams:i32", 5, L_hc_mix},
    {"strata_hc_write", "Residual:f32*,Output:f32*,Inject:f32*,width:i32,streams:i32", 5, L_hc_write},
    {"strata_conv", "History:f32*,X:f32*,W:f32*,Y:f32*,channels:i32,taps:i32,dilation:i32,activation:i32", 8, L_conv},
    {"strata_gdn_gates", "Alpha:f32*,Beta:f32*,A:f32*,Dt:f32*,Decay:f32*,Strength:f32*,heads:i32", 7, L_gdn_gates},
    {"strata_gdn_step",
     "State:f32*,Q:f32*,K:f32*,V:f32*,Decay:f32*,Beta:f32*,Y:f32*,dim:i32,keyHeads:i32,valueHeads:i32", 10,
     L_gdn_step},
    {"strata_slice", "X:f32*,Y:f32*,width:i32,rows:i32,stride:i32,offset:i32", 6, L_slice},
    {"strata_kv_append", "K:f32*,V:f32*,Keys:f32*,Values:f32*,width:i32,position:i32", 6, L_kv_append},
    {"strata_attention",
     "Q:f32*,Keys:f32*,Values:f32*,Cells:i32*,Y:f32*,dim:i32,heads:i32,kvHeads:i32,count:i32,scale:f32", 10,
     L_attention},
    {"strata_attention_gate", "Attention:f32*,FullQ:f32*,Y:f32*,dim:i32,heads:i32", 5, L_attention_gate},
    {"strata_ple_gate", "Key:f32*,Query:f32*,Gate:f32*,width:i32,streams:i32", 5, L_ple_gate},
    {"strata_ple_broadcast", "Value:f32*,Gate:f32*,Y:f32*,width:i32,streams:i32", 5, L_ple_broadcast},
    {"strata_ple_add", "Residual:f32*,Gated:f32*,Conv:f32*,n:i32", 4, L_ple_add},
    {"strata_argmax", "Logits:f32*,Token:i32*,count:i32", 3, L_argmax},
    {"strata_ple_decode", "Packed:u32*,Values:f32*,count:i32", 3, L_ple_decode},
    {"strata_embed", "Row:f32*,Residual:f32*,width:i32,streams:i32", 4, L_embed},
    {"strata_rope", "X:f32*,Cos:f32*,Sin:f32*,Y:f32*,dim:i32,heads:i32,rotary:i32", 7, L_rope},
    {"strata_embed_batch", "Rows:f32*,Residual:f32*,width:i32,streams:i32,tokens:i32", 5, L_embed_batch},
    {"strata_hc_mix_batch", "Norm:f32*,Gate:f32*,Mixed:f32*,width:i32,streams:i32,tokens:i32", 6, L_hc_mix_batch},
    {"strata_hc_write_batch", "Residual:f32*,Output:f32*,Inject:f32*,width:i32,streams:i32,tokens:i32", 6,
     L_hc_write_batch},
    {"strata_conv_batch",
     "History:f32*,X:f32*,W:f32*,Y:f32*,channels:i32,taps:i32,dilation:i32,activation:i32,tokens:i32", 9,
     L_conv_batch},
    {"strata_gdn_gates_batch", "Alpha:f32*,Beta:f32*,A:f32*,Dt:f32*,Decay:f32*,Strength:f32*,heads:i32,tokens:i32", 8,
     L_gdn_gates_batch},
    {"strata_gdn_batch",
     "State:f32*,Q:f32*,K:f32*,V:f32*,Decay:f32*,Beta:f32*,Y:f32*,dim:i32,keyHeads:i32,valueHeads:i32,tokens:i32", 11,
     L_gdn_batch},
    {"strata_rope_batch", "X:f32*,Cos:f32*,Sin:f32*,Y:f32*,dim:i32,heads:i32,rotary:i32,tokens:i32", 8, L_rope_batch},
    {"strata_kv_append_batch", "K:f32*,V:f32*,Keys:f32*,Values:f32*,width:i32,position:i32,tokens:i32", 7,
     L_kv_append_batch},
    {"strata_attention_gate_batch", "Attention:f32*,FullQ:f32*,Y:f32*,dim:i32,heads:i32,tokens:i32", 6,
     L_attention_gate_batch},
    {"strata_ple_broadcast_batch", "Value:f32*,Gate:f32*,Y:f32*,width:i32,streams:i32,tokens:i32", 6,
     L_ple_broadcast_batch},
    {"strata_attention_batch",
     "Q:f32*,Keys:f32*,Values:f32*,Y:f32*,dim:i32,heads:i32,kvHeads:i32,position:i32,scale:f32", 9, L_attention_batch},
};

}  // namespace

namespace smi {
const Entry *model_entries(int *count) {
    *count = (int)(sizeof(kModelEntries) / sizeof(kModelEntries[0]));
    return kModelEntries;
}
}  // namespace smi
