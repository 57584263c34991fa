/*
 * CPU oracle, part 2: the kernels of the reference's untrained-fixture decode
 * (StrataEngine.step, src/engine.js:76-196) that lie outside the MoE stage:
 * embedding, RoPE frequencies/table/rotation, hyper-connection mix and
 * write-back, causal convolution, gated-delta-rule gates and state step,
 * slice, KV append, attention and its output gate, the PLE gate / broadcast /
 * add, and greedy argmax.
 *
 * TEST INFRASTRUCTURE ONLY, like strata_oracle.c: loaded by tests/ as the
 * checker, never by the product.
 *
 * Each function restates the kernels/strata.cu entry named in its comment
 * with the reference's f32 operation order (64-lane workgroups, lane-strided
 * sums, the s = 32 ... 1 tree). Built with -ffp-contract=off: no FMA, as in
 * the reference's WebAssembly build.
 *
 * Transcendentals. expf is strata_oracle.c's restatement of the ARM
 * optimized-routines design (musl's expf). logf, sinf and cosf are evaluated
 * here in double arithmetic and rounded once to float (series below), the
 * same operations as the HIP kernels' device functions, so CPU and GPU agree
 * bit for bit; against the reference's WebAssembly libm (musl, unpinned
 * version) they agree to within an ulp, not bitwise (checked against glibc
 * over the argument ranges the fixture uses, tests/test_oracle_model.py).
 *
 * Parity pins: the reference's own known answers for the whole fixture decode
 * (reports/wasm.json:172-178 tokens and routes, reports/validation.md:25) and
 * the float64 equations of tests/reference.mjs, plus the kernel recipes of
 * tests/conformance.js:45-69 (tests/test_oracle_model.py).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define LANES 64
#define NEG_BIG (-3.402823e38f) /* the reference's initial maximum, kernels/strata.cu:243,337,388 */

float or_expf(float x);
float or_sigmoid(float x);
float or_silu(float x);

static float tree_sum64(float *p) {
    for (int s = 32; s > 0; s >>= 1)
        for (int l = 0; l < s; l++) p[l] += p[l + s];
    return p[0];
}
static float tree_max64(float *p) {
    for (int s = 32; s > 0; s >>= 1)
        for (int l = 0; l < s; l++) p[l] = fmaxf(p[l], p[l + s]);
    return p[0];
}

/* ------------------------------------------------------- logf, sin, cos --- */
static uint64_t bits_of(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static double double_of(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* ln x for float x: x = m 2^e with m in [sqrt(1/2), sqrt(2)); ln m =
 * 2 atanh(y), y = (m-1)/(m+1), |y| <= 0.1716, by the odd series to y^27
 * (Horner in y^2, highest term first); result rounded once to float. */
float or_logf(float x) {
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (isinf(x)) return x;
    double d = (double)x;
    uint64_t u = bits_of(d);
    int e = (int)((u >> 52) & 2047u) - 1023; /* float inputs are normal in double */
    double m = double_of((u & 0x000fffffffffffffull) | 0x3ff0000000000000ull);
    if (m >= 1.4142135623730951) { m = m * 0.5; e = e + 1; }
    double y = (m - 1.0) / (m + 1.0), y2 = y * y, p = 1.0 / 27.0;
    for (int n = 25; n >= 1; n -= 2) p = p * y2 + 1.0 / (double)n;
    double r = 2.0 * (y * p) + (double)e * 0.6931471805599453;
    return (float)r;
}

/* sin and cos of a float r with |r| <= 4: r = k pi/2 + t, |t| <= pi/4,
 * pi/2 as a 33-bit head plus tail (k*head is exact for |k| <= 3), Taylor
 * series of sin t to t^19 and cos t to t^20 (Horner in t^2), quadrant by k. */
static void sincos_reduced(float r, double *s, double *c) {
    const double PIO2_HI = 1.57079632673412561417e+00, PIO2_LO = 6.07710050650619224932e-11;
    double x = (double)r;
    double kd = x * 0.63661977236758134308;
    int k = (int)(kd >= 0.0 ? kd + 0.5 : kd - 0.5);
    double t = (x - (double)k * PIO2_HI) - (double)k * PIO2_LO, t2 = t * t;
    /* 1/(2j+1)! and 1/(2j)! by repeated division */
    double as[10], ac[11], fs = 1.0, fc = 1.0, sn = 0.0, cs = 0.0;
    as[0] = 1.0;
    ac[0] = 1.0;
    for (int j = 1; j < 10; j++) { fs = fs / (double)(2 * j) / (double)(2 * j + 1); as[j] = fs; }
    for (int j = 1; j < 11; j++) { fc = fc / (double)(2 * j - 1) / (double)(2 * j); ac[j] = fc; }
    for (int j = 9; j >= 0; j--) sn = sn * (-t2) + as[j];
    for (int j = 10; j >= 0; j--) cs = cs * (-t2) + ac[j];
    sn = sn * t;
    switch (k & 3) {
    case 0: *s = sn; *c = cs; break;
    case 1: *s = cs; *c = -sn; break;
    case 2: *s = -sn; *c = -cs; break;
    default: *s = -cs; *c = sn; break;
    }
}
float or_sinf(float r) { double s, c; sincos_reduced(r, &s, &c); return (float)s; }
float or_cosf(float r) { double s, c; sincos_reduced(r, &s, &c); return (float)c; }

/* ---------------------------------------------------------------- kernels --- */
static float iq4_value(int c) {
    static const float t[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    return t[c & 15];
}

/* kernels/strata.cu:72-80 strata_embedding: one decoded row replicated over streams. */
void or_embedding(const float *Values, const uint32_t *Codes, const float *Scales, const float *Offsets,
                  float *Residual, int width, int streams, int outputOffset, int format, int bits,
                  int groupSize, int bias, int codebook, int hasOffset) {
    for (int i = 0; i < width; i++) {
        float value = 0.0f;
        if (format == 0) {
            value = Values[i];
        } else if (format == 1) {
            uint32_t u = ((Codes[i / 2] >> ((i % 2) * 16)) & 65535u) << 16;
            memcpy(&value, &u, 4);
        } else {
            int bit = i * bits, group = i / groupSize;
            int code = (int)((Codes[bit / 32] >> (bit % 32)) & ((1u << bits) - 1u));
            value = (codebook == 1 ? iq4_value(code) : (float)(code + bias)) * Scales[group];
            if (hasOffset != 0) value += Offsets[group];
        }
        for (int s = 0; s < streams; s++) Residual[outputOffset + s * width + i] = value;
    }
}

/* kernels/strata.cu:90-104 strata_rope_frequencies: base^(-2i/rotary) from a
 * double atanh series for ln(base) and a 20-term exp series, split into a
 * float head and a float tail. */
void or_rope_frequencies(float *High, float *Low, int rotary, float base) {
    const double ln2 = 0.693147180559945309417232121458176568;
    for (int i = 0; i < rotary / 2; i++) {
        double m = (double)base;
        int ex = 0;
        while (m >= 2.0) { m = m * 0.5; ex += 1; }
        double y = (m - 1.0) / (m + 1.0), term = y, lg = 0.0;
        for (int n = 1; n <= 49; n += 2) { lg += term / (double)n; term = term * y * y; }
        lg = 2.0 * lg + (double)ex * ln2;
        double power = -lg * (double)(2 * i) / (double)rotary;
        int whole = (int)(float)(power / ln2);
        double rem = power - (double)whole * ln2, result = 1.0;
        term = 1.0;
        for (int n = 1; n <= 20; ++n) { term = term * rem / (double)n; result += term; }
        for (; whole < 0; whole++) result = result * 0.5;
        High[i] = (float)result;
        Low[i] = (float)(result - (double)High[i]);
    }
}

/* kernels/strata.cu:105-111 strata_rope_table: angle = position * frequency
 * in double, reduced by whole turns, then cos/sin in float. */
void or_rope_table(const float *High, const float *Low, float *Cos, float *Sin, int rotary, int context) {
    const double turn = 6.283185307179586476925286766559005768;
    int half = rotary / 2;
    for (int i = 0; i < context * half; i++) {
        int pair = i % half;
        double angle = (double)(i / half) * ((double)High[pair] + (double)Low[pair]);
        int wraps = (int)(float)(angle / turn + 0.5);
        float reduced = (float)(angle - (double)wraps * turn);
        Cos[i] = or_cosf(reduced);
        Sin[i] = or_sinf(reduced);
    }
}

/* kernels/strata.cu:113-120 strata_rope_position: NeoX half-split rotation of
 * the first `rotary` components of each head at position + token. */
void or_rope_position(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int heads, int rotary,
                      int position, int tokens) {
    int half = rotary / 2;
    for (int i = 0; i < dim * heads * tokens; i++) {
        int d = i % dim;
        if (d >= rotary) { Y[i] = X[i]; continue; }
        int pair = d % half, row = i - d;
        int angle = (position + i / (dim * heads)) * half + pair;
        float c = Cos[angle], s = Sin[angle], a = X[row + pair], b = X[row + pair + half];
        Y[i] = d < half ? a * c - b * s : b * c + a * s;
    }
}

/* kernels/strata.cu:273-277 strata_hc_mix */
void or_hc_mix(const float *Norm, const float *Gate, float *Mixed, int width, int streams) {
    for (int i = 0; i < width; i++) {
        float v = 0.0f;
        for (int c = 0; c < streams; ++c) v += Norm[c * width + i] * or_sigmoid(Gate[c * width + i]);
        Mixed[i] = v / (float)streams;
    }
}
/* kernels/strata.cu:278-281 strata_hc_write */
void or_hc_write(float *Residual, const float *Output, const float *Inject, int width, int streams) {
    for (int i = 0; i < width * streams; i++)
        Residual[i] += Output[i % width] * (2.0f * or_sigmoid(Inject[i / width] / (float)streams));
}

/* kernels/strata.cu:287-295 strata_conv: channel-major history, W[c][taps],
 * tap taps-1 is the current input; the history shifts by one afterwards. */
void or_conv(float *History, const float *X, const float *W, float *Y, int channels, int taps, int dilation,
             int activation) {
    int span = (taps - 1) * dilation;
    for (int c = 0; c < channels; c++) {
        float *h = History + (int64_t)c * span;
        float sum = 0.0f;
        for (int t = 0; t < taps - 1; ++t) sum += h[t * dilation] * W[c * taps + t];
        sum += X[c] * W[c * taps + taps - 1];
        Y[c] = activation == 1 ? or_silu(sum) : sum;
        for (int t = 0; t < span - 1; ++t) h[t] = h[t + 1];
        if (span > 0) h[span - 1] = X[c];
    }
}

/* kernels/strata.cu:296-302 strata_gdn_gates: decay = exp(A softplus(alpha + dt)),
 * strength = sigmoid(beta); softplus is the identity above 20. */
void or_gdn_gates(const float *Alpha, const float *Beta, const float *A, const float *Dt, float *Decay,
                  float *Strength, int heads) {
    for (int h = 0; h < heads; h++) {
        float a = Alpha[h] + Dt[h];
        float sp = a > 20.0f ? a : or_logf(1.0f + or_expf(a));
        Decay[h] = or_expf(A[h] * sp);
        Strength[h] = or_sigmoid(Beta[h]);
    }
}

/* kernels/strata.cu:304-313 strata_gdn_step: state [key dim][value head][value dim];
 * value head h reads key head h % keyHeads. */
void or_gdn_step(float *State, const float *Q, const float *K, const float *V, const float *Decay,
                 const float *Beta, float *Y, int dim, int keyHeads, int valueHeads) {
    int stride = valueHeads * dim;
    for (int jh = 0; jh < dim * valueHeads; jh++) {
        int h = jh / dim, kh = h % keyHeads;
        float prediction = 0.0f;
        for (int i = 0; i < dim; ++i) {
            int ix = i * stride + jh;
            State[ix] *= Decay[h];
            prediction += State[ix] * K[kh * dim + i];
        }
        float delta = (V[jh] - prediction) * Beta[h], result = 0.0f;
        for (int i = 0; i < dim; ++i) {
            int ix = i * stride + jh;
            State[ix] += K[kh * dim + i] * delta;
            result += State[ix] * Q[kh * dim + i];
        }
        Y[jh] = result;
    }
}

/* kernels/strata.cu:314-316 strata_slice */
void or_slice(const float *X, float *Y, int width, int rows, int stride, int offset) {
    for (int i = 0; i < width * rows; i++) Y[i] = X[(i / width) * stride + offset + i % width];
}

/* kernels/strata.cu:328-330 strata_kv_append */
void or_kv_append(const float *K, const float *V, float *Keys, float *Values, int width, int position) {
    for (int i = 0; i < width; i++) {
        Keys[position * width + i] = K[i];
        Values[position * width + i] = V[i];
    }
}

/* kernels/strata.cu:334-356 strata_attention: per head, scores over the
 * selected cells (lane-strided, sequential dot), tree maximum, exponentials
 * and lane-strided sum with the tree, then per output component the
 * sequential weighted sum over cells divided by the total. Every output tile
 * of a head computes the same scores, so one pass per head suffices. */
void or_attention(const float *Q, const float *Keys, const float *Values, const int *Cells, float *Y, int dim,
                  int heads, int kvHeads, int count, float scale) {
    static float scores[2048];
    for (int h = 0; h < heads; h++) {
        float part[LANES];
        int kh = h / (heads / kvHeads);
        for (int l = 0; l < LANES; l++) {
            float mx = NEG_BIG;
            for (int t = l; t < count; t += LANES) {
                int base = (Cells[t] * kvHeads + kh) * dim;
                float score = 0.0f;
                for (int j = 0; j < dim; ++j) score += Q[h * dim + j] * Keys[base + j];
                score *= scale;
                scores[t] = score;
                mx = fmaxf(mx, score);
            }
            part[l] = mx;
        }
        float mx = tree_max64(part);
        for (int l = 0; l < LANES; l++) {
            float sum = 0.0f;
            for (int t = l; t < count; t += LANES) {
                float p = or_expf(scores[t] - mx);
                scores[t] = p;
                sum += p;
            }
            part[l] = sum;
        }
        float total = tree_sum64(part);
        for (int d = 0; d < dim; d++) {
            float value = 0.0f;
            for (int t = 0; t < count; ++t) value += scores[t] * Values[(Cells[t] * kvHeads + kh) * dim + d];
            Y[h * dim + d] = value / total;
        }
    }
}

/* kernels/strata.cu:357-359 strata_attention_gate: the second half of each
 * head's query row gates the attention output. */
void or_attention_gate(const float *Attention, const float *FullQ, float *Y, int dim, int heads) {
    for (int i = 0; i < dim * heads; i++)
        Y[i] = Attention[i] * or_sigmoid(FullQ[(i / dim) * dim * 2 + dim + i % dim]);
}

/* kernels/strata.cu:367-377 strata_ple_gate: per stream, gate =
 * sigmoid(sign(v) sqrt(max(|v|, 1e-6))), v = key.query / sqrt(width). */
void or_ple_gate(const float *Key, const float *Query, float *Gate, int width, int streams) {
    for (int c = 0; c < streams; c++) {
        float part[LANES];
        for (int l = 0; l < LANES; l++) {
            float dot = 0.0f;
            for (int d = l; d < width; d += LANES) dot += Key[c * width + d] * Query[c * width + d];
            part[l] = dot;
        }
        float v = tree_sum64(part) / sqrtf((float)width);
        float sign = v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
        Gate[c] = or_sigmoid(sign * sqrtf(fmaxf(fabsf(v), 0.000001f)));
    }
}
/* kernels/strata.cu:378-380 strata_ple_broadcast */
void or_ple_broadcast(const float *Value, const float *Gate, float *Y, int width, int streams) {
    for (int i = 0; i < width * streams; i++) Y[i] = Value[i % width] * Gate[i / width];
}
/* kernels/strata.cu:381-383 strata_ple_add */
void or_ple_add(float *Residual, const float *Gated, const float *Conv, int n) {
    for (int i = 0; i < n; i++) Residual[i] += Gated[i] + Conv[i];
}

/* kernels/strata.cu:386-396 strata_argmax: lane-strided best (first index on
 * ties), then the tree with the same rule. */
int or_argmax(const float *Logits, int count) {
    float v[LANES];
    int id[LANES];
    for (int l = 0; l < LANES; l++) {
        float best = NEG_BIG;
        int b = count;
        for (int i = l; i < count; i += LANES)
            if (Logits[i] > best || (Logits[i] == best && i < b)) { best = Logits[i]; b = i; }
        v[l] = best;
        id[l] = b;
    }
    for (int s = 32; s > 0; s >>= 1)
        for (int l = 0; l < s; l++)
            if (v[l + s] > v[l] || (v[l + s] == v[l] && id[l + s] < id[l])) { v[l] = v[l + s]; id[l] = id[l + s]; }
    return id[0];
}

/* kernels/strata.cu:168-176 strata_bf16_project: bf16 weights (the high
 * halves of f32 bit patterns, two per word) in strata_project's order. */
void or_bf16_project(const float *X, const uint32_t *Codes, float *Y, int cols, int rows, int tokens,
                     int outputStride, int outputOffset) {
    for (int token = 0; token < tokens; token++)
        for (int row = 0; row < rows; row++) {
            float p[LANES];
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int i = l; i < cols; i += LANES) {
                    int ix = row * cols + i;
                    uint32_t bits = ((Codes[ix / 2] >> ((ix % 2) * 16)) & 65535u) << 16;
                    float w;
                    memcpy(&w, &bits, 4);
                    sum += w * X[token * cols + i];
                }
                p[l] = sum;
            }
            Y[token * outputStride + outputOffset + row] = tree_sum64(p);
        }
}

float or_half_bits(uint32_t h);

/* kernels/strata.cu:81-89 strata_ple_decode: IQ4_NL blocks of 18 bytes (an
 * fp16 scale, then 16 bytes holding 32 4-bit codes: value j of the block is
 * the low nibble of byte j (j < 16) or the high nibble of byte j - 16). */
void or_ple_decode(const uint32_t *Packed, float *Values, int count) {
    for (int i = 0; i < count; i++) {
        int block = i / 32, scaleByte = block * 18, codeByte = scaleByte + 2 + i % 16;
        uint32_t half = (Packed[scaleByte / 4] >> ((scaleByte % 4) * 8)) & 65535u;
        int code = (int)((Packed[codeByte / 4] >> ((codeByte % 4) * 8 + (i % 32 < 16 ? 0 : 4))) & 15u);
        Values[i] = or_half_bits(half) * iq4_value(code);
    }
}

/* kernels/strata.cu:282-285 strata_embed: a row replicated over the streams. */
void or_embed(const float *Row, float *Residual, int width, int streams) {
    for (int i = 0; i < width * streams; i++) Residual[i] = Row[i % width];
}

/* kernels/strata.cu:319-327 strata_rope: NeoX half-split rotation of the
 * first `rotary` components of each head with the given cos/sin. */
void or_rope(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int heads, int rotary) {
    int half = rotary / 2;
    for (int i = 0; i < dim * heads; i++) {
        int d = i % dim, base = i - d;
        if (d >= rotary) { Y[i] = X[i]; continue; }
        int pair = d % half;
        float a = X[base + pair], b = X[base + pair + half];
        Y[i] = d < half ? a * Cos[pair] - b * Sin[pair] : b * Cos[pair] + a * Sin[pair];
    }
}

/* ------------------------------------------------- prompt (batch) kernels --- */
/* kernels/strata.cu:399-402 strata_embed_batch: token t's row over the streams. */
void or_embed_batch(const float *Rows, float *Residual, int width, int streams, int tokens) {
    int hc = width * streams;
    for (int i = 0; i < hc * tokens; i++) Residual[i] = Rows[(i / hc) * width + i % width];
}
/* kernels/strata.cu:403-408 strata_hc_mix_batch */
void or_hc_mix_batch(const float *Norm, const float *Gate, float *Mixed, int width, int streams, int tokens) {
    for (int i = 0; i < width * tokens; i++) {
        int token = i / width, d = i % width;
        float v = 0.0f;
        for (int c = 0; c < streams; ++c) {
            int p = (token * streams + c) * width + d;
            v += Norm[p] * or_sigmoid(Gate[p]);
        }
        Mixed[i] = v / (float)streams;
    }
}
/* kernels/strata.cu:409-412 strata_hc_write_batch */
void or_hc_write_batch(float *Residual, const float *Output, const float *Inject, int width, int streams, int tokens) {
    int hc = width * streams;
    for (int i = 0; i < hc * tokens; i++)
        Residual[i] += Output[(i / hc) * width + i % width] * (2.0f * or_sigmoid(Inject[i / width] / (float)streams));
}
/* kernels/strata.cu:413-424 strata_conv_batch: each channel's tokens in order. */
void or_conv_batch(float *History, const float *X, const float *W, float *Y, int channels, int taps, int dilation,
                   int activation, int tokens) {
    int span = (taps - 1) * dilation;
    for (int c = 0; c < channels; c++) {
        float *h = History + (int64_t)c * span;
        for (int token = 0; token < tokens; ++token) {
            float sum = 0.0f;
            for (int t = 0; t < taps - 1; ++t) sum += h[t * dilation] * W[c * taps + t];
            sum += X[token * channels + c] * W[c * taps + taps - 1];
            Y[token * channels + c] = activation == 1 ? or_silu(sum) : sum;
            for (int t = 0; t < span - 1; ++t) h[t] = h[t + 1];
            if (span > 0) h[span - 1] = X[token * channels + c];
        }
    }
}
/* kernels/strata.cu:425-431 strata_gdn_gates_batch */
void or_gdn_gates_batch(const float *Alpha, const float *Beta, const float *A, const float *Dt, float *Decay,
                        float *Strength, int heads, int tokens) {
    for (int i = 0; i < heads * tokens; i++) {
        float x = Alpha[i] + Dt[i % heads];
        float sp = x > 20.0f ? x : or_logf(1.0f + or_expf(x));
        Decay[i] = or_expf(A[i % heads] * sp);
        Strength[i] = or_sigmoid(Beta[i]);
    }
}
/* kernels/strata.cu:432-445 strata_gdn_batch: each (head, component)'s tokens in order. */
void or_gdn_batch(float *State, const float *Q, const float *K, const float *V, const float *Decay, const float *Beta,
                  float *Y, int dim, int keyHeads, int valueHeads, int tokens) {
    int stride = valueHeads * dim;
    for (int jh = 0; jh < dim * valueHeads; jh++) {
        int h = jh / dim, kh = h % keyHeads;
        for (int token = 0; token < tokens; ++token) {
            int qbase = (token * keyHeads + kh) * dim, gh = token * valueHeads + h;
            float prediction = 0.0f;
            for (int i = 0; i < dim; ++i) {
                int ix = i * stride + jh;
                State[ix] *= Decay[gh];
                prediction += State[ix] * K[qbase + i];
            }
            float delta = (V[token * stride + jh] - prediction) * Beta[gh], result = 0.0f;
            for (int i = 0; i < dim; ++i) {
                int ix = i * stride + jh;
                State[ix] += K[qbase + i] * delta;
                result += State[ix] * Q[qbase + i];
            }
            Y[token * stride + jh] = result;
        }
    }
}
/* kernels/strata.cu:446-453 strata_rope_batch: token t at table row t. */
void or_rope_batch(const float *X, const float *Cos, const float *Sin, float *Y, int dim, int heads, int rotary,
                   int tokens) {
    int half = rotary / 2;
    for (int i = 0; i < dim * heads * tokens; i++) {
        int d = i % dim;
        if (d >= rotary) { Y[i] = X[i]; continue; }
        int pair = d % half, base = i - d, angle = (i / (dim * heads)) * half + pair;
        float a = X[base + pair], b = X[base + pair + half];
        Y[i] = d < half ? a * Cos[angle] - b * Sin[angle] : b * Cos[angle] + a * Sin[angle];
    }
}
/* kernels/strata.cu:454-457 strata_kv_append_batch */
void or_kv_append_batch(const float *K, const float *V, float *Keys, float *Values, int width, int position,
                        int tokens) {
    for (int i = 0; i < width * tokens; i++) {
        Keys[position * width + i] = K[i];
        Values[position * width + i] = V[i];
    }
}
/* kernels/strata.cu:458-460 strata_attention_gate_batch */
void or_attention_gate_batch(const float *Attention, const float *FullQ, float *Y, int dim, int heads, int tokens) {
    for (int i = 0; i < dim * heads * tokens; i++)
        Y[i] = Attention[i] * or_sigmoid(FullQ[(i / dim) * dim * 2 + dim + i % dim]);
}
/* kernels/strata.cu:461-464 strata_ple_broadcast_batch */
void or_ple_broadcast_batch(const float *Value, const float *Gate, float *Y, int width, int streams, int tokens) {
    int hc = width * streams;
    for (int i = 0; i < hc * tokens; i++) Y[i] = Value[(i / hc) * width + i % width] * Gate[i / width];
}
/* kernels/strata.cu:512-534 strata_attention_batch: token t of the prompt
 * attends to cells 0 .. position + t (all rows already appended). */
void or_attention_batch(const float *Q, const float *Keys, const float *Values, float *Y, int dim, int heads,
                        int kvHeads, int position, float scale, int tokens) {
    static float scores[2048];
    for (int token = 0; token < tokens; token++)
        for (int h = 0; h < heads; h++) {
            float part[LANES];
            int count = position + token + 1, kh = h / (heads / kvHeads);
            for (int l = 0; l < LANES; l++) {
                float mx = NEG_BIG;
                for (int t = l; t < count; t += LANES) {
                    int base = (t * kvHeads + kh) * dim;
                    float score = 0.0f;
                    for (int j = 0; j < dim; ++j) score += Q[(token * heads + h) * dim + j] * Keys[base + j];
                    score *= scale;
                    scores[t] = score;
                    mx = fmaxf(mx, score);
                }
                part[l] = mx;
            }
            float mx = tree_max64(part);
            for (int l = 0; l < LANES; l++) {
                float sum = 0.0f;
                for (int t = l; t < count; t += LANES) {
                    float p = or_expf(scores[t] - mx);
                    scores[t] = p;
                    sum += p;
                }
                part[l] = sum;
            }
            float total = tree_sum64(part);
            for (int d = 0; d < dim; d++) {
                float value = 0.0f;
                for (int t = 0; t < count; ++t) value += scores[t] * Values[(t * kvHeads + kh) * dim + d];
                Y[(token * heads + h) * dim + d] = value / total;
            }
        }
}

/* ------------------------------------------------------------ self checks --- */
/* Counts, over float bit patterns u = start, start+step, ... < end, the inputs
 * where fn (0 logf, 1 sinf, 2 cosf) differs from this platform's libm (out[0])
 * and by more than one ulp from it (out[1]). */
void or_math_survey(int fn, uint32_t start, uint32_t end, uint32_t step, uint64_t *out) {
    uint64_t diff = 0, far = 0;
    for (int64_t u = start; u < (int64_t)end; u += step) {
        uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        float a = fn == 0 ? or_logf(x) : fn == 1 ? or_sinf(x) : or_cosf(x);
        float r = fn == 0 ? logf(x) : fn == 1 ? sinf(x) : cosf(x);
        int32_t ia, ir;
        memcpy(&ia, &a, 4);
        memcpy(&ir, &r, 4);
        if (ia != ir) {
            diff++;
            int64_t gap = (int64_t)ia - (int64_t)ir;
            if ((ia ^ ir) < 0 || gap > 1 || gap < -1) far++;
        }
    }
    out[0] = diff;
    out[1] = far;
}
