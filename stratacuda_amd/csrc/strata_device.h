// Device-side building blocks shared by the MI355X kernels.
//
// Arithmetic contract: the library is compiled with -ffp-contract=off, so
// every f32/f64 product and sum written here rounds separately, exactly as in
// the reference's CPU path (WebAssembly has no FMA). Kernels that may trade
// operation order for speed ask for fused multiply-adds explicitly (fmaf).
// Bit-identical router logits are what make the selected expert IDs bit-exact.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SM_WAVE 64

namespace sm {

// ------------------------------------------------------------------ fp16
// IEEE binary16 -> f32, including subnormals, signed zero, inf and NaN
// (kernels/strata.cu:13-18 strata_half_bits).
__device__ __forceinline__ float half_bits(uint32_t h) {
    uint32_t sign = (h & 32768u) << 16, exponent = (h >> 10) & 31u, fraction = h & 1023u;
    if (exponent == 0u) {
        if (fraction == 0u) return __uint_as_float(sign);
        float v = (float)fraction * 0.000000059604644775390625f;
        return sign != 0u ? -v : v;
    }
    if (exponent == 31u) return __uint_as_float(sign | 2139095040u | (fraction << 13));
    return __uint_as_float(sign | ((exponent + 112u) << 23) | (fraction << 13));
}

// ------------------------------------------------------------------ expf
// expf evaluated by the ARM optimized-routines design (the libm expf of
// musl, which the reference's WebAssembly build links): 2^(k/32) from a
// 32-entry table, a cubic for 2^(r/32), double arithmetic with every
// operation rounded separately (no FMA, as on wasm32).
// Table entry i holds the bits of 2^(i/32) (rounded to double) minus i<<47;
// tests/test_oracle_math.py recomputes every entry from exact arithmetic.
__constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
// `tab` may point at a copy of kExp2Tab in LDS (a per-lane indexed load from
// __constant__ memory goes through the vector memory path).
// Branch-free: the main path runs on x clamped into the range where it
// applies, and the special cases (the branches of the reference's expf:
// -inf -> 0, inf / NaN -> x + x, overflow -> inf, underflow -> 0) are
// selected afterwards, so a caller's independent exponentials interleave.
// For every input the result equals the branching form's.
__device__ __forceinline__ float expf_or(float x, const uint64_t *tab = kExp2Tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double Shift = 0x1.8p+52;
    const float kOver = 0x1.62e42ep6f, kUnder = -0x1.9fe368p6f;
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    const float xc = fminf(fmaxf(x, kUnder), kOver);  // NaN -> kUnder; its result is replaced below
    double xd = (double)xc;
    double z = InvLn2N * xd;
    double kd = z + Shift;
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - Shift;
    double r = z - kd;
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double zz = C0 * r + C1;
    double r2 = r * r;
    double y = C2 * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    float out = (float)y;
    const bool special = abstop >= 0x42bu;
    out = special && x < kUnder ? 0.0f : out;
    out = special && x > kOver ? __uint_as_float(0x7f800000u) : out;
    out = abstop >= 0x7f8u ? x + x : out;
    out = ux == 0xff800000u ? 0.0f : out;
    return out;
}
// N independent exponentials. Each main path is pinned (an empty asm that
// consumes all N results) before its special cases are selected, so the
// compiler cannot sink the N evaluations into separate conditional blocks
// and they interleave (their table reads are issued together).
template <int N>
__device__ __forceinline__ void expf_or_n(const float (&x)[N], float (&out)[N], const uint64_t *tab = kExp2Tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double Shift = 0x1.8p+52;
    const float kOver = 0x1.62e42ep6f, kUnder = -0x1.9fe368p6f;
#pragma unroll
    for (int i = 0; i < N; i++) {
        const float xc = fminf(fmaxf(x[i], kUnder), kOver);
        double xd = (double)xc;
        double z = InvLn2N * xd;
        double kd = z + Shift;
        uint64_t ki = (uint64_t)__double_as_longlong(kd);
        kd = kd - Shift;
        double r = z - kd;
        uint64_t t = tab[ki % 32] + (ki << 47);
        double s = __longlong_as_double((long long)t);
        double zz = C0 * r + C1;
        double r2 = r * r;
        double y = C2 * r + 1.0;
        y = zz * r2 + y;
        y = y * s;
        out[i] = (float)y;
    }
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" : "+v"(out[i]));
#pragma unroll
    for (int i = 0; i < N; i++) {
        const uint32_t ux = __float_as_uint(x[i]);
        const uint32_t abstop = (ux >> 20) & 0x7ffu;
        const bool special = abstop >= 0x42bu;
        float o = out[i];
        o = special && x[i] < kUnder ? 0.0f : o;
        o = special && x[i] > kOver ? __uint_as_float(0x7f800000u) : o;
        o = abstop >= 0x7f8u ? x[i] + x[i] : o;
        o = ux == 0xff800000u ? 0.0f : o;
        out[i] = o;
    }
}
// Fills an LDS copy of kExp2Tab (lanes 0-31 of every wave, one entry each,
// all waves writing the same values) from values known at compile time: no
// vector-memory load, so nothing delays the kernel's first loads. A wave may
// read the table after wave_lds_sync() (its own writes are then complete),
// without waiting for the other waves.
__device__ __forceinline__ void fill_exp_table(uint64_t *s_tab) {
    const int t = threadIdx.x & 63;
    if (t < 32) {
        uint64_t v = kExp2Tab[0];
#pragma unroll
        for (int i = 1; i < 32; i++) v = t == i ? kExp2Tab[i] : v;
        s_tab[t] = v;
    }
}
// kernels/strata.cu:7-8
__device__ __forceinline__ float sigmoid(float x, const uint64_t *tab = kExp2Tab) {
    return 1.0f / (1.0f + expf_or(-x, tab));
}
__device__ __forceinline__ float silu(float x, const uint64_t *tab = kExp2Tab) { return x * sigmoid(x, tab); }

// ------------------------------------------------------ logf, sin, cos
// Evaluated in double arithmetic (every operation rounded separately) and
// rounded once to float; the CPU oracle evaluates the same operations, so
// both produce the same bits. Within one ulp of libm over the ranges used.
//
// ln x: x = m 2^e, m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(y) with
// y = (m-1)/(m+1) by the odd series to y^27 (Horner in y^2).
__device__ inline float logf_or(float x) {
    if (x != x) return x;
    if (x < 0.0f) return __uint_as_float(0x7fc00000u);
    if (x == 0.0f) return __uint_as_float(0xff800000u);
    if (x == __uint_as_float(0x7f800000u)) return x;
    uint64_t u = (uint64_t)__double_as_longlong((double)x);
    int e = (int)((u >> 52) & 2047u) - 1023;
    double m = __longlong_as_double((long long)((u & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
    if (m >= 1.4142135623730951) {
        m = m * 0.5;
        e = e + 1;
    }
    double y = (m - 1.0) / (m + 1.0), y2 = y * y, p = 1.0 / 27.0;
#pragma unroll
    for (int n = 25; n >= 1; n -= 2) p = p * y2 + 1.0 / (double)n;
    return (float)(2.0 * (y * p) + (double)e * 0.6931471805599453);
}
// sin and cos of |r| <= 4: r = k pi/2 + t, |t| <= pi/4 (pi/2 as a 33-bit
// head plus a tail), Taylor series of sin t to t^19 and cos t to t^20.
__device__ inline void sincos_or(float r, float &s_out, float &c_out) {
    const double PIO2_HI = 1.57079632673412561417e+00, PIO2_LO = 6.07710050650619224932e-11;
    double x = (double)r;
    double kd = x * 0.63661977236758134308;
    int k = (int)(kd >= 0.0 ? kd + 0.5 : kd - 0.5);
    double t = (x - (double)k * PIO2_HI) - (double)k * PIO2_LO, t2 = t * t;
    double as[10], ac[11], fs = 1.0, fc = 1.0, sn = 0.0, cs = 0.0;
    as[0] = 1.0;
    ac[0] = 1.0;
#pragma unroll
    for (int j = 1; j < 10; j++) {
        fs = fs / (double)(2 * j) / (double)(2 * j + 1);
        as[j] = fs;
    }
#pragma unroll
    for (int j = 1; j < 11; j++) {
        fc = fc / (double)(2 * j - 1) / (double)(2 * j);
        ac[j] = fc;
    }
#pragma unroll
    for (int j = 9; j >= 0; j--) sn = sn * (-t2) + as[j];
#pragma unroll
    for (int j = 10; j >= 0; j--) cs = cs * (-t2) + ac[j];
    sn = sn * t;
    double s, c;
    switch (k & 3) {
    case 0: s = sn; c = cs; break;
    case 1: s = cs; c = -sn; break;
    case 2: s = -sn; c = -cs; break;
    default: s = -cs; c = sn; break;
    }
    s_out = (float)s;
    c_out = (float)c;
}

// --------------------------------------------------------- wave reductions
// Cross-lane moves use DPP where the pattern allows: a DPP move costs a few
// cycles, while a ds_bpermute shuffle (__shfl*) costs ~55 ns of latency on
// MI355X. DPP controls (GFX9 encoding):
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i within 8
constexpr int kDppRowMirror = 0x140;    // lane i <- lane 15-i within 16
constexpr int kDppRowBcast15 = 0x142;   // row r+1 <- lane 15 of row r
constexpr int kDppRowBcast31 = 0x143;   // rows 2,3 <- lane 31

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f32(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                                                 false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_i32(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}

// Tree sum over the 64 lanes in the reference order (s = 32, 16, ..., 1: lane
// l adds lane l+s), so the result is bit-identical to the reference's
// shared-memory tree. Valid in lane 0. Levels 8..1 stay inside a 16-lane row
// (DPP row_shl: lane i receives lane i+s); levels 32 and 16 cross rows
// through the gfx950 lane-swap instructions.
__device__ __forceinline__ float tree_sum64(float v) {
    // v_permlane32_swap(v, v).second holds lane l+32 in lanes 0-31;
    // v_permlane16_swap(v, v).second holds lane l+16 in rows 0 and 2.
    v = v + __builtin_bit_cast(float, (int)__builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, v),
                                                                          __builtin_bit_cast(int, v), false, false)[1]);
    v = v + __builtin_bit_cast(float, (int)__builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v),
                                                                          __builtin_bit_cast(int, v), false, false)[1]);
    v = v + dpp_f32<0x108>(0.0f, v);
    v = v + dpp_f32<0x104>(0.0f, v);
    v = v + dpp_f32<0x102>(0.0f, v);
    v = v + dpp_f32<0x101>(0.0f, v);
    return v;
}
// Maximum over the 64 lanes (order-free), returned in every lane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<kDppQuadXor1>(v, v));
    v = fmaxf(v, dpp_f32<kDppQuadXor2>(v, v));
    v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v, v));
    v = fmaxf(v, dpp_f32<kDppRowMirror>(v, v));
    v = fmaxf(v, dpp_f32<kDppRowBcast15, 0xa>(v, v));
    v = fmaxf(v, dpp_f32<kDppRowBcast31, 0xc>(v, v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ int wave_min_i32(int v) {
    v = min(v, dpp_i32<kDppQuadXor1>(v, v));
    v = min(v, dpp_i32<kDppQuadXor2>(v, v));
    v = min(v, dpp_i32<kDppRowHalfMirror>(v, v));
    v = min(v, dpp_i32<kDppRowMirror>(v, v));
    v = min(v, dpp_i32<kDppRowBcast15, 0xa>(v, v));
    v = min(v, dpp_i32<kDppRowBcast31, 0xc>(v, v));
    return __builtin_amdgcn_readlane(v, 63);
}
// Exact integer sum over the wave, in every lane.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v = v + dpp_i32<kDppQuadXor1>(0, v);
    v = v + dpp_i32<kDppQuadXor2>(0, v);
    v = v + dpp_i32<kDppRowHalfMirror>(0, v);
    v = v + dpp_i32<kDppRowMirror>(0, v);
    v = v + dpp_i32<kDppRowBcast15, 0xa>(0, v);
    v = v + dpp_i32<kDppRowBcast31, 0xc>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t u) {
    int v = (int)u;
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppQuadXor1>(v, v));
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppQuadXor2>(v, v));
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppRowHalfMirror>(v, v));
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppRowMirror>(v, v));
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppRowBcast15, 0xa>(v, v));
    v = (int)max((uint32_t)v, (uint32_t)dpp_i32<kDppRowBcast31, 0xc>(v, v));
    return (uint32_t)__builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, dpp_i32<kDppQuadXor1>(v, v));
    v = max(v, dpp_i32<kDppQuadXor2>(v, v));
    v = max(v, dpp_i32<kDppRowHalfMirror>(v, v));
    v = max(v, dpp_i32<kDppRowMirror>(v, v));
    v = max(v, dpp_i32<kDppRowBcast15, 0xa>(v, v));
    v = max(v, dpp_i32<kDppRowBcast31, 0xc>(v, v));
    return __builtin_amdgcn_readlane(v, 63);
}
// Sum within each group of 8 consecutive lanes (any order), in every lane.
__device__ __forceinline__ float group8_sum(float v) {
    v = v + dpp_f32<kDppQuadXor1>(0.0f, v);
    v = v + dpp_f32<kDppQuadXor2>(0.0f, v);
    v = v + dpp_f32<kDppRowHalfMirror>(0.0f, v);
    return v;
}
// Sum within each 32-lane half (any order): valid in lanes 31 and 63.
__device__ __forceinline__ float half32_sum(float v) {
    v = v + dpp_f32<kDppQuadXor1>(0.0f, v);
    v = v + dpp_f32<kDppQuadXor2>(0.0f, v);
    v = v + dpp_f32<kDppRowHalfMirror>(0.0f, v);
    v = v + dpp_f32<kDppRowMirror>(0.0f, v);
    v = v + dpp_f32<kDppRowBcast15, 0xa>(0.0f, v);
    return v;
}

// Inclusive prefix sum over the 64 lanes (integers), by DPP: lane l gets
// the sum of lanes 0..l.
__device__ __forceinline__ int wave_scan_incl(int v) {
    v = v + dpp_i32<0x111>(0, v);  // row_shr:1
    v = v + dpp_i32<0x112>(0, v);  // row_shr:2
    v = v + dpp_i32<0x114>(0, v);  // row_shr:4
    v = v + dpp_i32<0x118>(0, v);  // row_shr:8
    v = v + dpp_i32<kDppRowBcast15, 0xa>(0, v);
    v = v + dpp_i32<kDppRowBcast31, 0xc>(0, v);
    return v;
}

// -------------------------------------------------------- synthetic data
// Counter-based generator for the seeded synthetic workloads (the same
// definition is restated independently in the CPU oracle):
//   rand(seed, stream, i) = mix(mix(seed + G*(stream+1)) + i), mix = SplitMix64
//   normal(i) = (sum of 12 uniform u32 from rand(6i .. 6i+5)) * 2^-32 - 6
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t rand_key(uint64_t seed, uint64_t stream) {
    return mix64(seed + 0x9E3779B97F4A7C15ull * (stream + 1));
}
__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i) {
    uint64_t s = 0;
#pragma unroll
    for (int j = 0; j < 6; j++) {
        uint64_t r = mix64(key + 6 * i + j);
        s += (r & 0xffffffffull) + (r >> 32);
    }
    return (double)s * 0x1p-32 - 6.0;
}
// f32 -> binary16, round to nearest even.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    uint32_t x = __float_as_uint(f);
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

// Population count of a wave mask as a 32-bit int: two 32-bit counts keep
// the comparison that follows on the scalar unit (a 64-bit count compared
// with a constant becomes a vector compare and a round trip through VALU).
__device__ __forceinline__ int popc64(unsigned long long m) {
    return __builtin_popcount((uint32_t)m) + __builtin_popcount((uint32_t)(m >> 32));
}

// Selection keys for the reference's top-k rounds (kernels/strata.cu:252-265).
// A probability p >= +0 is keyed by its bit pattern read as int, which orders
// exactly like the value; an expert past `experts` or with a NaN probability
// gets kNoneKey (INT_MIN), which the reference's `>` / `==` tests never pick.
constexpr int kNoneKey = (int)0x80000000u;
__device__ __forceinline__ int select_key(float p, bool valid) {
    return valid && p == p ? __builtin_bit_cast(int, p) : kNoneKey;
}
// Sorts eight packed entries in descending order (Batcher's odd-even merge
// network, 19 compare-exchanges; all registers, no branches).
__device__ __forceinline__ void sort8_desc(uint64_t (&P)[8]) {
    constexpr int kNet[19][2] = {{0, 1}, {2, 3}, {4, 5}, {6, 7}, {0, 2}, {1, 3}, {4, 6}, {5, 7}, {1, 2}, {5, 6},
                                 {0, 4}, {1, 5}, {2, 6}, {3, 7}, {2, 4}, {3, 5}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int c = 0; c < 19; c++) {
        const uint64_t a = P[kNet[c][0]], b = P[kNet[c][1]];
        const bool swap = b > a;
        P[kNet[c][0]] = swap ? b : a;
        P[kNet[c][1]] = swap ? a : b;
    }
}
// topK selection rounds over one wave, with the reference's results; lane l
// holds the keys of experts l + 64 j (j < 8). The reference takes, each
// round, the largest probability (lower ID on ties) and sets it to -1.0f.
// Here every lane first sorts its eight entries, packed as
// (key ^ 2^31) << 3 | (7 - j), so its head is its best entry (the lower j,
// hence the lower ID, on equal keys). A round is then one wave maximum over
// the heads, a ballot for ties between lanes (the lowest ID among tied heads
// wins) and a shift of the winning lane's list. Once no entry with p >= 0 is
// left, the reference's rounds pick the lowest-ID expert already set to -1.0f
// (or ID `experts` when there is none), which `lowest_picked` tracks.
// Lane 0 writes Ids[k]; lane k returns the selected probability of round k.
__device__ __forceinline__ void select_rounds(const int (&key)[8], int experts, int topK, int *Ids, float &mine) {
    const int lane = threadIdx.x & 63;
    uint64_t P[8];
#pragma unroll
    for (int j = 0; j < 8; j++) P[j] = ((uint64_t)((uint32_t)key[j] ^ 0x80000000u) << 3) | (uint64_t)(7 - j);
    sort8_desc(P);
    int lowest_picked = experts;
    mine = 0.0f;
    for (int k = 0; k < topK; ++k) {
        const uint32_t head = (uint32_t)(P[0] >> 3);
        const uint32_t top = wave_max_u32(head);
        int winner = lowest_picked;
        float value = -1.0f;
        if (top != 0u) {
            const unsigned long long tied = __ballot(head == top);
            const int id = lane + 64 * (7 - (int)(P[0] & 7u));
            if (popc64(tied) == 1) winner = __builtin_amdgcn_readlane(id, __ffsll((long long)tied) - 1);
            else winner = wave_min_i32(head == top ? id : 0x7fffffff);
            value = __builtin_bit_cast(float, top ^ 0x80000000u);
            lowest_picked = min(lowest_picked, winner);
            const bool pop = lane == (winner & 63);
#pragma unroll
            for (int j = 0; j < 7; j++) P[j] = pop ? P[j + 1] : P[j];
            P[7] = pop ? 0ull : P[7];
        }
        if (lane == 0) Ids[k] = winner;
        if (lane == k) mine = value;
    }
}
// kernels/strata.cu:266-269: weights = selected / max(sum(selected), 2^-14),
// the sum taken sequentially over k. Lane k holds selected[k].
__device__ __forceinline__ void router_weights(float mine, int topK, float *Weights) {
    const int lane = threadIdx.x & 63;
    float denom = 0.0f;
    for (int k = 0; k < topK; ++k)
        denom = denom + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), k));
    denom = fmaxf(denom, 0.00006103515625f);
    if (lane < topK) Weights[lane] = mine / denom;
}

// kernels/strata.cu:240-270 strata_router / :479-509 strata_router_batch for
// one token, by one 64-lane wave, with the reference's results bit for bit:
// probabilities follow the reference's operation order (lane-strided
// sequential sums, then the reference tree), lane l holds experts l, l+64, ...
// (at most 8 for 512 experts), and each of the topK rounds takes every lane's
// best (the reference's lane loop, including its handling of already
// selected experts) and the wave maximum; ties in probability go to the
// lower expert ID, so the winner of a round is the same expert the
// reference's tree reduction finds. The wave maximum uses DPP and a ballot
// instead of a shuffle tree.
__device__ __forceinline__ void router_wave(const float *Logits, int *Ids, float *Weights, int experts, int topK,
                                            const uint64_t *tab = kExp2Tab) {
    const int lane = threadIdx.x & 63;
    float p[8];
    float mx = -3.402823e38f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int e = lane + 64 * j;
        if (e < experts) mx = fmaxf(mx, Logits[e]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int e = lane + 64 * j;
        p[j] = 0.0f;
        if (e < experts) {
            p[j] = expf_or(Logits[e] - mx, tab);
            sum = sum + p[j];
        }
    }
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, tree_sum64(sum))));
    const float inv = 1.0f / sum;
    int key[8];
#pragma unroll
    for (int j = 0; j < 8; j++) key[j] = select_key(p[j] * inv, lane + 64 * j < experts);
    float mine;
    select_rounds(key, experts, topK, Ids, mine);
    router_weights(mine, topK, Weights);
}

// Orders LDS accesses of one wave (no other wave takes part): the fences
// keep the compiler from moving LDS reads and writes across this point, and
// a wave's LDS instructions complete in order.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A block barrier that orders LDS accesses only: each wave's LDS accesses
// complete before the barrier, and its outstanding global loads and stores
// stay in flight (__syncthreads waits for those too).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// LDS for router_block: probabilities, the cross-wave max, and the scratch of
// select_ranked.
struct RouterScratch {
    float p[512];
    float red[4];
    alignas(16) uint64_t cand[128];  // up to 64 candidates, zeros after the last (read 8 at a time)
    float val[32];
};

// Gathers the entries with in[j] set (at most 64, else returns false and
// writes nothing) into x.cand, one per lane, and ranks each against the
// others by its packed key Q = order key << 9 | (511 - e): the entry of rank
// k (k < topK) goes to s_ids[k], and with `with_val` its key's upper 32 bits,
// read back as a probability, to x.val[k]. Lane l's entries land after the
// entries of lanes 0..l-1 (a lane scan of the per-lane counts, all on the
// vector unit); the slots after the last hold 0, below every candidate.
__device__ __forceinline__ bool rank_candidates(const uint64_t (&Q)[8], const bool (&in)[8], int topK,
                                                RouterScratch &x, int *s_ids, bool with_val) {
    const int lane = threadIdx.x & 63;
    int pos[8], n = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        pos[j] = n;
        n += in[j] ? 1 : 0;
    }
    const int incl = wave_scan_incl(n);
    const int count = __builtin_amdgcn_readlane(incl, 63);
    if (count > 64) return false;
    x.cand[lane] = 0ull;
    // entries that are not candidates go to slot 64 + lane, never read
#pragma unroll
    for (int j = 0; j < 8; j++) x.cand[in[j] ? incl - n + pos[j] : 64 + lane] = Q[j];
    wave_lds_sync();
    // Candidate `lane` against every candidate: 8 at a time through
    // broadcast 16-byte LDS reads (every lane reads the same address).
    // Slots 0..15 always (those past `count` hold 0, below every candidate),
    // then 8 at a time; four partial counts keep the additions independent.
    const uint64_t q = x.cand[lane];
    int rk[4] = {0, 0, 0, 0};
    auto rank8 = [&](int c) {
        const uint4 *src = (const uint4 *)&x.cand[c];
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = src[u];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint64_t a = ((uint64_t)v[u].y << 32) | v[u].x, b = ((uint64_t)v[u].w << 32) | v[u].z;
            rk[u] += (a > q ? 1 : 0) + (b > q ? 1 : 0);
        }
    };
    rank8(0);
    rank8(8);
    for (int c = 16; c < count; c += 8) rank8(c);
    const int rank = (rk[0] + rk[1]) + (rk[2] + rk[3]);
    if (lane < count && rank < topK) {
        s_ids[rank] = 511 - (int)(q & 511u);
        if (with_val) x.val[rank] = __builtin_bit_cast(float, (uint32_t)(q >> 9) ^ 0x80000000u);
    }
    return true;
}

// The same selection as select_rounds in one pass. Entry e gets the 41-bit
// order key Q = (key ^ 2^31) << 9 | (511 - e): Q descending is exactly the
// order in which the reference's rounds pick experts (larger probability
// first, lower ID on equal probabilities), so round k picks the entry of
// rank k. Any threshold T at or below the topK-th largest of the 64 lane
// maxima (those maxima are topK distinct entries) keeps every selected entry
// among those with key >= T; a bitwise search with ballots sets T's upper
// bits. The entries with key >= T are gathered in LDS (one per lane) and
// each is ranked against the others. With more than 64 such entries (heavy
// ties), or fewer than topK lanes holding a probability >= 0 (NaN routing
// input), the rounds of select_rounds run instead. Results: the IDs in
// s_ids[0, topK) and the selected probabilities in x.val[0, topK) (LDS).
__device__ __forceinline__ void select_ranked(const int (&key)[8], int experts, int topK, RouterScratch &x,
                                              int *s_ids) {
    const int lane = threadIdx.x & 63;
    float mine;
    uint32_t hk = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) hk = max(hk, (uint32_t)key[j] ^ 0x80000000u);
    // Every valid entry (p >= 0) has a key >= 2^31 here; fewer than topK
    // lanes with one means NaN routing input or topK > 64.
    if (popc64(__ballot(hk >= 0x80000000u)) < topK) {
        select_rounds(key, experts, topK, s_ids, mine);
        if (lane < topK) x.val[lane] = mine;
        return;
    }
    // Bits 29..16 of T (p <= 1 keeps bit 30 clear). Any T at or below the
    // topK-th largest lane maximum is a valid threshold: the low bits only
    // trim candidates, and with them unset the candidates are typically
    // topK + 1 (measured on random logits: at most 17 for topK = 10).
    uint32_t T = 0x80000000u;
#pragma unroll
    for (int b = 29; b >= 16; b--) {
        const uint32_t c = T | (1u << b);
        if (popc64(__ballot(hk >= c)) >= topK) T = c;
    }
    uint64_t Q[8];
    bool in[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t k = (uint32_t)key[j] ^ 0x80000000u;
        Q[j] = ((uint64_t)k << 9) | (uint64_t)(511 - (lane + 64 * j));
        in[j] = k >= T;
    }
    if (!rank_candidates(Q, in, topK, x, s_ids, true)) {
        select_rounds(key, experts, topK, s_ids, mine);
        if (lane < topK) x.val[lane] = mine;
    }
}

// The same routing for one token by a 256-thread block: the 512 exponentials
// are spread over all threads (table in LDS), wave 0 forms the reference sum
// and runs the selection. The IDs land in s_ids and the selected
// probabilities in s.val[0, topK) (LDS; router_weights forms the weights). Needs
// blockDim.x == 256 and experts <= 512. s_tab must already hold kExp2Tab.
// Thread t's logits (experts t and t + 256); issued before a kernel's other
// loads, as vector loads complete in order.
// Every wave loads all the token's logits (lane l: experts l + 64 j; past
// `experts`: -FLT_MAX), so each forms the maximum itself, with no barrier.
// Unconditional loads (clamped index), so a later wait covers exactly these.
__device__ __forceinline__ void router_load(const float *Logits, int experts, float (&l)[8]) {
    const int lane = threadIdx.x & 63;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = Logits[min(lane + 64 * j, experts - 1)];
#pragma unroll
    for (int j = 0; j < 8; j++) l[j] = lane + 64 * j < experts ? v[j] : -3.402823e38f;
}
__device__ __forceinline__ void router_select_lds(int experts, int topK, RouterScratch &s, int *s_ids);
__device__ __forceinline__ void router_block(const float (&l)[8], int experts, int topK, const uint64_t *s_tab,
                                             RouterScratch &s, int *s_ids) {
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e0 = tid, e1 = tid + 256;
    // fmaxf returns one of its operands, so the order of the maximum does
    // not change its value
    float mx = l[0];
#pragma unroll
    for (int j = 1; j < 8; j++) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    wave_lds_sync();  // this wave's copy of the exp table is in LDS
    float l0 = l[0], l1 = l[4];  // experts e0 = lane + 64 wave and e1 = e0 + 256
#pragma unroll
    for (int j = 1; j < 4; j++)
        if (wave == j) {
            l0 = l[j];
            l1 = l[j + 4];
        }
    // Entries past `experts` hold +0: adding them to the (non-negative or
    // NaN) sums below changes nothing, so wave 0 reads all eight at once.
    const float d[2] = {l0 - mx, l1 - mx};
    float ex[2];
    expf_or_n<2>(d, ex, s_tab);
    s.p[e0] = e0 < experts ? ex[0] : 0.0f;
    s.p[e1] = e1 < experts ? ex[1] : 0.0f;
    __syncthreads();
    if (wave != 0) return;
    router_select_lds(experts, topK, s, s_ids);
}
// The exponentials of a 512-thread block (8 waves): thread t forms expert
// t's exp(l - max) in s.p[t] (+0 past `experts`); every wave forms the
// maximum itself from its copy of the logits. No barrier: the caller's makes
// s.p visible. s_tab must already hold kExp2Tab.
__device__ __forceinline__ void router_exps512(const float (&l)[8], int experts, const uint64_t *s_tab,
                                               RouterScratch &s) {
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float mx = l[0];
#pragma unroll
    for (int j = 1; j < 8; j++) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    wave_lds_sync();  // this wave's copy of the exp table is in LDS
    float lw = l[0];  // expert tid = lane + 64 wave
#pragma unroll
    for (int j = 1; j < 8; j++) lw = wave == j ? l[j] : lw;
    const float d[1] = {lw - mx};
    float ex[1];
    expf_or_n<1>(d, ex, s_tab);
    s.p[tid] = tid < experts ? ex[0] : 0.0f;
}
// The same routing as router_block with 512 threads: thread t forms expert
// t's exponential. Needs blockDim.x == 512 and experts <= 512.
__device__ __forceinline__ void router_block512(const float (&l)[8], int experts, int topK, const uint64_t *s_tab,
                                                RouterScratch &s, int *s_ids) {
    router_exps512(l, experts, s_tab, s);
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) != 0) return;
    router_select_lds(experts, topK, s, s_ids);
}
// Wave 0's part of router_block / router_block512: the reference sum of the
// probabilities in s.p, the selection, and the selected probabilities in
// s.val[0, topK).
__device__ __forceinline__ void router_select_lds(int experts, int topK, RouterScratch &s, int *s_ids) {
    const int lane = threadIdx.x & 63;
    float p[8];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) p[j] = s.p[lane + 64 * j];
#pragma unroll
    for (int j = 0; j < 8; j++) sum = sum + p[j];
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, tree_sum64(sum))));
    const float inv = 1.0f / sum;
    int key[8];
#pragma unroll
    for (int j = 0; j < 8; j++) key[j] = select_key(p[j] * inv, lane + 64 * j < experts);
    // IDs into s_ids, selected probabilities into s.val (for router_weights
    // once the block has issued its expert loads: the IDs alone gate those)
    select_ranked(key, experts, topK, s, s_ids);
}

// ---------------------------------------------------------- routing by logit
// A routing split in two so that expert loads need not wait for the
// exponentials. Probabilities are p = fl(fl(expf(l - max)) * inv), each step
// non-decreasing in l for every l where the rounding of expf is monotone, so
// the reference's selection (kernels/strata.cu:255-265: p descending, lower
// ID on ties) is nearly always the top-topK by (logit descending, lower ID);
// select_by_logit finds that candidate from the logits alone, and
// router_confirm_lds later proves or replaces it from the probabilities.
//
// Order key of a logit: its bits mapped so that unsigned comparison orders
// like the values (negative values reversed; NaNs at either end).
__device__ __forceinline__ uint32_t logit_key(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// The selection threshold over one wave's lane maxima hk (logit keys, 0 for
// none): the largest T whose bits 31..18 are set greedily such that at least
// topK lanes have hk >= T, as in select_ranked. Any T at or below the topK-th
// largest lane maximum keeps every one of the topK largest entries at or
// above it, and so does a T found over a subset of the entries. Returns 0
// when fewer than topK lanes hold an entry.
__device__ __forceinline__ uint32_t logit_threshold(uint32_t hk, int topK) {
    if (popc64(__ballot(hk != 0u)) < topK) return 0u;
    uint32_t T = 0;
#pragma unroll
    for (int b = 31; b >= 18; b--) {
        const uint32_t c = T | (1u << b);
        if (popc64(__ballot(hk >= c)) >= topK) T = c;
    }
    return T;
}
// One wave; lane l holds the logits of experts l + 64 j (j < 8). Writes the
// topK entries of largest (logit key, lower ID) to s_ids[0, topK), ranked,
// and returns true; returns false (s_ids untouched) when fewer than topK
// lanes hold a valid entry or more than 64 entries pass the threshold (heavy
// ties). `T0`, when not 0, is a threshold already found over a subset of
// these logits (logit_threshold); with more than 64 entries at or above it,
// the threshold of the complete set is searched and used instead.
__device__ __forceinline__ bool select_by_logit(const float (&lg)[8], int experts, int topK, uint32_t T0,
                                                RouterScratch &x, int *s_ids) {
    const int lane = threadIdx.x & 63;
    uint32_t k[8], hk = 0;
    uint64_t Q[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        k[j] = lane + 64 * j < experts ? logit_key(lg[j]) : 0u;
        hk = max(hk, k[j]);
        Q[j] = ((uint64_t)k[j] << 9) | (uint64_t)(511 - (lane + 64 * j));
    }
    bool in[8];
    if (T0 != 0u) {
#pragma unroll
        for (int j = 0; j < 8; j++) in[j] = k[j] != 0u && k[j] >= T0;
        if (rank_candidates(Q, in, topK, x, s_ids, false)) return true;
    }
    const uint32_t T = logit_threshold(hk, topK);
    if (T == 0u) return false;
#pragma unroll
    for (int j = 0; j < 8; j++) in[j] = k[j] != 0u && k[j] >= T;
    return rank_candidates(Q, in, topK, x, s_ids, false);
}
// One wave: the reference's probabilities for one token (kernels/strata.cu:
// 243-254); lane l holds the logits of experts l + 64 j (-FLT_MAX past
// `experts`). The maximum, the exponentials, the lane-strided sum (entries
// past `experts` add +0, which changes nothing) and its tree, then
// p = e * (1 / sum): q[j] in registers and in s.p[l + 64 j] (+0 past
// `experts`). s_tab must already hold kExp2Tab.
__device__ __forceinline__ void router_probs_wave(const float (&l)[8], int experts, const uint64_t *s_tab,
                                                  RouterScratch &s, float (&q)[8]) {
    const int lane = threadIdx.x & 63;
    float mx = l[0];
#pragma unroll
    for (int j = 1; j < 8; j++) mx = fmaxf(mx, l[j]);
    mx = wave_max(mx);
    wave_lds_sync();  // this wave's copy of the exp table is in LDS
    float d[8], e[8];
#pragma unroll
    for (int j = 0; j < 8; j++) d[j] = l[j] - mx;
    expf_or_n<8>(d, e, s_tab);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        e[j] = lane + 64 * j < experts ? e[j] : 0.0f;
        sum = sum + e[j];
    }
    sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, tree_sum64(sum))));
    const float inv = 1.0f / sum;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        q[j] = e[j] * inv;
        s.p[lane + 64 * j] = q[j];
    }
}
// One wave, after router_probs_wave (q, and the same values in s.p). With
// `spec`, s_ids[0, topK) holds select_by_logit's candidate c_0..c_{topK-1};
// it is exactly the reference's selection when p(c_0) > p(c_1) > ... >
// p(c_{topK-1}) and exactly topK entries have p >= p(c_{topK-1}): those topK
// entries are then the candidate's (each of them has p >= p(c_{topK-1})),
// every other entry has a smaller p (NaN never compares), and round k's
// unique largest is c_k. Otherwise select_ranked overwrites s_ids. The
// selected probabilities go to s.val[0, topK). Returns true when the
// candidate stood.
__device__ __forceinline__ bool router_confirm(const float (&q)[8], int experts, int topK, bool spec,
                                               RouterScratch &s, int *s_ids) {
    const int lane = threadIdx.x & 63;
    bool stood = false;
    if (spec) {
        const float P = s.p[lane < topK ? s_ids[lane] : 0];
        const float next = __builtin_bit_cast(
            float, __builtin_amdgcn_ds_bpermute(((lane + 1) & 63) << 2, __builtin_bit_cast(int, P)));
        const bool chain = lane >= topK - 1 || P > next;
        const float last = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, P), topK - 1));
        int count = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) count += popc64(__ballot(lane + 64 * j < experts && q[j] >= last));
        stood = __ballot(!chain) == 0 && count == topK;
        if (stood && lane < topK) s.val[lane] = P;
    }
    if (!stood) {
        int key[8];
#pragma unroll
        for (int j = 0; j < 8; j++) key[j] = select_key(q[j], lane + 64 * j < experts);
        select_ranked(key, experts, topK, s, s_ids);
    }
    return stood;
}

// One thread's part of the fp16 hi/lo split of X [rows x K] f32 into
// [rows][K/64][2][64] in the expert GEMMs' K order (position q of a group
// holds element 16 (q / 16) + (q / 2) % 8 + 8 (q % 2)): thread `at` (group
// at / 8, chunk c = at % 8) writes positions 8c .. 8c+7 of the group's hi and
// lo halves, i.e. elements 16w + 4h + {0, 8, 1, 9, 2, 10, 3, 11} with
// w = c / 2, h = c % 2: two float4 reads and two 16-byte writes.
__device__ __forceinline__ void split_hilo_chunk(const float *__restrict__ X, _Float16 *__restrict__ out, int64_t at,
                                                 int64_t groups) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const int64_t rg = at >> 3;
    if (rg >= groups) return;
    const int c = (int)(at & 7), src = 16 * (c >> 1) + 4 * (c & 1);
    const float4 a = *(const float4 *)(X + rg * 64 + src), b = *(const float4 *)(X + rg * 64 + src + 8);
    const float x[8] = {a.x, b.x, a.y, b.y, a.z, b.z, a.w, b.w};
    h8 hi, lo;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const _Float16 h = (_Float16)x[u];
        hi[u] = h;
        lo[u] = (_Float16)(x[u] - (float)h);
    }
    *(h8 *)(out + rg * 128 + 8 * c) = hi;
    *(h8 *)(out + rg * 128 + 64 + 8 * c) = lo;
}

}  // namespace sm
