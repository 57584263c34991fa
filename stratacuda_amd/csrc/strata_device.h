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
__device__ __forceinline__ float expf_or(float x) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double Shift = 0x1.8p+52;
    uint32_t ux = __float_as_uint(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + Shift;
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - Shift;
    double r = z - kd;
    uint64_t t = kExp2Tab[ki % 32] + (ki << 47);
    double s = __longlong_as_double((long long)t);
    double zz = C0 * r + C1;
    double r2 = r * r;
    double y = C2 * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    return (float)y;
}
// kernels/strata.cu:7-8
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf_or(-x)); }
__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }

// --------------------------------------------------------- wave reductions
// Tree sum over the 64 lanes in the reference order (s = 32, 16, ..., 1: lane
// l adds lane l+s). The returned value is valid in lane 0.
__device__ __forceinline__ float tree_sum64(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = v + __shfl_down(v, s, 64);
    return v;
}
__device__ __forceinline__ float tree_max64(float v) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) v = fmaxf(v, __shfl_down(v, s, 64));
    return v;
}
// Sum over groups of `width` consecutive lanes (valid in the group's first lane).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int s = WIDTH / 2; s > 0; s >>= 1) v += __shfl_down(v, s, 64);
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

// kernels/strata.cu:240-270 strata_router / :479-509 strata_router_batch, one
// 64-lane wave per token. Probabilities live in registers: lane l holds the
// experts l, l+64, ... (at most 8 of them for 512 experts).
__device__ __forceinline__ void router_wave(const float *Logits, int *Ids, float *Weights, int experts, int topK) {
    const int lane = threadIdx.x & 63;
    float p[8];
    float mx = -3.402823e38f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int e = lane + 64 * j;
        if (e < experts) mx = fmaxf(mx, Logits[e]);
    }
    mx = __shfl(sm::tree_max64(mx), 0, 64);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int e = lane + 64 * j;
        p[j] = 0.0f;
        if (e < experts) {
            p[j] = sm::expf_or(Logits[e] - mx);
            sum = sum + p[j];
        }
    }
    float inv = 1.0f / __shfl(sm::tree_sum64(sum), 0, 64);
#pragma unroll
    for (int j = 0; j < 8; j++) p[j] = p[j] * inv;
    float mine = 0.0f;  // lane k keeps selected[k]
    for (int k = 0; k < topK; ++k) {
        float best = -1.0f;
        int id = experts;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int e = lane + 64 * j;
            if (e < experts && (p[j] > best || (p[j] == best && e < id))) {
                best = p[j];
                id = e;
            }
        }
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) {
            float v = __shfl_down(best, s, 64);
            int w = __shfl_down(id, s, 64);
            if (v > best || (v == best && w < id)) {
                best = v;
                id = w;
            }
        }
        best = __shfl(best, 0, 64);
        id = __shfl(id, 0, 64);
        if (lane == 0) Ids[k] = id;
        if (lane == k) mine = best;
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (id == lane + 64 * j) p[j] = -1.0f;
    }
    float denom = 0.0f;
    for (int k = 0; k < topK; ++k) denom = denom + __shfl(mine, k, 64);
    denom = fmaxf(denom, 0.00006103515625f);
    if (lane < topK) Weights[lane] = mine / denom;
}

}  // namespace sm
