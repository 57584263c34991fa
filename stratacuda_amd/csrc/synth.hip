// Seeded synthetic inputs generated on the device (tests and benchmark).
// No reference counterpart. The generator is integer arithmetic plus one
// IEEE double multiply per value, so the CPU oracle's independent restatement
// produces the same bits.
#include <hip/hip_runtime.h>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

__global__ void k_synth_normal(float *dst, uint64_t n, uint64_t key, double sigma) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = (float)(sm::normal_at(key, i) * sigma);
}

__global__ void k_synth_uniform_pm(float *dst, uint64_t n, uint64_t key, double amp) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        double u = (double)(sm::mix64(key + i) & 0xffffffffull) * 0x1p-31 - 1.0;
        dst[i] = (float)(1.0 + amp * u);
    }
}

// grid.y = blob index; code words then fp16 scales.
__global__ void k_synth_blobs(uint8_t *dst, uint64_t stride, uint64_t code_words, uint64_t halves, uint64_t seed,
                              uint64_t first_stream, double sigma) {
    const uint64_t b = blockIdx.y, i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint8_t *blob = dst + b * stride;
    const uint64_t stream = first_stream + b;
    if (i < code_words) {
        const uint64_t key = sm::rand_key(seed, stream);
        ((uint32_t *)blob)[i] = (uint32_t)(sm::mix64(key + i) & 0xffffffffull);
    } else if (i < code_words + halves) {
        const uint64_t jh = i - code_words, key = sm::rand_key(seed, stream + (1ull << 32));
        float v = (float)fabs(sigma * sm::normal_at(key, jh));
        ((uint16_t *)(blob + code_words * 4))[jh] = sm::f32_to_f16_bits(v);
    }
}

__global__ void k_zero_words(uint32_t *dst, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = 0u;
}

}  // namespace

namespace smi {

int zero_words(sm_ctx *ctx, void *dst, uint64_t n) {
    if (!n) return SM_OK;
    k_zero_words<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>((uint32_t *)dst, n);
    return launched(ctx);
}

}  // namespace smi

extern "C" {

int sm_synth_normal(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t n, uint64_t seed, uint64_t stream,
                    double sigma) {
    if (!ctx || offset_bytes % 4) return SM_E_ARG;
    if (int rc = need(ctx, dst, offset_bytes + n * 4, "synth destination")) return rc;
    if (!n) return SM_OK;
    uint64_t key = 0;
    {  // rand_key on the host: same integer arithmetic as the device
        uint64_t z = seed + 0x9E3779B97F4A7C15ull * (stream + 1);
        z += 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        key = z ^ (z >> 31);
    }
    k_synth_normal<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>((float *)((char *)dst + offset_bytes), n, key,
                                                                         sigma);
    return launched(ctx);
}

int sm_synth_uniform_pm(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t n, uint64_t seed, uint64_t stream,
                        double amp) {
    if (!ctx || offset_bytes % 4) return SM_E_ARG;
    if (int rc = need(ctx, dst, offset_bytes + n * 4, "synth destination")) return rc;
    if (!n) return SM_OK;
    uint64_t z = seed + 0x9E3779B97F4A7C15ull * (stream + 1);
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    uint64_t key = z ^ (z >> 31);
    k_synth_uniform_pm<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>((float *)((char *)dst + offset_bytes), n,
                                                                             key, amp);
    return launched(ctx);
}

int sm_synth_blobs(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t stride, int count, int width, int ff,
                   uint64_t seed, uint64_t first_stream, double sigma) {
    if (!ctx || count < 1 || width < 64 || ff < 64 || width % 64 || ff % 64 || offset_bytes % 4) return SM_E_ARG;
    BlobLayout L = blob_layout(width, ff);
    if (stride < L.bytes || stride % 4) return fail(ctx, SM_E_ARG, "blob stride too small");
    if (int rc = need(ctx, dst, offset_bytes + stride * (uint64_t)(count - 1) + L.bytes, "synth blobs")) return rc;
    const uint64_t code_words = L.gate_up_scales / 4, halves = (L.bytes - L.gate_up_scales) / 2;
    dim3 grid((unsigned)((code_words + halves + 255) / 256), (unsigned)count);
    k_synth_blobs<<<grid, 256, 0, ctx->stream>>>((uint8_t *)dst + offset_bytes, stride, code_words, halves, seed,
                                                 first_stream, sigma);
    return launched(ctx);
}

}  // extern "C"
