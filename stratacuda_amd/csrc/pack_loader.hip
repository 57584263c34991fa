// Loading a layer's expert blobs from a pack file (experts.bin) into the
// resident arena, the MI355X side of PackStore.readExpertBlob
// (src/model.js:160-167): blob `id` of a layer is the blob_bytes bytes at
// layer offset + id * blob_bytes of experts.bin (vendor/strata/tools/
// pack_layer.py:68-115 writes them). Instead of one read per routed expert,
// the whole layer streams into HBM once and stays resident.
//
// Host side: the file is read with pread into two pinned staging buffers in
// turn (32 MiB each, whole blobs); while one is being filled, the other is
// copied to the arena on the context's stream (a pitched copy, so the arena
// stride may exceed the blob size). Device side: every fp16 scale of every
// loaded blob (bytes [scales_offset, blob_bytes)) is checked to be finite
// (exponent field not all ones), and the first blob holding a non-finite
// scale is named in the error, as the reference rejects such blobs.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <string>

#include "internal.h"

using namespace smi;

namespace {

constexpr uint64_t kStageBytes = 32ull << 20;

// One thread per 16-byte word of a blob's scale region (8 fp16 values);
// `tail` halves past the last whole word are checked by word -1's threads.
__global__ void k_check_scales(const uint8_t *__restrict__ arena, uint64_t stride, uint64_t scales_offset,
                               uint64_t words, uint64_t tail, int count, int *__restrict__ first_bad) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t per = words + (tail ? 1 : 0);
    if (i >= per * (uint64_t)count) return;
    const int e = (int)(i / per);
    const uint64_t w = i % per;
    const uint8_t *p = arena + (uint64_t)e * stride + scales_offset;
    bool bad = false;
    if (w < words) {
        const uint4 v = ((const uint4 *)p)[w];
        const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
            bad |= (u[k] & 0x7c00u) == 0x7c00u || (u[k] & 0x7c000000u) == 0x7c000000u;
    } else {
        const uint16_t *h = (const uint16_t *)(p + words * 16);
        for (uint64_t k = 0; k < tail; k++) bad |= (h[k] & 0x7c00u) == 0x7c00u;
    }
    if (bad) atomicMin(first_bad, e);
}

int staging(sm_ctx *ctx) {
    if (ctx->staging[0]) return SM_OK;
    for (int i = 0; i < 2; i++) {
        hipError_t e = hipHostMalloc(&ctx->staging[i], kStageBytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->staged[i], hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(ctx, e, "pinned staging buffer");
    }
    return SM_OK;
}

// Reads exactly `bytes` at `offset` (pread may return short counts).
bool read_fully(int fd, void *dst, uint64_t bytes, uint64_t offset) {
    uint8_t *p = (uint8_t *)dst;
    while (bytes) {
        const ssize_t got = pread(fd, p, std::min<uint64_t>(bytes, 1ull << 30), (off_t)offset);
        if (got <= 0) return false;
        p += got;
        bytes -= (uint64_t)got;
        offset += (uint64_t)got;
    }
    return true;
}

}  // namespace

namespace smi {
void pack_release(sm_ctx *ctx) {
    for (int i = 0; i < 2; i++) {
        if (ctx->staged[i]) (void)hipEventDestroy(ctx->staged[i]);
        if (ctx->staging[i]) (void)hipHostFree(ctx->staging[i]);
        ctx->staged[i] = nullptr;
        ctx->staging[i] = nullptr;
    }
}
}  // namespace smi

extern "C" int sm_load_experts(sm_ctx *ctx, const char *path, uint64_t file_offset, uint64_t blob_bytes, int count,
                               uint64_t arena, uint64_t dst_offset, uint64_t stride, uint64_t scales_offset) {
    if (!ctx) return SM_E_ARG;
    if (ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!path) return fail(ctx, SM_E_ARG, "a pack file path is required");
    if (count < 0 || blob_bytes == 0 || stride < blob_bytes || scales_offset >= blob_bytes || scales_offset % 16 ||
        (blob_bytes - scales_offset) % 2 || dst_offset % 16 || stride % 16)
        return fail(ctx, SM_E_ARG, "sm_load_experts: blob_bytes >= 1, stride >= blob_bytes, stride and the arena "
                                   "offset 16-byte aligned, the scale region 16-byte aligned inside the blob");
    if (count == 0) return SM_OK;
    if (int rc = need(ctx, arena, dst_offset + (uint64_t)(count - 1) * stride + blob_bytes, "expert arena")) return rc;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(ctx, SM_E_ARG, std::string("Select the model file ") + path);
    struct stat st;
    const uint64_t end = file_offset + (uint64_t)count * blob_bytes;
    if (fstat(fd, &st) != 0 || (uint64_t)st.st_size < end) {
        close(fd);
        return fail(ctx, SM_E_ARG, std::string("File range out of bounds: ") + path);
    }
    if (int rc = staging(ctx)) {
        close(fd);
        return rc;
    }
    // Whole blobs per staging buffer (a blob larger than a buffer goes in
    // pieces of one row of the pitched copy: then stride == blob size only).
    const uint64_t per = std::max<uint64_t>(1, kStageBytes / blob_bytes);
    int rc = SM_OK;
    if (blob_bytes > kStageBytes && stride != blob_bytes)
        rc = fail(ctx, SM_E_ARG, "sm_load_experts: blobs above 32 MiB need stride == blob_bytes");
    uint8_t *dst = (uint8_t *)arena + dst_offset;
    if (rc == SM_OK && blob_bytes <= kStageBytes) {
        for (int e0 = 0, turn = 0; e0 < count; e0 += (int)per, turn ^= 1) {
            const int n = (int)std::min<uint64_t>(per, (uint64_t)(count - e0));
            hipError_t err = hipEventSynchronize(ctx->staged[turn]);  // the copy that used this buffer is done
            if (err != hipSuccess) { rc = hip_fail(ctx, err, "staging wait"); break; }
            if (!read_fully(fd, ctx->staging[turn], (uint64_t)n * blob_bytes, file_offset + (uint64_t)e0 * blob_bytes)) {
                rc = fail(ctx, SM_E_ARG, std::string("File read failed: ") + path);
                break;
            }
            err = hipMemcpy2DAsync(dst + (uint64_t)e0 * stride, stride, ctx->staging[turn], blob_bytes, blob_bytes,
                                   (size_t)n, hipMemcpyHostToDevice, ctx->stream);
            if (err == hipSuccess) err = hipEventRecord(ctx->staged[turn], ctx->stream);
            if (err != hipSuccess) { rc = hip_fail(ctx, err, "staging copy"); break; }
        }
    } else if (rc == SM_OK) {
        uint64_t total = (uint64_t)count * blob_bytes;
        for (uint64_t at = 0, turn = 0; at < total; at += kStageBytes, turn ^= 1) {
            const uint64_t n = std::min<uint64_t>(kStageBytes, total - at);
            hipError_t err = hipEventSynchronize(ctx->staged[turn]);
            if (err != hipSuccess) { rc = hip_fail(ctx, err, "staging wait"); break; }
            if (!read_fully(fd, ctx->staging[turn], n, file_offset + at)) {
                rc = fail(ctx, SM_E_ARG, std::string("File read failed: ") + path);
                break;
            }
            err = hipMemcpyAsync(dst + at, ctx->staging[turn], n, hipMemcpyHostToDevice, ctx->stream);
            if (err == hipSuccess) err = hipEventRecord(ctx->staged[turn], ctx->stream);
            if (err != hipSuccess) { rc = hip_fail(ctx, err, "staging copy"); break; }
        }
    }
    close(fd);
    if (rc != SM_OK) {
        (void)hipStreamSynchronize(ctx->stream);
        return rc;
    }
    // Scale check on the device: first_bad = min over blobs with a non-finite scale.
    int *first_bad = (int *)(ctx->counters + 254);
    const int init = INT_MAX;
    hipError_t err = hipMemcpyAsync(first_bad, &init, 4, hipMemcpyHostToDevice, ctx->stream);
    if (err != hipSuccess) return hip_fail(ctx, err, "scale check setup");
    const uint64_t region = blob_bytes - scales_offset, words = region / 16, tail = (region % 16) / 2;
    const uint64_t threads = (words + (tail ? 1 : 0)) * (uint64_t)count;
    k_check_scales<<<(unsigned)((threads + 255) / 256), 256, 0, ctx->stream>>>(dst, stride, scales_offset, words, tail,
                                                                               count, first_bad);
    if (int lrc = launched(ctx)) return lrc;
    int bad = INT_MAX;
    err = hipMemcpyAsync(&bad, first_bad, 4, hipMemcpyDeviceToHost, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (err != hipSuccess) return hip_fail(ctx, err, "scale check");
    ctx->bytes_written += (uint64_t)count * blob_bytes;
    if (bad != INT_MAX) return fail(ctx, SM_E_ARG, "Non-finite expert scales (blob " + std::to_string(bad) + ")");
    return SM_OK;
}
