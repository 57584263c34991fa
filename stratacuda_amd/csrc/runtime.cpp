// Context, buffer registry, copies, events and the MoE entry points of
// libstrata_mi355x.so. Every device buffer the library touches is an
// allocation it made, so every launch is bounds-checked on the host first.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "internal.h"

namespace smi {

int fail(sm_ctx *ctx, int code, const std::string &msg) {
    if (ctx) ctx->error = msg;
    return code;
}

int hip_fail(sm_ctx *ctx, hipError_t err, const char *what) {
    return fail(ctx, SM_E_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

int need(sm_ctx *ctx, uint64_t handle, uint64_t bytes, const char *what) {
    auto it = ctx->buffers.find(handle);
    if (it == ctx->buffers.end())
        return fail(ctx, SM_E_HANDLE, std::string(what) + ": not a live buffer of this context");
    if (it->second < bytes)
        return fail(ctx, SM_E_BOUNDS, std::string(what) + ": needs " + std::to_string(bytes) + " bytes, buffer has " +
                                          std::to_string(it->second));
    return SM_OK;
}

// A layer call's use of the router-prefetch hint (sm_prefetch_router): kept
// only while its buffer is still a live buffer of this context holding the
// named rows; cleared once the call is issued (a hint serves one call).
static void check_prefetch(sm_ctx *ctx) {
    if (!ctx->next_wr) return;
    auto it = ctx->buffers.find(ctx->next_wr);
    if (it == ctx->buffers.end() || it->second < (uint64_t)ctx->next_rows * ctx->next_width * 4) ctx->next_wr = 0;
}
static int clear_prefetch(sm_ctx *ctx, int rc) {
    ctx->next_wr = 0;
    return rc;
}

int launched(sm_ctx *ctx) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(ctx, err, "kernel launch");
    ctx->launches++;
    return SM_OK;
}

int fork_aux(sm_ctx *ctx) {
    hipError_t err = hipEventRecord(ctx->fork, ctx->stream);
    if (err == hipSuccess) err = hipStreamWaitEvent(ctx->aux, ctx->fork, 0);
    return err == hipSuccess ? SM_OK : hip_fail(ctx, err, "stream fork");
}

int join_aux(sm_ctx *ctx) {
    hipError_t err = hipEventRecord(ctx->join, ctx->aux);
    if (err == hipSuccess) err = hipStreamWaitEvent(ctx->stream, ctx->join, 0);
    return err == hipSuccess ? SM_OK : hip_fail(ctx, err, "stream join");
}

int aux_mark(sm_ctx *ctx) {
    const hipError_t err = hipEventRecord(ctx->mid, ctx->aux);
    return err == hipSuccess ? SM_OK : hip_fail(ctx, err, "aux mark");
}

int wait_aux_mark(sm_ctx *ctx) {
    const hipError_t err = hipStreamWaitEvent(ctx->stream, ctx->mid, 0);
    return err == hipSuccess ? SM_OK : hip_fail(ctx, err, "wait for aux mark");
}

// Folds recorded stage events into the per-stage totals (synchronises).
static int stage_fold(sm_ctx *ctx) {
    if (ctx->marks.empty()) return SM_OK;
    hipError_t e = hipEventSynchronize(ctx->stage_pool[ctx->marks.back().event]);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventSynchronize");
    for (size_t i = 0; i + 1 < ctx->marks.size(); i++) {
        const auto &a = ctx->marks[i], &b = ctx->marks[i + 1];
        if (a.stage < 0) continue;
        float ms = 0.0f;
        e = hipEventElapsedTime(&ms, ctx->stage_pool[a.event], ctx->stage_pool[b.event]);
        if (e != hipSuccess) return hip_fail(ctx, e, "hipEventElapsedTime");
        ctx->stage_ms[a.stage] += ms;
        ctx->stage_calls[a.stage] += 1;
    }
    ctx->marks.clear();
    ctx->stage_used = 0;
    return SM_OK;
}

int stage_mark(sm_ctx *ctx, int stage) {
    if (!ctx->stage_timing) return SM_OK;
    if (ctx->stage_used == ctx->stage_pool.size()) {
        // Pool exhausted: fold at a call boundary only (a mark of -1 ends a call).
        if (int rc = stage_fold(ctx)) return rc;
    }
    size_t idx = ctx->stage_used++;
    hipError_t e = hipEventRecord(ctx->stage_pool[idx], ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipEventRecord");
    ctx->marks.push_back({stage, idx});
    if (stage < 0 && ctx->stage_used + 16 > ctx->stage_pool.size()) return stage_fold(ctx);
    return SM_OK;
}

}  // namespace smi

using namespace smi;

#define HIP_TRY(ctx, call)                                    \
    do {                                                      \
        hipError_t e_ = (call);                               \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
    } while (0)

extern "C" {

int sm_init(int device, sm_ctx **out) {
    if (!out) return SM_E_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return SM_E_HIP;
    if (device < 0 || device >= count) return SM_E_ARG;
    sm_ctx *ctx = new sm_ctx();
    ctx->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return SM_E_HIP;
    }
    if (hipStreamCreateWithFlags(&ctx->aux, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->join, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->mid, hipEventDisableTiming) != hipSuccess) {
        sm_shutdown(ctx);
        return SM_E_HIP;
    }
    for (auto &e : ctx->events) {
        if (hipEventCreate(&e) != hipSuccess) {
            sm_shutdown(ctx);
            return SM_E_HIP;
        }
    }
    if (hipMalloc((void **)&ctx->counters, kCounterWords * sizeof(uint32_t)) != hipSuccess ||
        hipMalloc((void **)&ctx->attn_scores, kAttnScoresBytes) != hipSuccess ||
        hipMemset(ctx->counters, 0, kCounterWords * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        sm_shutdown(ctx);
        return SM_E_HIP;
    }
    if (static_scratch_init(ctx) != SM_OK) {
        sm_shutdown(ctx);
        return SM_E_HIP;
    }
    // The fused decode layer's host-visible fault word: coherent pinned host
    // memory, so a kernel's store reaches it without a copy.
    if (hipHostMalloc((void **)&ctx->fault_host, 64, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) {
        ctx->fault_host = nullptr;
        sm_shutdown(ctx);
        return SM_E_HIP;
    }
    *(volatile uint32_t *)ctx->fault_host = 0;
    if (hipHostGetDevicePointer((void **)&ctx->fault_dev, ctx->fault_host, 0) != hipSuccess || !ctx->fault_dev ||
        fused_decode_init(ctx) != SM_OK) {
        sm_shutdown(ctx);
        return SM_E_HIP;
    }
    *out = ctx;
    return SM_OK;
}

void sm_shutdown(sm_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->aux) (void)hipStreamSynchronize(ctx->aux);
    for (auto &kv : ctx->buffers) (void)hipFree((void *)kv.first);
    ctx->buffers.clear();
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->attn_scores) (void)hipFree(ctx->attn_scores);
    pack_release(ctx);
    for (auto &e : ctx->stage_pool) (void)hipEventDestroy(e);
    for (auto &g : ctx->graphs)
        if (g) (void)hipGraphExecDestroy(g);
    for (auto &g : ctx->graph_sources)
        if (g) (void)hipGraphDestroy(g);
    if (ctx->fault_host) (void)hipHostFree(ctx->fault_host);
    for (auto &e : ctx->events)
        if (e) (void)hipEventDestroy(e);
    if (ctx->fork) (void)hipEventDestroy(ctx->fork);
    if (ctx->join) (void)hipEventDestroy(ctx->join);
    if (ctx->mid) (void)hipEventDestroy(ctx->mid);
    if (ctx->aux) (void)hipStreamDestroy(ctx->aux);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char *sm_last_error(sm_ctx *ctx) { return ctx ? ctx->error.c_str() : "no context"; }

int sm_info(sm_ctx *ctx, char *buf, size_t cap) {
    if (!ctx || !buf) return SM_E_ARG;
    hipDeviceProp_t p;
    HIP_TRY(ctx, hipGetDeviceProperties(&p, ctx->device));
    // The fused decode layer's sticky fault word (a wait that gave up); read
    // after a synchronisation, so only outside a capture (-1 while capturing).
    long long faults = -1;
    if (!ctx->capturing) {
        uint32_t f = 0;
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        HIP_TRY(ctx, hipMemcpy(&f, ctx->counters + fused_fault_word(), sizeof(f), hipMemcpyDeviceToHost));
        faults = f | *(volatile uint32_t *)ctx->fault_host;
    }
    int n = snprintf(buf, cap,
                     "{\"backend\":\"hip\",\"device\":%d,\"name\":\"%s\",\"arch\":\"%s\",\"computeUnits\":%d,"
                     "\"globalMemoryBytes\":%llu,\"dispatches\":%llu,\"allocatedBytes\":%llu,\"buffers\":%zu,"
                     "\"uploadedBytes\":%llu,\"readbackBytes\":%llu,\"fusedDecode\":%s,\"fusedDecode2560\":%s,"
                     "\"fusedDecodeFault\":%lld}",
                     ctx->device, p.name, p.gcnArchName, p.multiProcessorCount, (unsigned long long)p.totalGlobalMem,
                     (unsigned long long)ctx->launches, (unsigned long long)ctx->allocated, ctx->buffers.size(),
                     (unsigned long long)ctx->bytes_written, (unsigned long long)ctx->bytes_read,
                     ctx->fused_capable ? "true" : "false", ctx->fused_capable_rg ? "true" : "false", faults);
    return n;
}

int sm_fused_fits(int compute_units, int blocks_per_cu) { return fused_fits(compute_units, blocks_per_cu) ? 1 : 0; }

int sm_fused_reset(sm_ctx *ctx) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx) return SM_E_ARG;
    // Every queued launch has ended (each wait is bounded) before the
    // synchronisation area is cleared: go words, flags and tags back to 0
    // (the next launch is number 1, which nothing left behind carries), and
    // the fault word with its host mirror.
    HIP_TRY(ctx, hipStreamSynchronize(ctx->aux));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipMemsetAsync(ctx->counters + kFusedSyncBase, 0, (size_t)fused_sync_words() * sizeof(uint32_t),
                                ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    *(volatile uint32_t *)ctx->fault_host = 0;
    return SM_OK;
}

int sm_prefetch_router(sm_ctx *ctx, uint64_t Wr, int rows, int width) {
    if (!ctx) return SM_E_ARG;
    if (Wr && (rows <= 0 || rows > 4096 || width <= 0 || width % 64 != 0 || width > 8192))
        return fail(ctx, SM_E_ARG, "prefetch: 1-4096 rows and a width that is a multiple of 64 up to 8192");
    if (Wr) {
        if (int rc = need(ctx, Wr, (uint64_t)rows * (uint64_t)width * 4, "prefetch router")) return rc;
    }
    ctx->next_wr = Wr;
    ctx->next_rows = rows;
    ctx->next_width = width;
    return SM_OK;
}

int sm_fused_test_hooks(sm_ctx *ctx, uint32_t spin_limit, int withhold) {
    if (!ctx) return SM_E_ARG;
    if (ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    ctx->fused_spin_limit = spin_limit ? spin_limit : (1u << 20);
    ctx->fused_withhold = withhold ? 1u : 0u;
    return SM_OK;
}

int sm_alloc(sm_ctx *ctx, uint64_t bytes, int zero, uint64_t *handle) {
    if (!ctx || !handle) return SM_E_ARG;
    if (bytes == 0) return fail(ctx, SM_E_ARG, "allocation must be at least 1 byte");
    // A zero fill would be a memset node in a captured graph.
    if (zero && ctx->capturing) return fail(ctx, SM_E_ARG, "a zero-filled allocation is not allowed while capturing a graph");
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return fail(ctx, SM_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    if (zero) {
        e = hipMemsetAsync(p, 0, bytes, ctx->stream);
        if (e != hipSuccess) {
            (void)hipFree(p);
            return hip_fail(ctx, e, "hipMemsetAsync");
        }
    }
    ctx->buffers[(uint64_t)p] = bytes;
    ctx->allocated += bytes;
    *handle = (uint64_t)p;
    return SM_OK;
}

int sm_free(sm_ctx *ctx, uint64_t handle) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx) return SM_E_ARG;
    auto it = ctx->buffers.find(handle);
    if (it == ctx->buffers.end()) return fail(ctx, SM_E_HANDLE, "free: not a live buffer of this context");
    // Kernels already queued may still read the buffer.
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipFree((void *)handle));
    ctx->allocated -= it->second;
    ctx->buffers.erase(it);
    return SM_OK;
}

int sm_size(sm_ctx *ctx, uint64_t handle, uint64_t *bytes) {
    if (!ctx || !bytes) return SM_E_ARG;
    auto it = ctx->buffers.find(handle);
    if (it == ctx->buffers.end()) return fail(ctx, SM_E_HANDLE, "size: not a live buffer of this context");
    *bytes = it->second;
    return SM_OK;
}

int sm_write(sm_ctx *ctx, uint64_t dst, uint64_t dst_offset, const void *src, uint64_t bytes) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx || (!src && bytes)) return SM_E_ARG;
    if (int rc = need(ctx, dst, dst_offset + bytes, "write")) return rc;
    if (!bytes) return SM_OK;
    HIP_TRY(ctx, hipMemcpyAsync((char *)dst + dst_offset, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    ctx->bytes_written += bytes;
    return SM_OK;
}

// After a synchronisation: SM_E_FAULT when a wait of the single-launch
// decode layer gave up (its outputs, and those of every later launch until
// sm_fused_reset, are NaN).
static int fused_fault_check(sm_ctx *ctx) {
    if (ctx->fault_host && *(volatile uint32_t *)ctx->fault_host)
        return fail(ctx, SM_E_FAULT,
                    "the single-launch decode layer gave up waiting for other blocks (not all of them resident); "
                    "its outputs are NaN until sm_fused_reset");
    return SM_OK;
}

int sm_read(sm_ctx *ctx, uint64_t src, uint64_t src_offset, void *dst, uint64_t bytes) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx || (!dst && bytes)) return SM_E_ARG;
    if (int rc = need(ctx, src, src_offset + bytes, "read")) return rc;
    if (bytes) HIP_TRY(ctx, hipMemcpyAsync(dst, (const char *)src + src_offset, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    ctx->bytes_read += bytes;
    return fused_fault_check(ctx);
}

int sm_copy(sm_ctx *ctx, uint64_t src, uint64_t src_offset, uint64_t dst, uint64_t dst_offset, uint64_t bytes) {
    if (!ctx) return SM_E_ARG;
    if (int rc = need(ctx, src, src_offset + bytes, "copy source")) return rc;
    if (int rc = need(ctx, dst, dst_offset + bytes, "copy destination")) return rc;
    if (bytes)
        HIP_TRY(ctx, hipMemcpyAsync((char *)dst + dst_offset, (const char *)src + src_offset, bytes,
                                    hipMemcpyDeviceToDevice, ctx->stream));
    return SM_OK;
}

int sm_zero(sm_ctx *ctx, uint64_t dst, uint64_t offset, uint64_t bytes) {
    if (!ctx) return SM_E_ARG;
    if (int rc = need(ctx, dst, offset + bytes, "zero")) return rc;
    if (!bytes) return SM_OK;
    if (ctx->capturing) {
        // No memset node in a captured graph: a fill kernel instead, which
        // clears whole 32-bit words only.
        if (offset % 4 || bytes % 4)
            return fail(ctx, SM_E_ARG, "while capturing a graph, zero takes whole 32-bit words");
        return zero_words(ctx, (char *)dst + offset, bytes / 4);
    }
    HIP_TRY(ctx, hipMemsetAsync((char *)dst + offset, 0, bytes, ctx->stream));
    return SM_OK;
}

int sm_sync(sm_ctx *ctx) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx) return SM_E_ARG;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return fused_fault_check(ctx);
}

int sm_stage_timing(sm_ctx *ctx, int enable) {
    if (ctx && ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    if (!ctx) return SM_E_ARG;
    if (int rc = stage_fold(ctx)) return rc;
    for (int i = 0; i < kStageCount; i++) {
        ctx->stage_ms[i] = 0.0;
        ctx->stage_calls[i] = 0;
    }
    if (enable && ctx->stage_pool.empty()) {
        ctx->stage_pool.resize(4096);
        for (auto &e : ctx->stage_pool) HIP_TRY(ctx, hipEventCreate(&e));
    }
    ctx->stage_timing = enable != 0;
    return SM_OK;
}

int sm_stage_report(sm_ctx *ctx, double *total_ms, uint64_t *calls, int n) {
    if (!ctx || !total_ms || !calls || n < kStageCount) return SM_E_ARG;
    if (int rc = stage_fold(ctx)) return rc;
    for (int i = 0; i < kStageCount; i++) {
        total_ms[i] = ctx->stage_ms[i];
        calls[i] = ctx->stage_calls[i];
    }
    return kStageCount;
}

int sm_stage_select(sm_ctx *ctx, uint32_t mask) {
    if (!ctx) return SM_E_ARG;
    ctx->stage_mask = mask;
    return SM_OK;
}

int sm_graph_begin(sm_ctx *ctx) {
    if (!ctx) return SM_E_ARG;
    if (ctx->capturing) return fail(ctx, SM_E_ARG, "a capture is already open");
    if (ctx->stage_timing) return fail(ctx, SM_E_ARG, "disable stage timing before capturing a graph");
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->capturing = true;
    return SM_OK;
}

int sm_graph_end(sm_ctx *ctx, int *graph_id) {
    if (!ctx || !graph_id) return SM_E_ARG;
    if (!ctx->capturing) return fail(ctx, SM_E_ARG, "no capture is open");
    ctx->capturing = false;
    hipGraph_t graph = nullptr;
    HIP_TRY(ctx, hipStreamEndCapture(ctx->stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(ctx, e, "hipGraphInstantiate");
    }
    // The captured graph is kept until sm_graph_free, beside its executable:
    // a tool that maps an executable's nodes back to their source graph then
    // finds it alive.
    ctx->graphs.push_back(exec);
    ctx->graph_sources.push_back(graph);
    *graph_id = (int)ctx->graphs.size() - 1;
    return SM_OK;
}

int sm_graph_launch(sm_ctx *ctx, int graph_id) {
    if (!ctx || graph_id < 0 || graph_id >= (int)ctx->graphs.size() || !ctx->graphs[graph_id]) return SM_E_ARG;
    HIP_TRY(ctx, hipGraphLaunch(ctx->graphs[graph_id], ctx->stream));
    return SM_OK;
}

int sm_graph_free(sm_ctx *ctx, int graph_id) {
    if (!ctx || graph_id < 0 || graph_id >= (int)ctx->graphs.size() || !ctx->graphs[graph_id]) return SM_E_ARG;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipGraphExecDestroy(ctx->graphs[graph_id]));
    ctx->graphs[graph_id] = nullptr;
    if (ctx->graph_sources[graph_id]) HIP_TRY(ctx, hipGraphDestroy(ctx->graph_sources[graph_id]));
    ctx->graph_sources[graph_id] = nullptr;
    return SM_OK;
}

int sm_event_record(sm_ctx *ctx, int slot) {
    if (!ctx || slot < 0 || slot >= 64) return SM_E_ARG;
    HIP_TRY(ctx, hipEventRecord(ctx->events[slot], ctx->stream));
    return SM_OK;
}

int sm_event_elapsed(sm_ctx *ctx, int a, int b, float *ms) {
    if (!ctx || !ms || a < 0 || a >= 64 || b < 0 || b >= 64) return SM_E_ARG;
    HIP_TRY(ctx, hipEventSynchronize(ctx->events[b]));
    HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->events[a], ctx->events[b]));
    return SM_OK;
}

// ------------------------------------------------------------- MoE layer
static int check_geometry(sm_ctx *ctx, int tokens, int width, int ff, int experts, int topk) {
    // src/model.js:14 and src/backend.js:12-13,29
    if (tokens < 1 || width < 64 || ff < 64) return fail(ctx, SM_E_ARG, "tokens, width and ff must be positive");
    if (width % 64 || ff % 64) return fail(ctx, SM_E_ARG, "Packed expert dimensions must contain complete groups");
    if (experts < 1 || experts > 512 || topk < 1 || topk > (experts < 32 ? experts : 32))
        return fail(ctx, SM_E_ARG, "Router supports 1-512 experts and topK <= min(experts,32)");
    if ((int64_t)tokens * width > (int64_t)1 << 30 || (int64_t)tokens * topk > (int64_t)1 << 24)
        return fail(ctx, SM_E_ARG, "token batch too large");
    return SM_OK;
}

int sm_moe_route(sm_ctx *ctx, uint64_t X, int tokens, int width, uint64_t Wr, uint64_t bias, int experts, int topk,
                 uint64_t logits, uint64_t ids, uint64_t weights) {
    if (!ctx) return SM_E_ARG;
    if (int rc = check_geometry(ctx, tokens, width, 64, experts, topk)) return rc;
    return route(ctx, X, tokens, width, Wr, bias, experts, topk, logits, ids, weights, 0, 0);
}

int sm_moe_dispatch(sm_ctx *ctx, uint64_t ids, int tokens, int topk, int experts, uint64_t offsets, uint64_t rows,
                    uint64_t parts, uint64_t where_, uint64_t workspace, uint64_t workspace_bytes) {
    if (!ctx) return SM_E_ARG;
    if (int rc = check_geometry(ctx, tokens, 64, 64, experts, topk)) return rc;
    return dispatch(ctx, ids, tokens, topk, experts, offsets, rows, parts, where_, workspace, workspace_bytes, 0);
}

int sm_moe_block(sm_ctx *ctx, uint64_t H, int tokens, uint64_t gamma, float eps, uint64_t Wr, uint64_t bias,
                 uint64_t arena, uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff,
                 int experts, int topk, uint64_t Hout, uint64_t ids, uint64_t weights, uint64_t workspace,
                 uint64_t workspace_bytes) {
    if (!ctx) return SM_E_ARG;
    if (int rc = check_geometry(ctx, tokens, width, ff, experts, topk)) return rc;
    if (!(eps >= 0.0f)) return fail(ctx, SM_E_ARG, "epsilon must be >= 0");
    BlobLayout L = blob_layout(width, ff);
    if (blob_stride < L.bytes || blob_stride % 256)
        return fail(ctx, SM_E_ARG, "blob stride must be a multiple of 256 holding one blob");
    if (int rc = need(ctx, arena, blob_stride * (uint64_t)(experts - 1) + L.bytes, "expert arena")) return rc;
    if (int rc = need(ctx, shared_blob, L.bytes, "shared expert blob")) return rc;
    if (int rc = need(ctx, H, (uint64_t)tokens * width * 4, "H")) return rc;
    if (int rc = need(ctx, Hout, (uint64_t)tokens * width * 4, "Hout")) return rc;
    if (int rc = need(ctx, gamma, (uint64_t)width * 4, "gamma")) return rc;
    if (int rc = need(ctx, Wr, (uint64_t)experts * width * 4, "router weights")) return rc;
    if (int rc = need(ctx, Wsg, (uint64_t)width * 4, "shared gate weights")) return rc;
    if (bias)
        if (int rc = need(ctx, bias, (uint64_t)experts * 4, "router bias")) return rc;
    if (int rc = need(ctx, ids, (uint64_t)tokens * topk * 4, "ids")) return rc;
    if (int rc = need(ctx, weights, (uint64_t)tokens * topk * 4, "weights")) return rc;
    uint64_t ws = tokens <= kDecodeBatchMaxTokens ? moe_decode_workspace(tokens, width, ff, experts, topk)
                              : moe_prefill_workspace(tokens, width, ff, experts, topk, true);
    if (workspace_bytes < ws) return fail(ctx, SM_E_ARG, "workspace too small");
    if (int rc = need(ctx, workspace, ws, "workspace")) return rc;
    if (Hout != H && Hout < H + (uint64_t)tokens * width * 4 && H < Hout + (uint64_t)tokens * width * 4)
        return fail(ctx, SM_E_ARG, "Hout must be H itself or not overlap it");
    const BlockArgs block = {gamma, eps};
    check_prefetch(ctx);
    if (tokens <= kDecodeBatchMaxTokens)
        return clear_prefetch(ctx, moe_decode(ctx, H, tokens, Wr, bias, arena, blob_stride, shared_blob, Wsg, width, ff,
                                              experts, topk, Hout, ids, weights, workspace, workspace_bytes, &block));
    return clear_prefetch(ctx, moe_prefill(ctx, H, tokens, Wr, bias, arena, blob_stride, shared_blob, Wsg, width, ff,
                                           experts, topk, Hout, ids, weights, workspace, workspace_bytes, &block));
}

int sm_moe_block_workspace(int tokens, int width, int ff, int experts, int topk, uint64_t *bytes) {
    if (int rc = sm_moe_layer_workspace(tokens, width, ff, experts, topk, bytes)) return rc;
    if (tokens > kDecodeBatchMaxTokens) *bytes = moe_prefill_workspace(tokens, width, ff, experts, topk, true);
    return SM_OK;
}

int sm_moe_layer_workspace(int tokens, int width, int ff, int experts, int topk, uint64_t *bytes) {
    if (!bytes || tokens < 1 || width < 64 || ff < 64 || width % 64 || ff % 64 || experts < 1 || experts > 512 ||
        topk < 1 || topk > 32 || topk > experts)
        return SM_E_ARG;
    *bytes = tokens <= kDecodeBatchMaxTokens ? moe_decode_workspace(tokens, width, ff, experts, topk)
                         : moe_prefill_workspace(tokens, width, ff, experts, topk);
    return SM_OK;
}

int sm_moe_route_stats(sm_ctx *ctx, uint64_t workspace, int tokens, int width, int ff, int experts, int topk,
                       uint64_t *candidates, int *fallbacks) {
    if (!ctx || !candidates || !fallbacks) return SM_E_ARG;
    if (ctx->capturing) return fail(ctx, SM_E_ARG, "not allowed while capturing a graph");
    *candidates = 0;
    *fallbacks = 0;
    if (tokens <= kDecodeBatchMaxTokens) return 0;
    const int64_t off = moe_prefill_route_stats_offset(tokens, width, ff, experts, topk);
    if (off < 0) return 0;
    if (int rc = need(ctx, workspace, (uint64_t)off + (uint64_t)tokens * 4, "workspace")) return rc;
    std::vector<uint32_t> st((size_t)tokens);
    HIP_TRY(ctx, hipMemcpyAsync(st.data(), (const char *)workspace + off, (size_t)tokens * 4, hipMemcpyDeviceToHost,
                                ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    for (uint32_t v : st) {
        *candidates += v & 0xffffu;
        *fallbacks += (v >> 16) & 1u;
    }
    return tokens;
}

int sm_moe_layer_static(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena,
                        uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts,
                        int topk, uint64_t Y, uint64_t ids, uint64_t weights) {
    if (!ctx) return SM_E_ARG;
    if (int rc = check_geometry(ctx, tokens, width, ff, experts, topk)) return rc;
    if (tokens > kDecodeMaxTokens)
        return fail(ctx, SM_E_ARG, "the allocation-free entry runs the decode path: at most " +
                                       std::to_string(kDecodeMaxTokens) + " tokens per call");
    const uint64_t ws = moe_decode_workspace(tokens, width, ff, experts, topk);
    if (ws > kStaticScratchBytes)
        return fail(ctx, SM_E_ARG, "this shape needs " + std::to_string(ws) + " bytes of decode scratch; the static "
                                   "scratch holds " + std::to_string(kStaticScratchBytes));
    // Stage timing records host-side marks; keep this entry free of them.
    if (ctx->stage_timing) return fail(ctx, SM_E_ARG, "disable stage timing before the allocation-free entry");
    if (!ctx->scratch) return fail(ctx, SM_E_HIP, "static scratch not resolved for this device");
    BlobLayout L = blob_layout(width, ff);
    if (blob_stride < L.bytes || blob_stride % 256)
        return fail(ctx, SM_E_ARG, "blob stride must be a multiple of 256 holding one blob");
    if (int rc = need(ctx, arena, blob_stride * (uint64_t)(experts - 1) + L.bytes, "expert arena")) return rc;
    if (int rc = need(ctx, shared_blob, L.bytes, "shared expert blob")) return rc;
    if (int rc = need(ctx, X, (uint64_t)tokens * width * 4, "X")) return rc;
    if (int rc = need(ctx, Y, (uint64_t)tokens * width * 4, "Y")) return rc;
    if (int rc = need(ctx, Wr, (uint64_t)experts * width * 4, "router weights")) return rc;
    if (int rc = need(ctx, Wsg, (uint64_t)width * 4, "shared gate weights")) return rc;
    if (bias)
        if (int rc = need(ctx, bias, (uint64_t)experts * 4, "router bias")) return rc;
    if (int rc = need(ctx, ids, (uint64_t)tokens * topk * 4, "ids")) return rc;
    if (int rc = need(ctx, weights, (uint64_t)tokens * topk * 4, "weights")) return rc;
    check_prefetch(ctx);
    StaticScratchCall use(ctx);
    if (int rc = use.begin()) return clear_prefetch(ctx, rc);
    const int rc = moe_decode(ctx, X, tokens, Wr, bias, arena, blob_stride, shared_blob, Wsg, width, ff, experts, topk, Y,
                              ids, weights, (uint64_t)ctx->scratch, kStaticScratchBytes);
    if (rc) return clear_prefetch(ctx, rc);
    return clear_prefetch(ctx, use.done());
}

int sm_moe_layer(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
                 uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y, uint64_t ids,
                 uint64_t weights, uint64_t workspace, uint64_t workspace_bytes) {
    if (!ctx) return SM_E_ARG;
    if (int rc = check_geometry(ctx, tokens, width, ff, experts, topk)) return rc;
    BlobLayout L = blob_layout(width, ff);
    if (blob_stride < L.bytes || blob_stride % 256)
        return fail(ctx, SM_E_ARG, "blob stride must be a multiple of 256 holding one blob");
    if (int rc = need(ctx, arena, blob_stride * (uint64_t)(experts - 1) + L.bytes, "expert arena")) return rc;
    if (int rc = need(ctx, shared_blob, L.bytes, "shared expert blob")) return rc;
    if (int rc = need(ctx, X, (uint64_t)tokens * width * 4, "X")) return rc;
    if (int rc = need(ctx, Y, (uint64_t)tokens * width * 4, "Y")) return rc;
    if (int rc = need(ctx, Wr, (uint64_t)experts * width * 4, "router weights")) return rc;
    if (int rc = need(ctx, Wsg, (uint64_t)width * 4, "shared gate weights")) return rc;
    if (bias)
        if (int rc = need(ctx, bias, (uint64_t)experts * 4, "router bias")) return rc;
    if (int rc = need(ctx, ids, (uint64_t)tokens * topk * 4, "ids")) return rc;
    if (int rc = need(ctx, weights, (uint64_t)tokens * topk * 4, "weights")) return rc;
    uint64_t ws = tokens <= kDecodeBatchMaxTokens ? moe_decode_workspace(tokens, width, ff, experts, topk)
                              : moe_prefill_workspace(tokens, width, ff, experts, topk);
    if (workspace_bytes < ws) return fail(ctx, SM_E_ARG, "workspace too small");
    if (int rc = need(ctx, workspace, ws, "workspace")) return rc;
    check_prefetch(ctx);
    if (tokens <= kDecodeBatchMaxTokens)
        return clear_prefetch(ctx, moe_decode(ctx, X, tokens, Wr, bias, arena, blob_stride, shared_blob, Wsg, width, ff,
                                              experts, topk, Y, ids, weights, workspace, workspace_bytes));
    return clear_prefetch(ctx, moe_prefill(ctx, X, tokens, Wr, bias, arena, blob_stride, shared_blob, Wsg, width, ff,
                                           experts, topk, Y, ids, weights, workspace, workspace_bytes));
}

}  // extern "C"
