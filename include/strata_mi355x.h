/*
 * strata_mi355x.h - C ABI of the MI355X (gfx950) mixture-of-experts library
 * (libstrata_mi355x.so). Plain integers, pointers and sizes only.
 *
 * Device buffers are identified by handles: the device address returned by
 * sm_alloc. The library records the size of every allocation and checks each
 * launch's accesses against those sizes on the host before anything runs;
 * a handle that sm_alloc did not return is rejected.
 *
 * Return codes: 0 on success, a negative SM_E* value on failure; the message
 * of the last failure on a context is sm_last_error(ctx).
 *
 * Ordering: every call on one context is issued in order on that context's
 * HIP stream (default priority). sm_read waits for the copy; sm_write waits
 * until the host source may be reused; everything else is asynchronous until
 * sm_sync. One context must not be used from two threads at once.
 *
 * Reference interfaces each entry replaces (file:line in SamG-Coder/StrataCuda):
 *   sm_alloc / sm_free / sm_write / sm_read / sm_copy / sm_zero / sm_sync
 *       GpuBackend.alloc/free/write/read/copy/zero/idle, src/backend.js:84-119;
 *       WasmBackend, src/backend.js:128-149; ThreadedProgram.alloc/write/read,
 *       vendor/webcuda/src/wasm/runtime.js:7-9
 *   sm_run
 *       backend.run(name, args, groups), src/backend.js:101-113 and :144;
 *       the per-entry C ABI cw_<entry>(gx, gy, gz, params...),
 *       vendor/webcuda/src/wasm/compile.mjs:37, dispatched by
 *       ThreadedProgram.dispatch, vendor/webcuda/src/wasm/runtime.js:10-15
 *   sm_moe_route / sm_moe_dispatch / sm_moe_layer / sm_moe_layer_workspace
 *       the MoE stage driven from JavaScript by StrataEngine.moe,
 *       src/engine.js:133-156 (decode), and PromptBatch.moe,
 *       src/prefill.js:52-78 (prompt): router projection, strata_router,
 *       host grouping, per-expert strata_q2_gate_up / strata_q2_down,
 *       shared expert, shared gate and strata_moe_combine, done on the device
 *       without a host readback of the routed IDs
 *   sm_synth_*
 *       no reference counterpart: seeded synthetic inputs for tests and the
 *       benchmark, generated on the device
 */
#ifndef STRATA_MI355X_H
#define STRATA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SM_OK 0
#define SM_E_HIP (-1)        /* a HIP runtime call failed */
#define SM_E_ARG (-2)        /* invalid argument (RangeError in the reference) */
#define SM_E_BOUNDS (-3)     /* an access would leave a buffer (buffer layout error) */
#define SM_E_HANDLE (-4)     /* not a live handle of this context */
#define SM_E_NOKERNEL (-5)   /* unknown kernel name (src/backend.js:103) */
#define SM_E_ROUTE (-6)      /* invalid routing result detected on the device */
#define SM_E_NOMEM (-7)      /* allocation failed */
#define SM_E_FAULT (-8)      /* a device-side wait of the single-launch decode layer gave up (sm_fused_reset) */

typedef struct sm_ctx sm_ctx;

/* ---------------------------------------------------------------- context */
int sm_init(int device, sm_ctx **out);
void sm_shutdown(sm_ctx *ctx);
const char *sm_last_error(sm_ctx *ctx);
/* Writes a JSON object describing the device and counters (GpuBackend.info,
 * src/backend.js:120) into buf; returns the length or a negative code. */
int sm_info(sm_ctx *ctx, char *buf, size_t cap);

/* The single-launch decode layer (one token at hidden 2048 / ff 512; see
 * sm_moe_layer) spreads one layer over 256 blocks that wait for each other,
 * so it runs only when the device can hold all of them at once: sm_init
 * checks the CU count against the kernel's occupancy (sm_info "fusedDecode";
 * otherwise the three-kernel path runs). Every wait of the kernel is bounded:
 * one that gives up (blocks not all resident, e.g. CUs held by another
 * process) makes the layer's outputs NaN and sets a sticky fault, and so are
 * the outputs of every later such launch on the context. sm_sync and sm_read
 * then return SM_E_FAULT (the read still copies), as the reference rejects
 * read / idle after a failed dispatch (src/backend.js:95,118); the
 * reference's engine then marks the session failed (src/engine.js:195).
 * sm_fused_reset waits for the context's work and clears the fault and the
 * kernel's synchronisation words. sm_fused_fits(cus, blocks_per_cu) is the
 * selection rule (1 when 256 blocks fit). sm_fused_test_hooks exists for
 * tests of the give-up path only: spin_limit sets the polls before a wait
 * gives up (0 = the default 2^20), withhold != 0 makes the kernel's collector
 * wait for a flag no block writes, so the launch gives up with every kernel
 * still ending normally. No reference counterpart (the reference's WebGPU
 * and WASM kernels do not wait across workgroups). */
int sm_fused_fits(int compute_units, int blocks_per_cu);
int sm_fused_reset(sm_ctx *ctx);
int sm_fused_test_hooks(sm_ctx *ctx, uint32_t spin_limit, int withhold);

/* Next-layer router prefetch, a hint for the next layer call (sm_moe_layer,
 * sm_moe_block, sm_moe_layer_static) only: `Wr` (rows x width f32, 0 for
 * none) is the router matrix of the call after that one. When the next call
 * is a single-launch decode layer (one token), its blocks pull those rows
 * into the GPU's L2 caches while they wait for each other, so that the
 * following layer reads its router rows from L2 instead of HBM (each block's
 * rows on the XCD where the next launch's block of the same index reads
 * them). Any layer call clears the hint; a hint whose buffer is no longer
 * live is dropped. Results never change. No counterpart in the reference
 * (its engine prefetches expert blobs ahead of use, src/engine.js:144). */
int sm_prefetch_router(sm_ctx *ctx, uint64_t Wr, int rows, int width);

/* ---------------------------------------------------------------- buffers */
/* zero != 0 clears the new buffer; refused (SM_E_ARG) while a graph is being
 * captured. sm_zero while capturing records a fill kernel, not a memset, and
 * takes whole 32-bit words only (offset and bytes multiples of 4). */
int sm_alloc(sm_ctx *ctx, uint64_t bytes, int zero, uint64_t *handle);
int sm_free(sm_ctx *ctx, uint64_t handle);
int sm_size(sm_ctx *ctx, uint64_t handle, uint64_t *bytes);
int sm_write(sm_ctx *ctx, uint64_t dst, uint64_t dst_offset, const void *src, uint64_t bytes);
int sm_read(sm_ctx *ctx, uint64_t src, uint64_t src_offset, void *dst, uint64_t bytes);
int sm_copy(sm_ctx *ctx, uint64_t src, uint64_t src_offset, uint64_t dst, uint64_t dst_offset,
            uint64_t bytes);
int sm_zero(sm_ctx *ctx, uint64_t dst, uint64_t offset, uint64_t bytes);
int sm_sync(sm_ctx *ctx);

/* ------------------------------------------------------ kernels by name */
/* Launch a reference kernel by name with the reference's grid semantics:
 * groups = {gx, gy, gz} workgroups of 64 lanes (scripts/build.mjs:10).
 * args holds one 64-bit slot per parameter in the reference's parameter order:
 * a buffer handle for pointer parameters, the int32 or float32 bit pattern in
 * the low 32 bits for scalars. sm_kernel_signature gives the parameter list
 * as "Name:type,..." with types f32*, i32*, u32*, i32 and f32.
 * The kernels: the 16 on the MoE path (strata_project, strata_router, the Q2
 * expert family, strata_norm, strata_elementwise, strata_moe_combine, ...)
 * and the 17 that StrataEngine.step (src/engine.js:76-196) launches besides
 * them for the untrained fixture model (strata_embedding, strata_rope_*,
 * strata_hc_*, strata_conv, strata_gdn_*, strata_slice, strata_kv_append,
 * strata_attention[_gate], strata_ple_gate/_broadcast/_add, strata_argmax),
 * the dense formats (strata_bf16_project, strata_quant_gemv, strata_ple_decode,
 * strata_embed, strata_rope) and the 11 prompt-batch kernels that
 * PromptBatch (src/prefill.js:5-97) launches (strata_*_batch): all 49 of
 * kernels/strata.cu. sm_kernel_name lists them. Cells / Mapping / Indices buffers are checked
 * on the device before use (SM_E_BOUNDS), which synchronises the stream. */
int sm_run(sm_ctx *ctx, const char *name, const uint32_t groups[3], const uint64_t *args, int nargs);
int sm_kernel_count(void);
const char *sm_kernel_name(int index);
const char *sm_kernel_signature(const char *name);

/* ------------------------------------------------------- pack loading */
/* Streams `count` expert blobs of blob_bytes each, stored back to back at
 * file_offset of the pack file `path` (experts.bin: a layer's 512 blobs from
 * its manifest offset, vendor/strata/tools/pack_layer.py:68-115), into the
 * arena: blob i at arena + dst_offset + i * stride. Then checks on the device
 * that every fp16 scale of every blob (bytes [scales_offset, blob_bytes)) is
 * finite; a non-finite scale fails with SM_E_ARG naming the first such blob.
 * Replaces PackStore.readExpertBlob / prefetchExpert (src/model.js:120-167)
 * and the per-expert upload of WeightResidency.loadExpert
 * (src/residency.js:52-77): the whole layer becomes resident in one call.
 * Synchronous (returns when the copies and the check are done). */
int sm_load_experts(sm_ctx *ctx, const char *path, uint64_t file_offset, uint64_t blob_bytes, int count,
                    uint64_t arena, uint64_t dst_offset, uint64_t stride, uint64_t scales_offset);

/* ----------------------------------------------------------- MoE layer */
/* Router: logits[t, e] = X[t,:] . Wr[e,:] (+ bias[e] when bias != 0) in the
 * reference's f32 operation order, then softmax, top-k by repeated argmax
 * (lower ID wins ties) and renormalisation (kernels/strata.cu:156-165,
 * 240-270, 479-509). logits may be 0 when not wanted.
 * X [tokens x width] f32, Wr [experts x width] f32, ids/weights [tokens x topk]. */
int sm_moe_route(sm_ctx *ctx, uint64_t X, int tokens, int width, uint64_t Wr, uint64_t bias, int experts,
                 int topk, uint64_t logits, uint64_t ids, uint64_t weights);

/* Expert-contiguous dispatch of routed IDs: experts ascending, tokens
 * ascending within an expert (the within-expert order of src/prefill.js:56-61).
 * offsets [experts+1] exclusive scan of counts; rows[pos] = token;
 * parts[pos] = token*topk + k; where[token*topk + k] = pos. The checks of
 * src/engine.js:138 / src/prefill.js:57 run on the device, asynchronously:
 * an ID out of range is left out (where = -1) and sets bit 0 of the uint32
 * at workspace offset 0, an ID repeated within a token sets bit 1; the word
 * is 0 when every ID is valid. workspace_bytes of sm_moe_layer_workspace()
 * for the same shape always suffice (SM_E_ARG when too small). */
int sm_moe_dispatch(sm_ctx *ctx, uint64_t ids, int tokens, int topk, int experts, uint64_t offsets,
                    uint64_t rows, uint64_t parts, uint64_t where_, uint64_t workspace,
                    uint64_t workspace_bytes);

/* One MoE layer: Y = sigmoid(X . Wsg) * Shared(X) + sum_k w_k * Expert_{id_k}(X)
 * per token. Expert e's Q2 blob starts at arena + e*blob_stride; the shared
 * expert's blob is shared_blob. Blob layout (vendor/strata/tools/pack_layer.py:54-65):
 * gate/up codes (2*ff interleaved rows of width/4 B), down codes (width rows of
 * ff/4 B), gate/up fp16 scales, down fp16 scales; 64-weight groups; weight =
 * (code - 1) * scale. width and ff must be multiples of 64.
 * ids/weights (tokens x topk) receive the routing. workspace must hold
 * sm_moe_layer_workspace(...) bytes. Up to 6 tokens run the decode kernels
 * (GEMV, one grid slice per token); more tokens run dispatch + grouped MFMA
 * GEMMs. */
int sm_moe_layer_workspace(int tokens, int width, int ff, int experts, int topk, uint64_t *bytes);
int sm_moe_layer(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena,
                 uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts,
                 int topk, uint64_t Y, uint64_t ids, uint64_t weights, uint64_t workspace,
                 uint64_t workspace_bytes);

/* Diagnostics of the batch router (no reference counterpart). For 512 or
 * more tokens sm_moe_layer / sm_moe_block route with a certified router: every
 * logit approximately on fp16 MFMA with a worst-case error bound, then the
 * exact reference-order logits of the experts near each token's top-k
 * boundary only; a token whose order the bound cannot certify (ties within
 * rounding, underflow, NaN or inf, more than 64 candidates) takes every
 * logit exactly. IDs and their order are the reference's either way; the
 * routing weights agree with the reference's to a few ulp. After such a
 * call (synchronously) this reads the workspace's per-token records:
 * candidates = exact logits formed over all tokens, fallbacks = tokens that
 * took the exact path. Returns the number of tokens covered, 0 when the
 * batch did not use the certified router, or a negative code. */
int sm_moe_route_stats(sm_ctx *ctx, uint64_t workspace, int tokens, int width, int ff, int experts, int topk,
                       uint64_t *candidates, int *fallbacks);

/* Allocation-free variant of sm_moe_layer for the decode path (no reference
 * counterpart: it is for callers that cannot allocate, such as code under
 * HIP graph capture or a serving loop that forbids hipMalloc). Same
 * arguments as sm_moe_layer without the workspace: the decode scratch
 * (router logits, per-group fixed-point activations, hidden rows) lives in a
 * static device array of 2 MiB per GPU, held until the process ends. Runs
 * the decode kernels only: up to 6 tokens the same bits as sm_moe_layer
 * (which runs them too), from 7 to 16 the same routing and outputs within
 * the layer tolerance of its GEMM path. tokens <= 16, and the shape's decode
 * scratch must fit in 2 MiB (hidden 2048 / ff 512 / 512 experts / top-10
 * needs 512 KiB at 16 tokens); larger requests fail with SM_E_ARG. Nothing
 * is allocated (no hipMalloc / hipFree) and the scratch needs no clearing:
 * every word a call reads, that call wrote first. Every call on one GPU
 * shares the array; a call on another stream (or context) than the previous
 * one waits for that call on the GPU, so such calls run in turn instead of
 * racing. Calls on a capturing stream are not ordered by the library (the
 * caller orders them within its graph). Refused while stage timing is
 * enabled. */
int sm_moe_layer_static(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena,
                        uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff,
                        int experts, int topk, uint64_t Y, uint64_t ids, uint64_t weights);

/* One block of a stacked decoder built on the MoE stage, the per-layer step
 * of the 48-layer stack (no single reference entry point; it composes
 * strata_norm mode 0 with scale 1, kernels/strata.cu:214-227, the MoE stage of
 * sm_moe_layer, and strata_elementwise mode 5, :230-236):
 *   Hout = H + MoE(RMSNorm(H; gamma, eps))          per token.
 * gamma is [width] f32. Results are bit-identical to running those three
 * steps separately. Up to 6 tokens fold the normalisation into the router
 * kernel and the residual into the down kernel; more tokens normalise into
 * the workspace (up to 512 tokens together with the GEMMs' fp16 hi/lo
 * activations) and add the residual in the combine. Hout may be H itself;
 * otherwise it must not overlap H. workspace must hold
 * sm_moe_block_workspace(...) bytes. */
int sm_moe_block_workspace(int tokens, int width, int ff, int experts, int topk, uint64_t *bytes);
int sm_moe_block(sm_ctx *ctx, uint64_t H, int tokens, uint64_t gamma, float eps, uint64_t Wr, uint64_t bias,
                 uint64_t arena, uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff,
                 int experts, int topk, uint64_t Hout, uint64_t ids, uint64_t weights, uint64_t workspace,
                 uint64_t workspace_bytes);

/* ---------------------------------------------------------------- timing */
/* Events on the context's stream (the stream every launch above uses). */
int sm_event_record(sm_ctx *ctx, int slot);          /* slot in [0, 64) */
int sm_event_elapsed(sm_ctx *ctx, int start_slot, int end_slot, float *ms);

/* Per-stage timing of sm_moe_layer (no reference counterpart; the reference
 * exposes counters through GpuBackend.info, src/backend.js:120). When enabled,
 * an event is recorded on the context's stream at every stage boundary;
 * sm_stage_report synchronises and returns, per stage, the accumulated
 * milliseconds and call counts since enabling (n >= 9 slots). Stages:
 * 0 decode route, 1 decode gate/up, 2 decode down+combine, 3 prefill route
 * (router GEMM + top-k), 4 prefill dispatch, 5 prefill gate/up GEMM,
 * 6 prefill down GEMM, 7 prefill combine, 8 the single-launch decode layer
 * (one token at hidden 2048 / ff 512 / top-k <= 10; it runs when bits 0, 1,
 * 2 and 8 are all set, otherwise stages 0-2 run as three kernels). Returns
 * the number of stages. */
int sm_stage_timing(sm_ctx *ctx, int enable);
int sm_stage_report(sm_ctx *ctx, double *total_ms, uint64_t *calls, int n);
/* Runs only the sm_moe_layer stages whose bit (1 << stage) is set; the
 * default is all. A profiling aid: the caller must already have run the
 * skipped stages on the same workspace, ids and weights. */
int sm_stage_select(sm_ctx *ctx, uint32_t mask);

/* HIP graphs of launch sequences (no reference counterpart; the reference
 * batches up to 128 dispatches per WebGPU submit, src/backend.js:76-83).
 * Between sm_graph_begin and sm_graph_end, launches on the context are
 * captured instead of run; calls that synchronise (read, write, free, sync,
 * index validation of reference kernels) fail while capturing. */
int sm_graph_begin(sm_ctx *ctx);
int sm_graph_end(sm_ctx *ctx, int *graph_id);
int sm_graph_launch(sm_ctx *ctx, int graph_id);
int sm_graph_free(sm_ctx *ctx, int graph_id);

/* ------------------------------------------------------ synthetic inputs */
/* No reference counterpart. Deterministic seeded data, bit-identical to the
 * CPU oracle's generator:
 *   sm_synth_normal: f32 values sigma * normal(seed, stream, i)
 *   sm_synth_uniform_pm: f32 values 1 + amp * U(-1, 1)
 *   sm_synth_blobs: `count` Q2 blobs at dst + i*stride, blob i from stream
 *                   first_stream + i (codes uniform, scales fp16(|sigma*N|)) */
int sm_synth_normal(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t n, uint64_t seed,
                    uint64_t stream, double sigma);
int sm_synth_uniform_pm(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t n, uint64_t seed,
                        uint64_t stream, double amp);
int sm_synth_blobs(sm_ctx *ctx, uint64_t dst, uint64_t offset_bytes, uint64_t stride, int count, int width,
                   int ff, uint64_t seed, uint64_t first_stream, double sigma);

#ifdef __cplusplus
}
#endif
#endif /* STRATA_MI355X_H */
