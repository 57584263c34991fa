// Host-side internals shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/strata_mi355x.h"

struct sm_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    // Second stream (default priority) for independent work inside one call,
    // forked from and joined back to `stream` with the two events.
    hipStream_t aux = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    // Marks a point on `aux` that `stream` can wait for without waiting for
    // the rest of the aux work (aux_mark / wait_aux_mark).
    hipEvent_t mid = nullptr;
    std::map<uint64_t, uint64_t> buffers;  // handle (device address) -> bytes
    std::string error;
    hipEvent_t events[64] = {};
    // kCounterWords device words (zeroed at sm_init): 254 and 255 the pack
    // loader's and the index checks' flags; from kFusedSyncBase the fused
    // decode layer's hand-off counters, go words and sticky fault word.
    uint32_t *counters = nullptr;
    // Scores of the batched prompt attention (strata_attention_batch):
    // tokens x heads x 2,048 cells, kAttnScoresBytes, allocated by sm_init.
    float *attn_scores = nullptr;
    uint64_t launches = 0, bytes_written = 0, bytes_read = 0, allocated = 0;
    // Stage timing (sm_stage_timing): events recorded at stage boundaries.
    bool stage_timing = false;
    std::vector<hipEvent_t> stage_pool;
    size_t stage_used = 0;
    struct Mark {
        int stage;       // stage that starts at this event, -1 = end of a call
        size_t event;    // index into stage_pool
    };
    std::vector<Mark> marks;
    double stage_ms[16] = {};
    uint64_t stage_calls[16] = {};
    // Stages sm_moe_layer runs (bit per Stage); all by default. A caller that
    // clears bits must have run the skipped stages on the same workspace.
    uint32_t stage_mask = 0xffffffffu;
    // Instantiated HIP graphs (sm_graph_*); nullptr marks a freed slot.
    std::vector<hipGraphExec_t> graphs;
    bool capturing = false;
    // Pinned staging buffers of sm_load_experts (allocated at first use) and
    // the events that mark their copies done.
    void *staging[2] = {nullptr, nullptr};
    hipEvent_t staged[2] = {nullptr, nullptr};
    // Device address of this device's static decode scratch (sm_init).
    void *scratch = nullptr;
    // The single-launch decode layer: enabled when all its blocks can be
    // resident at once (sm_init); its poll limit and the test-only withhold
    // switch (sm_fused_test_hooks); a pinned host word its kernels set when a
    // wait gives up (read after every synchronisation, cleared by
    // sm_fused_reset).
    bool fused_capable = false;     // hidden 2048 / ff 512
    bool fused_capable_rg = false;  // hidden 2560 / ff 640
    uint32_t fused_spin_limit = 0, fused_withhold = 0;
    uint32_t *fault_host = nullptr, *fault_dev = nullptr;  // host pointer, and its device address
    // sm_prefetch_router: the router matrix of the layer call after the next
    // one (consumed by the next single-launch decode layer)
    uint64_t next_wr = 0;
    int next_rows = 0, next_width = 0;
    // Captured graphs kept beside their executables until sm_graph_free.
    std::vector<hipGraph_t> graph_sources;
};

namespace smi {

int fail(sm_ctx *ctx, int code, const std::string &msg);
// Frees the pack loader's staging buffers (sm_shutdown).
void pack_release(sm_ctx *ctx);
int hip_fail(sm_ctx *ctx, hipError_t err, const char *what);
// Checks that `handle` is a live allocation holding at least `bytes` bytes.
int need(sm_ctx *ctx, uint64_t handle, uint64_t bytes, const char *what);
int launched(sm_ctx *ctx);  // checks hipGetLastError after a launch
// fork_aux: work queued on ctx->aux after this runs after everything queued on
// ctx->stream so far. join_aux: work queued on ctx->stream after this runs
// after everything queued on ctx->aux so far. Both are graph-capturable.
int fork_aux(sm_ctx *ctx);
int join_aux(sm_ctx *ctx);
// aux_mark: records the work queued on ctx->aux so far; wait_aux_mark: work
// queued on ctx->stream after this runs after that work (not after aux work
// queued later).
int aux_mark(sm_ctx *ctx);
int wait_aux_mark(sm_ctx *ctx);

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Stage boundaries for sm_stage_timing: stage_mark(ctx, s) records the start
// of stage s (ending the previous one); stage_mark(ctx, -1) ends the call.
enum Stage {
    kStageDecodeRoute = 0,
    kStageDecodeGateUp = 1,
    kStageDecodeDown = 2,
    kStagePrefillRoute = 3,
    kStagePrefillDispatch = 4,
    kStagePrefillGateUp = 5,
    kStagePrefillDown = 6,
    kStagePrefillCombine = 7,
    kStageDecodeFused = 8,  // the single-launch decode layer (one token)
    kStageCount = 9
};
int stage_mark(sm_ctx *ctx, int stage);
constexpr int kCounterWords = 16384;
constexpr int kFusedSyncBase = 1024;
// Index in ctx->counters of the fused decode layer's sticky fault word, and
// the size in words of its synchronisation area (from kFusedSyncBase).
uint32_t fused_fault_word();
uint32_t fused_sync_words();
// Whether kFusedBlocks blocks fit at once on `compute_units` CUs holding
// `blocks_per_cu` blocks each; fused_decode_init sets ctx->fused_capable and
// ctx->fused_capable_rg from the device's CU count and the kernels' occupancy.
bool fused_fits(int compute_units, int blocks_per_cu);
int fused_decode_init(sm_ctx *ctx);
inline bool stage_on(const sm_ctx *ctx, int stage) { return (ctx->stage_mask >> stage) & 1u; }
// Zero-fills n 32-bit words with a kernel (graph-capturable, unlike a memset node).
int zero_words(sm_ctx *ctx, void *dst, uint64_t n);

// Launchers defined in the kernel translation units.
int route(sm_ctx *ctx, uint64_t X, int tokens, int width, uint64_t Wr, uint64_t bias, int experts, int topk,
          uint64_t logits, uint64_t ids, uint64_t weights, uint64_t gate_w, uint64_t gate_out);
// Unchecked launchers on raw device pointers (callers validated the buffers).
int route_launch(sm_ctx *ctx, const float *X, int tokens, int width, const float *Wr, const float *bias, int experts,
                 int topk, float *logits, int *ids, float *weights, const float *gate_w, float *gate_out);
// The certified batch router (moe_route_cert.hip): approximate logits on
// fp16 MFMA, exact reference-order logits for the candidates near the top-k
// boundary only, per-token certification with an exact fallback. IDs and
// their order bit-exact, weights within a few ulp. route_cert_prepare
// converts W_r (fp16, the split activations' K order) into the workspace,
// and with X given also writes X's fp16 hi/lo split to Xhl (k_split_hilo's
// layout) in the same launch; route_cert_launch then needs that split. Per-token stats (uint32 candidates | 1 << 16 on a fallback) at
// route_cert_stats_offset.
// From 512 tokens on (graph replays of 8 layers on one MI355X, hidden 2048,
// 512 experts, top-10: 384 tokens 253.5 us per layer certified against 253.1
// exact, 512 tokens 265.4 against 266.2, 1024 tokens 379.5 against 397.2;
// below 384 the exact router is 1-15 us faster).
constexpr int kRouteCertMinTokens = 512;
bool route_cert_applies(int tokens, int width, int experts, int topk);
uint64_t route_cert_workspace(int tokens, int width, int experts);
uint64_t route_cert_stats_offset(int tokens, int width, int experts);
int route_cert_prepare(sm_ctx *ctx, const float *Wr, int tokens, int width, int experts, char *ws,
                       const float *X = nullptr, _Float16 *Xhl = nullptr);
int route_cert_launch(sm_ctx *ctx, const float *X, const _Float16 *Xhl, int tokens, int width, const float *Wr,
                      const float *bias, int experts, int topk, int *ids, float *weights, const float *gate_w,
                      float *gate_out, char *ws);
// M-tile bases the dispatch writes for the grouped GEMMs: segments with at
// least `split` rows in tiles of mt_big rows (big[]), the others in tiles of
// mt_small rows (small[]); each array has experts + 2 entries. When set,
// info_small / info_big receive one record of 4 ints per tile: segment,
// first row, end row of the segment, 0.
struct GemmTiling {
    int *small, *big;
    int split, mt_small, mt_big;
    int *info_small = nullptr, *info_big = nullptr;
};
int dispatch_launch(sm_ctx *ctx, const int *ids, int tokens, int topk, int experts, int *offsets, int *rows, int *parts,
                    int *where_, char *workspace, int extra_rows, const GemmTiling *tiling);
int dispatch(sm_ctx *ctx, uint64_t ids, int tokens, int topk, int experts, uint64_t offsets, uint64_t rows,
             uint64_t parts, uint64_t where_, uint64_t workspace, uint64_t workspace_bytes, int extra_rows);
uint64_t dispatch_workspace(int tokens, int experts);
// One block of the 48-layer stack around the MoE stage: the stage's input is
// RMSNorm(X; gamma, eps) (strata_norm mode 0) and its output is X + y
// (strata_elementwise mode 5). Null means the plain stage.
struct BlockArgs {
    uint64_t gamma;
    float eps;
};
// The decode (GEMV) kernels take a token dimension of up to kDecodeMaxTokens
// tokens (the allocation-free entry runs them up to there). sm_moe_layer and
// sm_moe_block run them up to kDecodeBatchMaxTokens tokens and the dispatch +
// grouped GEMM path beyond it: graph replays of 8 stack blocks on one GPU,
// decode kernels vs GEMM path, 2 tokens 22.5 vs 35.2 us per block, 4 tokens
// 33.1 vs 40.8, 6 tokens 45.2 vs 45.3, 8 tokens 53.8 vs 46.6, 12 tokens 71.7
// vs 55.5, 16 tokens 89.8 vs 57.3.
constexpr int kDecodeMaxTokens = 16;
constexpr int kDecodeBatchMaxTokens = 6;
constexpr int kDecodeBlockRouting = 4;  // up to this many tokens the gate/up blocks route
constexpr int kRouteRowsMaxTokens = 8;  // router logits one wave per (row, token) up to here
// Exact per-token top-k (strata_router order) of logits [tokens x experts].
int topk_launch(sm_ctx *ctx, const float *logits, int *ids, float *weights, int tokens, int experts, int topk);
int moe_decode(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena, uint64_t blob_stride,
               uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts, int topk, uint64_t Y,
               uint64_t ids, uint64_t weights, uint64_t workspace, uint64_t workspace_bytes,
               const BlockArgs *block = nullptr);
uint64_t moe_decode_workspace(int tokens, int width, int ff, int experts, int topk);
// The static decode scratch of sm_moe_layer_static: its size, and the lookup
// of its device address for ctx->device (sets ctx->scratch; called by sm_init
// with that device current).
constexpr uint64_t kStaticScratchBytes = 2ull << 20;
constexpr int kMaxDevices = 64;
int static_scratch_init(sm_ctx *ctx);
// One allocation-free call's use of the device's static scratch: holds the
// device's lock while the call is enqueued; begin() makes the call's stream
// wait for the previous such call when that ran on another stream, so calls
// from two streams or contexts run one after the other instead of racing on
// the shared array; done() records the call's end. Calls on a capturing
// stream are neither ordered nor recorded.
class StaticScratchCall {
  public:
    explicit StaticScratchCall(sm_ctx *ctx);
    int begin();
    int done();

  private:
    sm_ctx *ctx_;
    std::lock_guard<std::mutex> lock_;
    bool capturing_ = false;
};
// Size of ctx->attn_scores: 1,024 (token, head) rows of 2,048 cells.
constexpr uint64_t kAttnScoresBytes = 1024ull * 2048 * 4;
int moe_prefill(sm_ctx *ctx, uint64_t X, int tokens, uint64_t Wr, uint64_t bias, uint64_t arena,
                uint64_t blob_stride, uint64_t shared_blob, uint64_t Wsg, int width, int ff, int experts,
                int topk, uint64_t Y, uint64_t ids, uint64_t weights, uint64_t workspace,
                uint64_t workspace_bytes, const BlockArgs *block = nullptr);
// With block != nullptr the workspace also holds the normalised input.
uint64_t moe_prefill_workspace(int tokens, int width, int ff, int experts, int topk, bool block = false);
// Byte offset in a prefill workspace of the certified router's per-token
// stats (uint32 each), -1 when the batch does not use that router.
int64_t moe_prefill_route_stats_offset(int tokens, int width, int ff, int experts, int topk);
// strata_norm mode 0 (scale 1) over `rows` rows of `cols`, on the context's stream.
int norm_launch(sm_ctx *ctx, const float *X, const float *gamma, float *Y, int cols, int rows, float eps);

// ------------------------------------------------ kernels by name (sm_run)
// One 64-bit slot per reference parameter: a buffer handle, or the int32 /
// float32 bit pattern in the low 32 bits.
struct Args {
    const uint64_t *a;
    uint64_t ptr(int i) const { return a[i]; }
    int i32(int i) const { return (int)(uint32_t)(a[i] & 0xffffffffu); }
    float f32(int i) const {
        uint32_t u = (uint32_t)(a[i] & 0xffffffffu);
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
};
// A launcher validates the arguments and every buffer access of the grid
// (G = workgroups of 64 lanes), then launches on ctx->stream.
typedef int (*Launcher)(sm_ctx *, const uint32_t *G, Args);
struct Entry {
    const char *name;
    const char *signature;  // "Name:type,..." in the reference's parameter order
    int nargs;
    Launcher launch;
};
// The fixture model's kernels outside the MoE path (kernels_model.hip).
const Entry *model_entries(int *count);
// Recorded size of a live buffer handle in bytes, -1 when it is not one.
int64_t buf_len(sm_ctx *ctx, uint64_t handle);
// Checks on the device that idx[first + i*stride], i < n, lie in [lo, hi):
// the host cannot see device-resident indices. Synchronises the stream;
// refused while capturing.
int check_indices(sm_ctx *ctx, uint64_t buf, int64_t n, int64_t stride, int64_t first, int lo, int hi,
                  const char *what);

// Byte sizes of the regions of one Q2 expert blob.
struct BlobLayout {
    uint64_t gate_up_codes, down_codes, gate_up_scales, down_scales, bytes;
};
inline BlobLayout blob_layout(int width, int ff) {
    BlobLayout L;
    L.gate_up_codes = 0;
    L.down_codes = (uint64_t)2 * ff * width / 4;
    L.gate_up_scales = L.down_codes + (uint64_t)width * ff / 4;
    L.down_scales = L.gate_up_scales + (uint64_t)2 * ff * (width / 64) * 2;
    L.bytes = L.down_scales + (uint64_t)width * (ff / 64) * 2;
    return L;
}

}  // namespace smi
