// Reference-named kernels for sm_run (backend.run(name, args, groups)).
//
// Each kernel computes what the entry of the same name in the reference's
// kernels/strata.cu computes, in the same f32 operation order, so results are
// bit-identical to the CPU oracle. One reference workgroup (64 lanes, one
// __syncthreads tree) maps to one 64-wide wavefront; a HIP block carries four
// such logical workgroups. Reductions use cross-lane shuffles in the
// reference's tree order instead of shared memory and barriers.
//
// Before any launch the host validates the arguments the way the reference's
// validateDispatch does (src/backend.js:10-56) and, in addition, checks every
// buffer access of the requested grid against the recorded allocation sizes;
// work items whose output the reference guards away are skipped, so no kernel
// reads outside its buffers.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <type_traits>

#include "internal.h"
#include "strata_device.h"

using namespace smi;

namespace {

constexpr int kGroupsPerBlock = 4;  // logical 64-lane workgroups per 256-thread block

__device__ __forceinline__ bool logical_group(uint64_t total, uint64_t &g) {
    g = (uint64_t)blockIdx.x * kGroupsPerBlock + (threadIdx.x >> 6);
    return g < total;
}
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ uint32_t q2_code(const uint32_t *blob, int64_t word_base, int64_t index) {
    return (blob[word_base + index / 16] >> ((index % 16) * 2)) & 3u;
}
__device__ __forceinline__ float blob_half(const uint32_t *blob, int64_t s) {
    return sm::half_bits((blob[s / 2] >> ((s % 2) * 16)) & 65535u);
}

// kernels/strata.cu:19-21
__global__ void k_unpack_half(const uint32_t *Packed, float *Values, int count) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) Values[i] = sm::half_bits((Packed[i / 2] >> ((i % 2) * 16)) & 65535u);
}
// kernels/strata.cu:35-37
__global__ void k_expert_scales(const uint32_t *Blob, float *Scales, int offset, int count) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) Scales[i] = blob_half(Blob, (int64_t)offset + i);
}

// Positions per lane whose loads the projections issue together: a lane's
// sum still takes them in the reference's order, so only latency changes.
constexpr int PU = 8;

// kernels/strata.cu:156-165 strata_project and :121-130 strata_gemv.
__global__ void k_project(const float *X, const float *W, float *Y, int cols, int rows, int tokens, int outputStride,
                          int outputOffset, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= rows || token >= tokens) return;
    const float *w = W + (int64_t)row * cols, *x = X + (int64_t)token * cols;
    float sum = 0.0f;
    // The reference's lane-strided order; PU positions' loads go out first.
    for (int i0 = lane; i0 < cols; i0 += PU * 64) {
        float wv[PU], xv[PU];
#pragma unroll
        for (int u = 0; u < PU; u++) {
            const int i = min(i0 + 64 * u, cols - 1);
            wv[u] = w[i];
            xv[u] = x[i];
        }
#pragma unroll
        for (int u = 0; u < PU; u++)
            if (i0 + 64 * u < cols) sum = sum + wv[u] * xv[u];
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) Y[(int64_t)token * outputStride + outputOffset + row] = sum;
}

// kernels/strata.cu:168-176 strata_bf16_project: bf16 weights, two per word
// (element ix in the half ix % 2 of word ix / 2), widened exactly to f32.
__global__ void k_bf16_project(const float *X, const uint32_t *Codes, float *Y, int cols, int rows, int tokens,
                               int outputStride, int outputOffset, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= rows || token >= tokens) return;
    const float *x = X + (int64_t)token * cols;
    const int64_t base = (int64_t)row * cols;
    float sum = 0.0f;
    // The reference's lane-strided order; PU positions' loads (clamped to
    // the row) go out before their products are added in order.
    for (int i0 = lane; i0 < cols; i0 += PU * 64) {
        uint32_t w[PU];
        float xv[PU];
#pragma unroll
        for (int u = 0; u < PU; u++) {
            const int i = min(i0 + 64 * u, cols - 1);
            w[u] = Codes[(base + i) / 2];
            xv[u] = x[i];
        }
#pragma unroll
        for (int u = 0; u < PU; u++) {
            const int64_t ix = base + i0 + 64 * u;
            if (i0 + 64 * u < cols) sum = sum + __uint_as_float(((w[u] >> ((ix % 2) * 16)) & 65535u) << 16) * xv[u];
        }
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) Y[(int64_t)token * outputStride + outputOffset + row] = sum;
}

// kernels/strata.cu:38-55 strata_q2_gate_up
__global__ void k_q2_gate_up(const float *X, const uint32_t *Blob, const float *Scales, const int *Mapping,
                             float *Hidden, int width, int ff, int tokens, int mapped, int expanded, int codeOffset,
                             int scaleOffset, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= ff || token >= tokens) return;
    int inputRow = mapped != 0 ? Mapping[2 * token] : token;
    float gsum = 0.0f, usum = 0.0f;
    for (int i = lane; i < width; i += 64) {
        int64_t gi = (int64_t)row * 2 * width + i, ui = gi + width;
        int gc = (int)q2_code(Blob, codeOffset, gi) - 1;
        int uc = (int)q2_code(Blob, codeOffset, ui) - 1;
        int64_t gs = scaleOffset + gi / 64, us = scaleOffset + ui / 64;
        float gw = (float)gc * (expanded != 0 ? Scales[gs] : blob_half(Blob, gs));
        float uw = (float)uc * (expanded != 0 ? Scales[us] : blob_half(Blob, us));
        float x = X[(int64_t)inputRow * width + i];
        gsum = gsum + gw * x;
        usum = usum + uw * x;
    }
    gsum = sm::tree_sum64(gsum);
    usum = sm::tree_sum64(usum);
    if (lane == 0) Hidden[(int64_t)token * ff + row] = sm::silu(gsum) * usum;
}

// kernels/strata.cu:56-69 strata_q2_down
__global__ void k_q2_down(const float *Hidden, const uint32_t *Blob, const float *Scales, const int *Mapping, float *Y,
                          int width, int ff, int tokens, int mapped, int expanded, int outputOffset, int codeOffset,
                          int scaleOffset, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= width || token >= tokens) return;
    float sum = 0.0f;
    for (int i = lane; i < ff; i += 64) {
        int64_t index = (int64_t)row * ff + i;
        int code = (int)q2_code(Blob, codeOffset, index) - 1;
        int64_t si = scaleOffset + index / 64;
        float w = (float)code * (expanded != 0 ? Scales[si] : blob_half(Blob, si));
        sum = sum + w * Hidden[(int64_t)token * ff + i];
    }
    sum = sm::tree_sum64(sum);
    int destination = mapped != 0 ? Mapping[2 * token + 1] : token;
    if (lane == 0) Y[(int64_t)outputOffset + (int64_t)destination * width + row] = sum;
}

// kernels/strata.cu:179-192 strata_q2_project
__global__ void k_q2_project(const float *X, const uint32_t *Blob, float *Y, int cols, int rows, int tokens,
                             int outputStride, int outputOffset, int codeOffset, int scaleOffset, int weightRow,
                             int rowStride, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= rows || token >= tokens) return;
    float sum = 0.0f;
    for (int i = lane; i < cols; i += 64) {
        int64_t ix = (int64_t)(weightRow + row * rowStride) * cols + i;
        int code = (int)q2_code(Blob, codeOffset, ix) - 1;
        float weight = (float)code * blob_half(Blob, scaleOffset + ix / 64);
        sum = sum + weight * X[(int64_t)token * cols + i];
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) Y[(int64_t)token * outputStride + outputOffset + row] = sum;
}

// kernels/strata.cu:22-31
__device__ __forceinline__ float iq4(int c) {
    const float t[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                         1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};
    return t[c & 15];
}

// kernels/strata.cu:193-211 strata_quant_project
__global__ void k_quant_project(const float *X, const uint32_t *Codes, const float *Scales, const float *Offsets,
                                float *Y, int cols, int rows, int tokens, int outputStride, int outputOffset, int bits,
                                int groupSize, int bias, int codebook, int hasOffset, uint32_t gx, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)(g % gx), token = (int)(g / gx), lane = lane_id();
    if (row >= rows || token >= tokens) return;
    const float *x = X + (int64_t)token * cols;
    float sum = 0.0f;
    // The reference's lane-strided order (index, bit and group in 31 bits,
    // as the launcher checks); PU positions' loads go out first.
    for (int i0 = lane; i0 < cols; i0 += PU * 64) {
        uint32_t w[PU];
        float sc[PU], of[PU], xv[PU];
#pragma unroll
        for (int u = 0; u < PU; u++) {
            const int index = row * cols + min(i0 + 64 * u, cols - 1), bit = index * bits;
            w[u] = Codes[bit / 32];
            sc[u] = Scales[index / groupSize];
            of[u] = hasOffset != 0 ? Offsets[index / groupSize] : 0.0f;
            xv[u] = x[min(i0 + 64 * u, cols - 1)];
        }
#pragma unroll
        for (int u = 0; u < PU; u++) {
            if (i0 + 64 * u >= cols) break;
            const int bit = (row * cols + i0 + 64 * u) * bits;
            const int code = (int)((w[u] >> (bit % 32)) & ((1u << bits) - 1u));
            const float value = codebook == 1 ? iq4(code) : (float)(code + bias);
            float weight = value * sc[u];
            if (hasOffset != 0) weight = weight + of[u];
            sum = sum + weight * xv[u];
        }
    }
    sum = sm::tree_sum64(sum);
    if (lane == 0) Y[(int64_t)token * outputStride + outputOffset + row] = sum;
}

// One-token projections with whole rows staged in LDS: the same per-lane
// sums as k_quant_project / k_bf16_project (lane l adds the products of
// elements l, l + 64, ... in order, then the reference's tree), with the
// loads reorganised. Each wave owns up to kRowsPerWave consecutive rows, one
// LDS buffer each; every row's codes go out at once by 16-byte DMA (its
// scales and offsets by 4-byte DMA), the wave waits once and sums the rows
// from LDS, and x stays in registers (element lane + 64 j in xv[j]). The
// generic kernels issue one narrow load per element and lane instead (64
// lanes of a quant_gemv load touch 8 distinct words), which leaves them
// issue-bound far below the memory's rate.
constexpr int kRowsPerWave = 4;
constexpr int kStagedMaxJ = 64;  // cols <= 4096: x in at most 64 registers (JB, a multiple of 8 >= cols / 64)
typedef __attribute__((address_space(3))) void lds_void_t;
__device__ __forceinline__ void dma_lds16(const void *src, uint32_t *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void dma_lds4(const void *src, uint32_t *lds_base) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)lds_base, 4, 0, 0);
}
// Every DMA of this wave has landed in LDS, and no LDS access moves across.
__device__ __forceinline__ void dma_wait_all() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
    asm volatile("" ::: "memory");
}

// The staged row sum of k_quant_gemv_staged: lane l's products in order,
// with the codebook and offset choices made once per row. Element
// i = lane + 64 j: its code word is lane / EPW + 64 j / EPW (an immediate
// offset from the lane's base), its group (64 j >> group_shift) +
// (lane >> group_shift) for every power-of-two group size, the offset of a
// group kStagedOffsets words after its scale.
constexpr int kStagedOffsets = 256;  // scales at [0, 256) of a row's group area, offsets at [256, 512)
template <int BITS, int JB, bool CODEBOOK, bool OFFSET>
__device__ __forceinline__ float staged_quant_row(const uint32_t *codes, const float *groups, int J, int group_shift,
                                                  int bias, const float (&xv)[JB], int lane) {
    constexpr int EPW = 32 / BITS;
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    const uint32_t *cl = codes + lane / EPW;
    const int shift = (lane % EPW) * BITS;
    const float *gl = groups + (lane >> group_shift);
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < JB; j++) {
        if (j < JB - 8 || j < J) {  // J > JB - 8
            const int code = (int)((cl[64 / EPW * j] >> shift) & MASK);
            const float *gj = gl + ((64 * j) >> group_shift);
            const float value = CODEBOOK ? iq4(code) : (float)(code + bias);
            float weight = value * gj[0];
            if (OFFSET) weight = weight + gj[kStagedOffsets];
            sum = sum + weight * xv[j];
        }
    }
    return sum;
}

// kernels/strata.cu:134-155 strata_quant_gemv (strata_quant_project's
// arithmetic, one token) for rows of cols % 64 == 0, cols <= 64 JB (JB - 8 <
// cols / 64), whole 16-byte code chunks per row, a power-of-two group size
// and at most 256 groups per row. Buffer words: codes (cw), scales (ng of
// kStagedOffsets), offsets (ng of kStagedOffsets).
template <int BITS, int JB>
__global__ void __launch_bounds__(256) k_quant_gemv_staged(const float *__restrict__ X,
                                                           const uint32_t *__restrict__ Codes,
                                                           const float *__restrict__ Scales,
                                                           const float *__restrict__ Offsets, float *__restrict__ Y,
                                                           int cols, int rows, int group_shift, int bias,
                                                           int codebook, int hasOffset, int rpw) {
    extern __shared__ uint32_t staged[];
    constexpr int EPW = 32 / BITS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int J = cols >> 6, cw = cols / EPW, ng = cols >> group_shift;
    const int bufw = cw + 2 * kStagedOffsets;
    uint32_t *bufs = staged + wave * rpw * bufw;
    const int r0 = (blockIdx.x * 4 + wave) * rpw;
    if (r0 >= rows) return;
    const int nr = min(rpw, rows - r0);
    // Every row of the wave in flight at once, then one wait.
    for (int k = 0; k < nr; k++) {
        const int r = r0 + k;
        uint32_t *buf = bufs + k * bufw;
        const uint8_t *crow = (const uint8_t *)Codes + (int64_t)r * cw * 4;
        for (int c = 0; c < cw / 4; c += 64)
            if (c + lane < cw / 4) dma_lds16(crow + (int64_t)(c + lane) * 16, buf + 4 * c);
        for (int c = 0; c < ng; c += 64)
            if (c + lane < ng) dma_lds4(Scales + (int64_t)r * ng + c + lane, buf + cw + c);
        if (hasOffset)
            for (int c = 0; c < ng; c += 64)
                if (c + lane < ng) dma_lds4(Offsets + (int64_t)r * ng + c + lane, buf + cw + kStagedOffsets + c);
    }
    float xv[JB];
#pragma unroll
    for (int j = 0; j < JB; j++) xv[j] = (j < JB - 8 || j < J) ? X[lane + 64 * j] : 0.0f;
    dma_wait_all();
    // The codebook and offset choices select one whole row loop (with the
    // stores inside, so the compiler cannot run the variants side by side).
    auto rows_loop = [&](auto codebook_tag, auto offset_tag) {
        for (int k = 0; k < nr; k++) {
            const uint32_t *buf = bufs + k * bufw;
            float sum = staged_quant_row<BITS, JB, decltype(codebook_tag)::value, decltype(offset_tag)::value>(
                buf, (const float *)(buf + cw), J, group_shift, bias, xv, lane);
            sum = sm::tree_sum64(sum);
            if (lane == 0) Y[r0 + k] = sum;
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    if (codebook == 1) {
        if (hasOffset) rows_loop(T{}, T{});
        else rows_loop(T{}, F{});
    } else {
        if (hasOffset) rows_loop(F{}, T{});
        else rows_loop(F{}, F{});
    }
}

// kernels/strata.cu:168-176 strata_bf16_project for one token and rows of
// cols % 64 == 0, cols <= 64 JB (JB - 8 < cols / 64). Each wave sums up to
// kRowsPerWave rows with two row buffers: the next row's DMA goes out before
// the current row is summed.
template <int JB>
__global__ void __launch_bounds__(256) k_bf16_gemv_staged(const float *__restrict__ X,
                                                          const uint32_t *__restrict__ Codes, float *__restrict__ Y,
                                                          int cols, int rows, int outputOffset) {
    extern __shared__ uint32_t staged[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int J = cols >> 6, cw = cols >> 1;
    uint32_t *buf0 = staged + wave * 2 * cw, *buf1 = buf0 + cw;
    const int r0 = (blockIdx.x * 4 + wave) * kRowsPerWave;
    if (r0 >= rows) return;
    auto issue = [&](int r, uint32_t *buf) {
        const uint8_t *crow = (const uint8_t *)Codes + (int64_t)r * cw * 4;
        for (int c = 0; c < cw / 4; c += 64)
            if (c + lane < cw / 4) dma_lds16(crow + (int64_t)(c + lane) * 16, buf + 4 * c);
    };
    issue(r0, buf0);
    float xv[JB];
#pragma unroll
    for (int j = 0; j < JB; j++) xv[j] = (j < JB - 8 || j < J) ? X[lane + 64 * j] : 0.0f;
    for (int k = 0; k < kRowsPerWave; k++) {
        const int r = r0 + k;
        if (r >= rows) break;
        dma_wait_all();
        if (k + 1 < kRowsPerWave && r + 1 < rows) issue(r + 1, (k & 1) ? buf0 : buf1);
        const uint32_t *buf = (k & 1) ? buf1 : buf0;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < JB; j++) {
            if (j < JB - 8 || j < J) {  // J > JB - 8
                const int i = lane + 64 * j;  // row * cols is even: element parity is i's
                sum = sum + __uint_as_float(((buf[i >> 1] >> ((i & 1) * 16)) & 65535u) << 16) * xv[j];
            }
        }
        sum = sm::tree_sum64(sum);
        if (lane == 0) Y[outputOffset + r] = sum;
    }
}

// kernels/strata.cu:214-227 strata_norm
__global__ void k_norm(const float *X, const float *W, float *Y, int cols, int rows, int weightRows, int mode,
                       float epsilon, float scale, uint64_t total) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int row = (int)g, lane = lane_id();
    if (row >= rows) return;
    // Lane-strided sum of squares in the reference order; the loads go out
    // eight at a time so their latencies overlap.
    const float *xr = X + (int64_t)row * cols;
    float ss = 0.0f;
    for (int i0 = lane; i0 < cols; i0 += 8 * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = xr[min(i0 + 64 * u, cols - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + 64 * u < cols) ss = ss + v[u] * v[u];
    }
    ss = __shfl(sm::tree_sum64(ss), 0, 64);
    float inv = scale / sqrtf((mode == 0 ? ss / (float)cols : ss) + epsilon);
    // Eight positions per lane are loaded before any is stored (Y may alias
    // X, and without the batching every store would wait for the next load).
    const float *wr = W + (int64_t)(row % weightRows) * cols;
    float *yr = Y + (int64_t)row * cols;
    for (int i0 = lane; i0 < cols; i0 += 8 * 64) {
        float x[8], w[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = min(i0 + 64 * u, cols - 1);
            x[u] = xr[i];
            w[u] = mode == 0 ? wr[i] : 1.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + 64 * u < cols) yr[i0 + 64 * u] = x[u] * inv * w[u];
    }
}

// The stack block's RMSNorm (k_norm mode 0, one gamma row, scale 1) for
// rows of NJ x 64 values held in registers: every load of a lane is issued
// before the sum (k_norm's batches of eight wait on each other), the same
// lane-strided order and tree, so the results are bit-identical.
template <int NJ>
__global__ void k_norm_reg(const float *X, const float *W, float *Y, int rows, float epsilon) {
    uint64_t g;
    if (!logical_group((uint64_t)rows, g)) return;
    const int row = (int)g, lane = lane_id();
    constexpr int cols = NJ * 64;
    const float *xr = X + (int64_t)row * cols;
    float x[NJ], w[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) x[j] = xr[lane + 64 * j];
#pragma unroll
    for (int j = 0; j < NJ; j++) w[j] = W[lane + 64 * j];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; j++) ss = ss + x[j] * x[j];
    ss = __shfl(sm::tree_sum64(ss), 0, 64);
    const float inv = 1.0f / sqrtf(ss / (float)cols + epsilon);
    float *yr = Y + (int64_t)row * cols;
#pragma unroll
    for (int j = 0; j < NJ; j++) yr[lane + 64 * j] = x[j] * inv * w[j];
}

// kernels/strata.cu:230-236 strata_elementwise
__global__ void k_elementwise(const float *A, const float *B, float *Y, int n, int mode, float scale) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float a = A[i] * scale, v = a;
    if (mode == 1) v = sm::silu(a);
    if (mode == 2) v = sm::sigmoid(a);
    if (mode == 3) v = sm::silu(a) * B[i];
    if (mode == 4) v = a * sm::sigmoid(B[i]);
    if (mode == 5) v = a + B[i];
    Y[i] = v;
}

__global__ void k_router_batch(const float *Logits, int *Ids, float *Weights, int experts, int topK, uint64_t total,
                               int batch) {
    uint64_t g;
    if (!logical_group(total, g)) return;
    int token = batch ? (int)g : 0;
    sm::router_wave(Logits + (int64_t)token * experts, Ids + (int64_t)token * topK, Weights + (int64_t)token * topK,
                experts, topK);
}

// kernels/strata.cu:360-365 and :470-476; tokens = 1 is strata_moe_combine.
__global__ void k_moe_combine(const float *Parts, const float *Weights, const float *Shared, const float *SharedGate,
                              float *Y, int width, int count, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t token = i / width, d = i % width;
    float value = Shared[i] * sm::sigmoid(SharedGate[token]);
    for (int k = 0; k < count; ++k) value = value + Parts[(token * count + k) * width + d] * Weights[token * count + k];
    Y[i] = value;
}

// kernels/strata.cu:464-469
__global__ void k_gather_rows(const float *X, const int *Indices, float *Y, int width, int rows) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (int64_t)width * rows) Y[i] = X[(int64_t)Indices[i / width] * width + i % width];
}
__global__ void k_scatter_rows(const float *X, const int *Indices, float *Y, int width, int rows) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < (int64_t)width * rows) Y[(int64_t)Indices[i / width] * width + i % width] = X[i];
}

// Checks that every index in an i32 device buffer lies in [lo, hi): the
// host cannot see device-resident indices, so the launcher validates them on
// the device before the gather/scatter or mapped kernel runs.
__global__ void k_check_indices(const int *idx, int64_t n, int64_t stride, int64_t first, int lo, int hi,
                                uint32_t *bad) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int v = idx[first + i * stride];
    if (v < lo || v >= hi) atomicOr(bad, 1u);
}

}  // namespace

namespace smi {

int64_t buf_len(sm_ctx *ctx, uint64_t h) {
    auto it = ctx->buffers.find(h);
    return it == ctx->buffers.end() ? -1 : (int64_t)it->second;
}

// Device-side index validation for Mapping / Indices / Cells buffers.
int check_indices(sm_ctx *ctx, uint64_t buf, int64_t n, int64_t stride, int64_t first, int lo, int hi,
                  const char *what) {
    if (n <= 0) return SM_OK;
    if (ctx->capturing) return fail(ctx, SM_E_ARG, std::string(what) + ": index validation is not allowed while capturing");
    uint32_t *bad_flag = ctx->counters + 255;
    hipError_t e = hipMemsetAsync(bad_flag, 0, 4, ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMemsetAsync");
    k_check_indices<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>((const int *)buf, n, stride, first, lo, hi,
                                                                          bad_flag);
    if (int rc = launched(ctx)) return rc;
    uint32_t flag = 0;
    e = hipMemcpyAsync(&flag, bad_flag, 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(ctx, e, "index check");
    if (flag) return fail(ctx, SM_E_BOUNDS, std::string(what) + ": an index points outside the buffer layout");
    return SM_OK;
}

}  // namespace smi

namespace {

// ---------------------------------------------------------- host side
int bad(sm_ctx *ctx, const std::string &m) { return fail(ctx, SM_E_ARG, m); }

unsigned blocks_for(uint64_t logical) { return (unsigned)((logical + kGroupsPerBlock - 1) / kGroupsPerBlock); }

int L_unpack_half(sm_ctx *ctx, const uint32_t *G, Args a) {
    int count = a.i32(2);
    if (count < 0) return bad(ctx, "count must be >= 0");
    int n = count < (int)(G[0] * 64) ? count : (int)(G[0] * 64);
    if (int rc = need(ctx, a.ptr(0), ((uint64_t)n + 1) / 2 * 4, "strata_unpack_half.Packed")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "strata_unpack_half.Values")) return rc;
    if (n == 0) return SM_OK;
    k_unpack_half<<<(n + 255) / 256, 256, 0, ctx->stream>>>((const uint32_t *)a.ptr(0), (float *)a.ptr(1), n);
    return launched(ctx);
}

int L_expert_scales(sm_ctx *ctx, const uint32_t *G, Args a) {
    int offset = a.i32(2), count = a.i32(3);
    if (offset < 0 || count < 0) return bad(ctx, "offset and count must be >= 0");
    int n = count < (int)(G[0] * 64) ? count : (int)(G[0] * 64);
    if (int rc = need(ctx, a.ptr(0), ((uint64_t)offset + n + 1) / 2 * 4, "strata_expert_scales.Blob")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)n * 4, "strata_expert_scales.Scales")) return rc;
    if (n == 0) return SM_OK;
    k_expert_scales<<<(n + 255) / 256, 256, 0, ctx->stream>>>((const uint32_t *)a.ptr(0), (float *)a.ptr(1), offset,
                                                              n);
    return launched(ctx);
}

// Shared layout checks of the projection family (src/backend.js:19-22).
int projection_layout(sm_ctx *ctx, const char *name, uint64_t X, uint64_t Y, int cols, int rows, int tokens,
                      int outputStride, int outputOffset, int *rr, int *tt, const uint32_t *G) {
    if (cols < 1 || rows < 1 || tokens < 1 || outputStride < 1 || outputOffset < 0)
        return bad(ctx, std::string(name) + ": cols, rows, tokens, outputStride must be >= 1 and outputOffset >= 0");
    if (outputOffset + rows > outputStride) return bad(ctx, "Projection batch exceeds buffer layout");
    *rr = rows < (int)G[0] ? rows : (int)G[0];
    *tt = tokens < (int)G[1] ? tokens : (int)G[1];
    if (int rc = need(ctx, X, (uint64_t)(*tt) * cols * 4, "projection X")) return rc;
    if (int rc = need(ctx, Y, ((uint64_t)(*tt - 1) * outputStride + outputOffset + *rr) * 4, "projection Y")) return rc;
    return SM_OK;
}

int L_project(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(3), rows = a.i32(4), tokens = a.i32(5), stride = a.i32(6), off = a.i32(7), rr, tt;
    if (int rc = projection_layout(ctx, "strata_project", a.ptr(0), a.ptr(2), cols, rows, tokens, stride, off, &rr, &tt,
                                   G))
        return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)rr * cols * 4, "strata_project.W")) return rc;
    uint64_t total = (uint64_t)G[0] * G[1];
    k_project<<<blocks_for(total), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const float *)a.ptr(1),
                                                          (float *)a.ptr(2), cols, rows, tokens, stride, off, G[0],
                                                          total);
    return launched(ctx);
}

int L_gemv(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(3), rows = a.i32(4), tokens = a.i32(5), rr, tt;
    if (int rc = projection_layout(ctx, "strata_gemv", a.ptr(0), a.ptr(2), cols, rows, tokens, rows, 0, &rr, &tt, G))
        return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)rr * cols * 4, "strata_gemv.W")) return rc;
    uint64_t total = (uint64_t)G[0] * G[1];
    k_project<<<blocks_for(total), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const float *)a.ptr(1),
                                                          (float *)a.ptr(2), cols, rows, tokens, rows, 0, G[0], total);
    return launched(ctx);
}

// Q2 expert family: src/backend.js:28-32.
int L_q2_expert(sm_ctx *ctx, const uint32_t *G, Args a, bool down) {
    const char *name = down ? "strata_q2_down" : "strata_q2_gate_up";
    int width = a.i32(5), ff = a.i32(6), tokens = a.i32(7), mapped = a.i32(8), expanded = a.i32(9);
    int outputOffset = down ? a.i32(10) : 0, codeOffset = a.i32(down ? 11 : 10), scaleOffset = a.i32(down ? 12 : 11);
    if (width < 1 || ff < 1 || tokens < 1) return bad(ctx, std::string(name) + ": width, ff, tokens must be >= 1");
    if (width % 64 || ff % 64) return bad(ctx, "Packed expert dimensions must contain complete groups");
    if (codeOffset < 0 || scaleOffset < 0 || outputOffset < 0) return bad(ctx, "offsets must be >= 0");
    int rows = down ? width : ff;
    int rr = rows < (int)G[0] ? rows : (int)G[0], tt = tokens < (int)G[1] ? tokens : (int)G[1];
    uint64_t Hidden = down ? a.ptr(0) : a.ptr(4);
    if (buf_len(ctx, Hidden) >= 0 && buf_len(ctx, Hidden) < (int64_t)tokens * ff * 4)
        return bad(ctx, "Packed expert batch exceeds buffer layout");
    if (mapped && buf_len(ctx, a.ptr(3)) >= 0 && buf_len(ctx, a.ptr(3)) < (int64_t)tokens * 2 * 4)
        return bad(ctx, "Packed expert batch exceeds buffer layout");
    // Code words and scales touched by rows [0, rr).
    uint64_t elems = down ? (uint64_t)rr * ff : (uint64_t)rr * 2 * width;
    if (int rc = need(ctx, a.ptr(1), ((uint64_t)codeOffset + (elems + 15) / 16) * 4, "Blob codes")) return rc;
    uint64_t scaleEnd = (uint64_t)scaleOffset + (elems + 63) / 64;
    if (expanded) {
        if (int rc = need(ctx, a.ptr(2), scaleEnd * 4, "Scales")) return rc;
    } else if (int rc = need(ctx, a.ptr(1), (scaleEnd + 1) / 2 * 4, "Blob scales")) {
        return rc;
    }
    if (mapped) {
        if (int rc = need(ctx, a.ptr(3), (uint64_t)tt * 2 * 4, "Mapping")) return rc;
    }
    if (!down) {
        if (int rc = need(ctx, a.ptr(4), (uint64_t)tt * ff * 4, "Hidden")) return rc;
        int inputRows = tt;
        if (mapped) {
            int64_t xrows = buf_len(ctx, a.ptr(0)) / 4 / width;
            if (int rc = check_indices(ctx, a.ptr(3), tt, 2, 0, 0, (int)xrows, "Mapping input rows")) return rc;
        } else if (int rc = need(ctx, a.ptr(0), (uint64_t)inputRows * width * 4, "X")) {
            return rc;
        }
        uint64_t total = (uint64_t)G[0] * G[1];
        k_q2_gate_up<<<blocks_for(total), 256, 0, ctx->stream>>>(
            (const float *)a.ptr(0), (const uint32_t *)a.ptr(1), (const float *)a.ptr(2), (const int *)a.ptr(3),
            (float *)a.ptr(4), width, ff, tokens, mapped, expanded, codeOffset, scaleOffset, G[0], total);
        return launched(ctx);
    }
    if (int rc = need(ctx, a.ptr(0), (uint64_t)tt * ff * 4, "Hidden")) return rc;
    int64_t ylen = buf_len(ctx, a.ptr(4));
    if (ylen < 0) return need(ctx, a.ptr(4), 0, "Y");
    if (mapped) {
        // Y[outputOffset + dest*width + row] for row < rr must stay in bounds.
        int64_t maxDest = (ylen / 4 - outputOffset - rr) / width + 1;
        if (ylen / 4 < outputOffset + rr) return need(ctx, a.ptr(4), ((uint64_t)outputOffset + rr) * 4, "Y");
        if (int rc = check_indices(ctx, a.ptr(3), tt, 2, 1, 0, (int)maxDest, "Mapping destinations")) return rc;
    } else if (int rc = need(ctx, a.ptr(4), ((uint64_t)outputOffset + (uint64_t)(tt - 1) * width + rr) * 4, "Y")) {
        return rc;
    }
    uint64_t total = (uint64_t)G[0] * G[1];
    k_q2_down<<<blocks_for(total), 256, 0, ctx->stream>>>(
        (const float *)a.ptr(0), (const uint32_t *)a.ptr(1), (const float *)a.ptr(2), (const int *)a.ptr(3),
        (float *)a.ptr(4), width, ff, tokens, mapped, expanded, outputOffset, codeOffset, scaleOffset, G[0], total);
    return launched(ctx);
}
int L_q2_gate_up(sm_ctx *ctx, const uint32_t *G, Args a) { return L_q2_expert(ctx, G, a, false); }
int L_q2_down(sm_ctx *ctx, const uint32_t *G, Args a) { return L_q2_expert(ctx, G, a, true); }

int L_q2_project(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(3), rows = a.i32(4), tokens = a.i32(5), stride = a.i32(6), off = a.i32(7);
    int codeOffset = a.i32(8), scaleOffset = a.i32(9), weightRow = a.i32(10), rowStride = a.i32(11), rr, tt;
    if (int rc = projection_layout(ctx, "strata_q2_project", a.ptr(0), a.ptr(2), cols, rows, tokens, stride, off, &rr,
                                   &tt, G))
        return rc;
    if (cols % 64) return bad(ctx, "Q2 expert columns must contain complete groups");
    if (codeOffset < 0 || scaleOffset < 0 || weightRow < 0) return bad(ctx, "codeOffset/scaleOffset/weightRow >= 0");
    if (rowStride < 1 || rowStride > 2) return bad(ctx, "expert row stride must be an integer in [1, 2]");
    uint64_t lastRow = (uint64_t)weightRow + (uint64_t)(rr - 1) * rowStride;
    uint64_t elems = (lastRow + 1) * cols;
    if (int rc = need(ctx, a.ptr(1), ((uint64_t)codeOffset + elems / 16) * 4, "Blob codes")) return rc;
    if (int rc = need(ctx, a.ptr(1), (((uint64_t)scaleOffset + elems / 64) + 1) / 2 * 4, "Blob scales")) return rc;
    uint64_t total = (uint64_t)G[0] * G[1];
    k_q2_project<<<blocks_for(total), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const uint32_t *)a.ptr(1),
                                                             (float *)a.ptr(2), cols, rows, tokens, stride, off,
                                                             codeOffset, scaleOffset, weightRow, rowStride, G[0],
                                                             total);
    return launched(ctx);
}

int L_quant_project(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(5), rows = a.i32(6), tokens = a.i32(7), stride = a.i32(8), off = a.i32(9);
    int bits = a.i32(10), groupSize = a.i32(11), bias = a.i32(12), codebook = a.i32(13), hasOffset = a.i32(14), rr, tt;
    if (bits != 2 && bits != 4 && bits != 8) return bad(ctx, "Canonical code width must be 2, 4 or 8");
    if (groupSize < 1 || cols % groupSize || (int64_t)cols * rows * bits > 0x7fffffff)
        return bad(ctx, "Quantized rows must contain whole groups and fit 31-bit indexing");
    if (int rc = projection_layout(ctx, "strata_quant_project", a.ptr(0), a.ptr(4), cols, rows, tokens, stride, off,
                                   &rr, &tt, G))
        return rc;
    uint64_t elems = (uint64_t)rr * cols;
    if (int rc = need(ctx, a.ptr(1), (elems * bits + 31) / 32 * 4, "Codes")) return rc;
    if (int rc = need(ctx, a.ptr(2), (elems / groupSize) * 4, "Scales")) return rc;
    if (hasOffset)
        if (int rc = need(ctx, a.ptr(3), (elems / groupSize) * 4, "Offsets")) return rc;
    uint64_t total = (uint64_t)G[0] * G[1];
    k_quant_project<<<blocks_for(total), 256, 0, ctx->stream>>>(
        (const float *)a.ptr(0), (const uint32_t *)a.ptr(1), (const float *)a.ptr(2), (const float *)a.ptr(3),
        (float *)a.ptr(4), cols, rows, tokens, stride, off, bits, groupSize, bias, codebook, hasOffset, G[0], total);
    return launched(ctx);
}

int L_bf16_project(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(3), rows = a.i32(4), tokens = a.i32(5), stride = a.i32(6), off = a.i32(7), rr, tt;
    if (int rc = projection_layout(ctx, "strata_bf16_project", a.ptr(0), a.ptr(2), cols, rows, tokens, stride, off,
                                   &rr, &tt, G))
        return rc;
    if (int rc = need(ctx, a.ptr(1), ((uint64_t)rr * cols + 1) / 2 * 4, "strata_bf16_project.Codes")) return rc;
    if (tt == 1 && cols % 64 == 0 && cols <= 64 * kStagedMaxJ && a.ptr(1) % 16 == 0) {
        // one token: whole rows staged in LDS (same sums, same order)
        const unsigned blocks = (unsigned)((rr + 4 * kRowsPerWave - 1) / (4 * kRowsPerWave));
        using KB = decltype(&k_bf16_gemv_staged<8>);
        const KB kb[8] = {k_bf16_gemv_staged<8>,  k_bf16_gemv_staged<16>, k_bf16_gemv_staged<24>,
                          k_bf16_gemv_staged<32>, k_bf16_gemv_staged<40>, k_bf16_gemv_staged<48>,
                          k_bf16_gemv_staged<56>, k_bf16_gemv_staged<64>};
        kb[(cols / 64 - 1) / 8]<<<blocks, 256, (size_t)4 * 2 * (cols / 2) * 4, ctx->stream>>>(
            (const float *)a.ptr(0), (const uint32_t *)a.ptr(1), (float *)a.ptr(2), cols, rr, off);
        return launched(ctx);
    }
    uint64_t total = (uint64_t)G[0] * G[1];
    k_bf16_project<<<blocks_for(total), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const uint32_t *)a.ptr(1),
                                                               (float *)a.ptr(2), cols, rows, tokens, stride, off,
                                                               G[0], total);
    return launched(ctx);
}

// kernels/strata.cu:134-155 strata_quant_gemv: strata_quant_project's
// arithmetic for one token, grid [rows, 1, 1].
int L_quant_gemv(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(5), rows = a.i32(6), bits = a.i32(7), groupSize = a.i32(8), bias = a.i32(9);
    int codebook = a.i32(10), hasOffset = a.i32(11), rr, tt;
    if (bits != 2 && bits != 4 && bits != 8) return bad(ctx, "Canonical code width must be 2, 4 or 8");
    if (groupSize < 1 || cols % groupSize || (int64_t)cols * rows * bits > 0x7fffffff)
        return bad(ctx, "Quantized rows must contain whole groups and fit 31-bit indexing");
    const uint32_t G1[3] = {G[0], 1, 1};
    if (int rc = projection_layout(ctx, "strata_quant_gemv", a.ptr(0), a.ptr(4), cols, rows, 1, rows, 0, &rr, &tt, G1))
        return rc;
    uint64_t elems = (uint64_t)rr * cols;
    if (int rc = need(ctx, a.ptr(1), (elems * bits + 31) / 32 * 4, "Codes")) return rc;
    if (int rc = need(ctx, a.ptr(2), (elems / groupSize) * 4, "Scales")) return rc;
    if (hasOffset)
        if (int rc = need(ctx, a.ptr(3), (elems / groupSize) * 4, "Offsets")) return rc;
    const int cw = cols * bits / 32, ng = cols / groupSize;
    if (cols % 64 == 0 && cols <= 64 * kStagedMaxJ && cw % 4 == 0 && (groupSize & (groupSize - 1)) == 0 &&
        ng <= 256 && a.ptr(1) % 16 == 0) {
        // whole rows staged in LDS (same sums, same order)
        int shift = 0;
        while ((1 << shift) < groupSize) shift++;
        const int bufw = cw + 2 * kStagedOffsets;
        // rows per wave: up to kRowsPerWave, the block's buffers within 64 KiB
        const int rpw = std::max(1, std::min(kRowsPerWave, 65536 / (4 * bufw * 4)));
        const unsigned blocks = (unsigned)((rr + 4 * rpw - 1) / (4 * rpw));
        const size_t lds = (size_t)4 * rpw * bufw * 4;
        using KQ = decltype(&k_quant_gemv_staged<4, 8>);
#define SM_QG_ROW(B)                                                                                               \
    {k_quant_gemv_staged<B, 8>,  k_quant_gemv_staged<B, 16>, k_quant_gemv_staged<B, 24>, k_quant_gemv_staged<B, 32>, \
     k_quant_gemv_staged<B, 40>, k_quant_gemv_staged<B, 48>, k_quant_gemv_staged<B, 56>, k_quant_gemv_staged<B, 64>}
        const KQ kq[3][8] = {SM_QG_ROW(2), SM_QG_ROW(4), SM_QG_ROW(8)};
#undef SM_QG_ROW
        const KQ k = kq[bits == 2 ? 0 : bits == 4 ? 1 : 2][(cols / 64 - 1) / 8];
        k<<<blocks, 256, lds, ctx->stream>>>((const float *)a.ptr(0), (const uint32_t *)a.ptr(1),
                                             (const float *)a.ptr(2), (const float *)a.ptr(3), (float *)a.ptr(4),
                                             cols, rr, shift, bias, codebook, hasOffset, rpw);
        return launched(ctx);
    }
    k_quant_project<<<blocks_for(G[0]), 256, 0, ctx->stream>>>(
        (const float *)a.ptr(0), (const uint32_t *)a.ptr(1), (const float *)a.ptr(2), (const float *)a.ptr(3),
        (float *)a.ptr(4), cols, rows, 1, rows, 0, bits, groupSize, bias, codebook, hasOffset, G[0], G[0]);
    return launched(ctx);
}

int L_norm(sm_ctx *ctx, const uint32_t *G, Args a) {
    int cols = a.i32(3), rows = a.i32(4), weightRows = a.i32(5), mode = a.i32(6);
    float eps = a.f32(7), scale = a.f32(8);
    if (cols < 1 || rows < 1 || weightRows < 1) return bad(ctx, "cols, rows, weightRows must be >= 1");
    if (rows % weightRows) return fail(ctx, SM_E_ARG, "Normalization weight rows must divide input rows");
    int rr = rows < (int)G[0] ? rows : (int)G[0];
    if (int rc = need(ctx, a.ptr(0), (uint64_t)rr * cols * 4, "strata_norm.X")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)rr * cols * 4, "strata_norm.Y")) return rc;
    if (mode == 0) {
        int wr = weightRows < rr ? weightRows : rr;
        if (int rc = need(ctx, a.ptr(1), (uint64_t)wr * cols * 4, "strata_norm.W")) return rc;
    }
    k_norm<<<blocks_for(rr), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const float *)a.ptr(1),
                                                    (float *)a.ptr(2), cols, rows, weightRows, mode, eps, scale, rr);
    return launched(ctx);
}

int L_elementwise(sm_ctx *ctx, const uint32_t *G, Args a) {
    int n = a.i32(3), mode = a.i32(4);
    float scale = a.f32(5);
    if (n < 0) return bad(ctx, "n must be >= 0");
    int m = n < (int)(G[0] * 64) ? n : (int)(G[0] * 64);
    if (int rc = need(ctx, a.ptr(0), (uint64_t)m * 4, "strata_elementwise.A")) return rc;
    if (mode >= 3 && mode <= 5)
        if (int rc = need(ctx, a.ptr(1), (uint64_t)m * 4, "strata_elementwise.B")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)m * 4, "strata_elementwise.Y")) return rc;
    if (m == 0) return SM_OK;
    k_elementwise<<<(m + 255) / 256, 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const float *)a.ptr(1),
                                                            (float *)a.ptr(2), m, mode, scale);
    return launched(ctx);
}

int router_common(sm_ctx *ctx, const uint32_t *G, Args a, bool batch) {
    int experts = a.i32(3), topK = a.i32(4);
    if (experts < 1 || topK < 1) return bad(ctx, "experts and topK must be >= 1");
    if (experts > 512 || topK > (experts < 32 ? experts : 32))
        return fail(ctx, SM_E_ARG, "Router supports 1-512 experts and topK <= min(experts,32)");
    uint64_t tokens = batch ? G[0] : 1;
    if (int rc = need(ctx, a.ptr(0), tokens * experts * 4, "router Logits")) return rc;
    if (int rc = need(ctx, a.ptr(1), tokens * topK * 4, "router Ids")) return rc;
    if (int rc = need(ctx, a.ptr(2), tokens * topK * 4, "router Weights")) return rc;
    k_router_batch<<<blocks_for(tokens), 256, 0, ctx->stream>>>((const float *)a.ptr(0), (int *)a.ptr(1),
                                                                (float *)a.ptr(2), experts, topK, tokens, batch);
    return launched(ctx);
}
int L_router(sm_ctx *ctx, const uint32_t *G, Args a) { return router_common(ctx, G, a, false); }
int L_router_batch(sm_ctx *ctx, const uint32_t *G, Args a) { return router_common(ctx, G, a, true); }

int combine_common(sm_ctx *ctx, const uint32_t *G, Args a, bool batch) {
    int width = a.i32(5), count = a.i32(6), tokens = batch ? a.i32(7) : 1;
    if (width < 1 || count < 0 || tokens < 1) return bad(ctx, "width, tokens must be >= 1 and count >= 0");
    int64_t n = (int64_t)width * tokens, lim = (int64_t)G[0] * 64;
    if (n > lim) n = lim;
    int64_t tt = (n + width - 1) / width;  // tokens touched
    if (n == 0) return SM_OK;
    if (int rc = need(ctx, a.ptr(0), (uint64_t)(tt * count * width) * 4, "Parts")) return rc;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)(tt * count) * 4, "Weights")) return rc;
    if (int rc = need(ctx, a.ptr(2), (uint64_t)n * 4, "Shared")) return rc;
    if (int rc = need(ctx, a.ptr(3), (uint64_t)tt * 4, "SharedGate")) return rc;
    if (int rc = need(ctx, a.ptr(4), (uint64_t)n * 4, "Y")) return rc;
    k_moe_combine<<<(unsigned)((n + 255) / 256), 256, 0, ctx->stream>>>(
        (const float *)a.ptr(0), (const float *)a.ptr(1), (const float *)a.ptr(2), (const float *)a.ptr(3),
        (float *)a.ptr(4), width, count, n);
    return launched(ctx);
}
int L_moe_combine(sm_ctx *ctx, const uint32_t *G, Args a) { return combine_common(ctx, G, a, false); }
int L_moe_combine_batch(sm_ctx *ctx, const uint32_t *G, Args a) { return combine_common(ctx, G, a, true); }

int rows_common(sm_ctx *ctx, const uint32_t *G, Args a, bool scatter) {
    int width = a.i32(3), rows = a.i32(4);
    if (width < 1 || rows < 0) return bad(ctx, "width >= 1 and rows >= 0");
    int64_t n = (int64_t)width * rows, lim = (int64_t)G[0] * 64;
    if (n > lim) n = lim;
    if (n == 0) return SM_OK;
    int64_t rr = (n + width - 1) / width;
    if (int rc = need(ctx, a.ptr(1), (uint64_t)rr * 4, "Indices")) return rc;
    uint64_t dense = scatter ? a.ptr(0) : a.ptr(2), sparse = scatter ? a.ptr(2) : a.ptr(0);
    if (int rc = need(ctx, dense, (uint64_t)n * 4, scatter ? "X" : "Y")) return rc;
    int64_t sparseRows = buf_len(ctx, sparse) / 4 / width;
    if (buf_len(ctx, sparse) < 0) return need(ctx, sparse, 0, "rows buffer");
    if (int rc = check_indices(ctx, a.ptr(1), rr, 1, 0, 0, (int)sparseRows, "Indices")) return rc;
    unsigned blocks = (unsigned)((n + 255) / 256);
    if (scatter)
        k_scatter_rows<<<blocks, 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const int *)a.ptr(1),
                                                        (float *)a.ptr(2), width, (int)rr);
    else
        k_gather_rows<<<blocks, 256, 0, ctx->stream>>>((const float *)a.ptr(0), (const int *)a.ptr(1),
                                                       (float *)a.ptr(2), width, (int)rr);
    return launched(ctx);
}
int L_gather_rows(sm_ctx *ctx, const uint32_t *G, Args a) { return rows_common(ctx, G, a, false); }
int L_scatter_rows(sm_ctx *ctx, const uint32_t *G, Args a) { return rows_common(ctx, G, a, true); }

// Parameter lists in the reference's order (kernels/strata.cu).
const Entry kEntries[] = {
    {"strata_unpack_half", "Packed:u32*,Values:f32*,count:i32", 3, L_unpack_half},
    {"strata_expert_scales", "Blob:u32*,Scales:f32*,offset:i32,count:i32", 4, L_expert_scales},
    {"strata_q2_gate_up",
     "X:f32*,Blob:u32*,Scales:f32*,Mapping:i32*,Hidden:f32*,width:i32,ff:i32,tokens:i32,mapped:i32,expanded:i32,"
     "codeOffset:i32,scaleOffset:i32",
     12, L_q2_gate_up},
    {"strata_q2_down",
     "Hidden:f32*,Blob:u32*,Scales:f32*,Mapping:i32*,Y:f32*,width:i32,ff:i32,tokens:i32,mapped:i32,expanded:i32,"
     "outputOffset:i32,codeOffset:i32,scaleOffset:i32",
     13, L_q2_down},
    {"strata_gemv", "X:f32*,W:f32*,Y:f32*,cols:i32,rows:i32,tokens:i32", 6, L_gemv},
    {"strata_project", "X:f32*,W:f32*,Y:f32*,cols:i32,rows:i32,tokens:i32,outputStride:i32,outputOffset:i32", 8,
     L_project},
    {"strata_q2_project",
     "X:f32*,Blob:u32*,Y:f32*,cols:i32,rows:i32,tokens:i32,outputStride:i32,outputOffset:i32,codeOffset:i32,"
     "scaleOffset:i32,weightRow:i32,rowStride:i32",
     12, L_q2_project},
    {"strata_quant_project",
     "X:f32*,Codes:u32*,Scales:f32*,Offsets:f32*,Y:f32*,cols:i32,rows:i32,tokens:i32,outputStride:i32,"
     "outputOffset:i32,bits:i32,groupSize:i32,bias:i32,codebook:i32,hasOffset:i32",
     15, L_quant_project},
    {"strata_bf16_project",
     "X:f32*,Codes:u32*,Y:f32*,cols:i32,rows:i32,tokens:i32,outputStride:i32,outputOffset:i32", 8, L_bf16_project},
    {"strata_quant_gemv",
     "X:f32*,Codes:u32*,Scales:f32*,Offsets:f32*,Y:f32*,cols:i32,rows:i32,bits:i32,groupSize:i32,bias:i32,"
     "codebook:i32,hasOffset:i32",
     12, L_quant_gemv},
    {"strata_norm", "X:f32*,W:f32*,Y:f32*,cols:i32,rows:i32,weightRows:i32,mode:i32,epsilon:f32,scale:f32", 9, L_norm},
    {"strata_elementwise", "A:f32*,B:f32*,Y:f32*,n:i32,mode:i32,scale:f32", 6, L_elementwise},
    {"strata_router", "Logits:f32*,Ids:i32*,Weights:f32*,experts:i32,topK:i32", 5, L_router},
    {"strata_router_batch", "Logits:f32*,Ids:i32*,Weights:f32*,experts:i32,topK:i32", 5, L_router_batch},
    {"strata_moe_combine", "Parts:f32*,Weights:f32*,Shared:f32*,SharedGate:f32*,Y:f32*,width:i32,count:i32", 7,
     L_moe_combine},
    {"strata_moe_combine_batch",
     "Parts:f32*,Weights:f32*,Shared:f32*,SharedGate:f32*,Y:f32*,width:i32,count:i32,tokens:i32", 8,
     L_moe_combine_batch},
    {"strata_gather_rows", "X:f32*,Indices:i32*,Y:f32*,width:i32,rows:i32", 5, L_gather_rows},
    {"strata_scatter_rows", "X:f32*,Indices:i32*,Y:f32*,width:i32,rows:i32", 5, L_scatter_rows},
};
const int kEntryCount = sizeof(kEntries) / sizeof(kEntries[0]);

// The MoE path's kernels (this file) first, then the fixture model's.
const Entry *entry_at(int index) {
    int model_count = 0;
    const Entry *model = model_entries(&model_count);
    if (index >= 0 && index < kEntryCount) return &kEntries[index];
    if (index >= kEntryCount && index < kEntryCount + model_count) return &model[index - kEntryCount];
    return nullptr;
}
int entry_count() {
    int model_count = 0;
    model_entries(&model_count);
    return kEntryCount + model_count;
}
const Entry *find_entry(const char *name) {
    if (!name) return nullptr;
    for (int i = 0, n = entry_count(); i < n; i++)
        if (!strcmp(entry_at(i)->name, name)) return entry_at(i);
    return nullptr;
}

}  // namespace

namespace smi {

int norm_launch(sm_ctx *ctx, const float *X, const float *gamma, float *Y, int cols, int rows, float eps) {
    if (cols == 2048)
        k_norm_reg<32><<<blocks_for((uint64_t)rows), 256, 0, ctx->stream>>>(X, gamma, Y, rows, eps);
    else if (cols == 2560)
        k_norm_reg<40><<<blocks_for((uint64_t)rows), 256, 0, ctx->stream>>>(X, gamma, Y, rows, eps);
    else
        k_norm<<<blocks_for((uint64_t)rows), 256, 0, ctx->stream>>>(X, gamma, Y, cols, rows, 1, 0, eps, 1.0f,
                                                                  (uint64_t)rows);
    return launched(ctx);
}

}  // namespace smi

extern "C" {

int sm_kernel_count(void) { return entry_count(); }
const char *sm_kernel_name(int index) {
    const Entry *e = entry_at(index);
    return e ? e->name : nullptr;
}
const char *sm_kernel_signature(const char *name) {
    const Entry *e = find_entry(name);
    return e ? e->signature : nullptr;
}

int sm_run(sm_ctx *ctx, const char *name, const uint32_t groups[3], const uint64_t *args, int nargs) {
    if (!ctx) return SM_E_ARG;
    const Entry *e = find_entry(name);
    if (!e) return fail(ctx, SM_E_NOKERNEL, std::string("Unknown kernel ") + (name ? name : "(null)"));
    if (!groups || !args) return fail(ctx, SM_E_ARG, "groups and args are required");
    if (nargs != e->nargs)
        return fail(ctx, SM_E_ARG, std::string(name) + ": expected " + std::to_string(e->nargs) + " arguments");
    // vendor/webcuda/src/wasm/runtime.js:11
    uint64_t prod = 1;
    for (int i = 0; i < 3; i++) {
        if (groups[i] < 1) return fail(ctx, SM_E_ARG, "Invalid dispatch size");
        prod *= groups[i];
    }
    if (prod > 100000000ull) return fail(ctx, SM_E_ARG, "Invalid dispatch size");
    return e->launch(ctx, groups, Args{args});
}

}  // extern "C"
