// Decode-step LM head: logits = x . W^T over a dense bf16 weight
// W [vocab, hidden] (Qwen2's tied embedding) for up to 16 rows of bf16
// hidden states, with the greedy argmax of every row.
//
// The weight (vocab * hidden * 2 bytes, 467 MB for Qwen2-1.5B) is streamed
// once, so the kernel is HBM-bound; the MFMA only saves VALU work.
//
// Layout of the work.  A workgroup owns kTiles tiles of 16 vocab rows; its
// four waves split the hidden dimension in blocks of 128 (wave w takes
// blocks w, w + 4, ...).  In v_mfma_f32_16x16x32_bf16, lane l = 16 q + j
// supplies A row j (vocab row) and B column j (batch row) at K slots
// [8 q, 8 q + 8); step i of block b uses elements 128 b + 32 i + [0, 32), so
// lane (q, j) loads the 16 bytes at element 128 b + 32 i + 8 q of its vocab
// row and of its batch row.  Each load instruction then reads 64 contiguous
// bytes of each of 16 weight rows: interleaving the lanes this way (rather
// than giving each lane 64 contiguous bytes) measured about twice the
// bandwidth.  The output D[4 q + r][j] (vocab 4 q + r, batch j) of the four
// waves is summed in LDS.
//
// Argmax.  A logit (after rounding to bf16) and its index form the key
// (orderable(bits) << 32) | (0xFFFFFFFF - index): the largest key is the
// largest value and, among equal values, the smallest index -- torch.argmax's
// rule, NaN counting as the largest value and -0 equal to +0.  Each
// workgroup stores its best key per batch row in the workspace; a second
// kernel (one workgroup per row) reduces them.  No state survives a call.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qwen2_decode.h"
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kHeadThreads = 256;
constexpr int kHeadWaves = 4;
constexpr int kBlockK = 128;  // hidden elements per block
constexpr int kMaxRows = 16;
constexpr int kReduceThreads = 1024;

struct LmHeadArgs {
    const uint16_t* x;   // [rows, hidden] bf16
    const uint16_t* w;   // [vocab, hidden] bf16
    uint16_t* logits;    // [rows, vocab] bf16
    uint64_t* keys;      // [rows, num_groups] best key per workgroup, or null
    int rows;
    int vocab;
    int hidden;
    int num_groups;      // gridDim.x
};

__device__ __forceinline__ uint64_t argmax_key(uint16_t bits, uint32_t index) {
    uint32_t ord;
    if ((bits & 0x7FFFu) > 0x7F80u) ord = 0xFFFFu;          // NaN: the largest
    else if (bits == 0x8000u) ord = 0x8000u;                // -0 == +0
    else ord = (bits & 0x8000u) ? (~bits & 0xFFFFu) : (bits | 0x8000u);
    return ((uint64_t)ord << 32) | (uint64_t)(0xFFFFFFFFu - index);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
    const uint32_t lo = __shfl_xor((uint32_t)v, mask);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), mask);
    return ((uint64_t)hi << 32) | lo;
}

template <int BPW, int kTiles>
__global__ __launch_bounds__(kHeadThreads) void lm_head_kernel(LmHeadArgs a) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int q = lane >> 4;
    const int j = lane & 15;
    const int nb = a.hidden / kBlockK;
    const int v0 = blockIdx.x * 16 * kTiles;

    // batch row j of x (zero beyond rows), this wave's blocks
    u32x4 xv[BPW][4];
#pragma unroll
    for (int bb = 0; bb < BPW; ++bb) {
        const int b = wave + kHeadWaves * bb;
        const bool live = j < a.rows && b < nb;
        const uint16_t* src = a.x + (int64_t)j * a.hidden + b * kBlockK + 8 * q;
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[bb][i] = live ? *(const u32x4*)(src + 32 * i) : u32x4{0u, 0u, 0u, 0u};
    }
    // vocab row v0 + 16 t + j (rows past the end re-read the last row; their
    // results are dropped)
    u32x4 wv[kTiles][BPW][4];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int row = min(v0 + 16 * t + j, a.vocab - 1);
#pragma unroll
        for (int bb = 0; bb < BPW; ++bb) {
            const int b = wave + kHeadWaves * bb;
            const uint16_t* src = a.w + (int64_t)row * a.hidden + b * kBlockK + 8 * q;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wv[t][bb][i] = b < nb ? *(const u32x4*)(src + 32 * i) : u32x4{0u, 0u, 0u, 0u};
        }
    }
    float4v acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        acc[t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int bb = 0; bb < BPW; ++bb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv[t][bb][i]),
                                                                 __builtin_bit_cast(bf16x8, xv[bb][i]), acc[t], 0, 0, 0);
    }

    __shared__ float4v red[kHeadWaves][kTiles][64];
    __shared__ uint64_t best[kTiles][16];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();

    // wave t (< kTiles) finishes tile t: lane (q, j) owns vocab 4q..4q+3 of batch j
    if (wave < kTiles) {
        const int t = wave;
        float4v s = red[0][t][lane];
#pragma unroll
        for (int w = 1; w < kHeadWaves; ++w) s += red[w][t][lane];
        uint64_t key = 0;
        if (j < a.rows) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int v = v0 + 16 * t + 4 * q + r;
                if (v < a.vocab) {
                    const uint16_t bits = float_to_bf16_bits(s[r]);
                    a.logits[(int64_t)j * a.vocab + v] = bits;
                    key = max_u64(key, argmax_key(bits, (uint32_t)v));
                }
            }
        }
        if (a.keys) {
            key = max_u64(key, shfl_xor_u64(key, 16));
            key = max_u64(key, shfl_xor_u64(key, 32));
            if (q == 0) best[t][j] = key;
        }
    }
    if (!a.keys) return;  // uniform over the grid
    __syncthreads();
    if (tid < a.rows) {
        uint64_t key = best[0][tid];
#pragma unroll
        for (int t = 1; t < kTiles; ++t) key = max_u64(key, best[t][tid]);
        a.keys[(int64_t)tid * a.num_groups + blockIdx.x] = key;
    }
}

// One workgroup per row: the largest of the row's workgroup keys.
__global__ __launch_bounds__(kReduceThreads) void lm_head_argmax_kernel(const uint64_t* keys, int num_groups,
                                                                        int64_t* argmax) {
    const int tid = threadIdx.x;
    const uint64_t* src = keys + (int64_t)blockIdx.x * num_groups;
    uint64_t key = 0;
#pragma unroll 4
    for (int g = tid; g < num_groups; g += kReduceThreads) key = max_u64(key, src[g]);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) key = max_u64(key, shfl_xor_u64(key, m));
    __shared__ uint64_t wave_best[kReduceThreads / 64];
    if ((tid & 63) == 0) wave_best[tid >> 6] = key;
    __syncthreads();
    if (tid == 0) {
        uint64_t k = wave_best[0];
#pragma unroll
        for (int w = 1; w < kReduceThreads / 64; ++w) k = max_u64(k, wave_best[w]);
        argmax[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu));
    }
}

// Tiles per workgroup: one for few rows (more workgroups in flight), two
// for many (halves the activation reads per weight byte), one again where
// two would not fit the registers.
int lm_head_tiles(int64_t rows, int64_t hidden) {
    const int64_t bpw = (hidden / kBlockK + kHeadWaves - 1) / kHeadWaves;
    return (rows > 8 && bpw <= 4) ? 2 : 1;
}

int64_t lm_head_groups(int64_t rows, int64_t vocab, int64_t hidden) {
    const int64_t per = 16 * lm_head_tiles(rows, hidden);
    return (vocab + per - 1) / per;
}

template <int BPW>
void launch_lm_head(const LmHeadArgs& a, int tiles, hipStream_t stream) {
    if constexpr (BPW <= 4) {
        if (tiles == 2) {
            hipLaunchKernelGGL((lm_head_kernel<BPW, 2>), dim3((unsigned)a.num_groups), dim3(kHeadThreads), 0, stream,
                               a);
            return;
        }
    }
    hipLaunchKernelGGL((lm_head_kernel<BPW, 1>), dim3((unsigned)a.num_groups), dim3(kHeadThreads), 0, stream, a);
}

}  // namespace
}  // namespace w4g64

using namespace w4g64;

extern "C" {

int64_t qwen2_lm_head_workspace_bytes(int64_t rows, int64_t vocab, int64_t hidden) {
    if (rows <= 0 || rows > kMaxRows || vocab <= 0 || vocab > 0x7FFFFFFF || hidden <= 0 || hidden % kBlockK ||
        hidden > 8 * kHeadWaves * kBlockK)
        return 0;
    return rows * lm_head_groups(rows, vocab, hidden) * (int64_t)sizeof(uint64_t);
}

int qwen2_lm_head(const void* x, const void* weight, void* logits, int64_t* argmax, int64_t rows, int64_t vocab,
                  int64_t hidden, void* workspace, int64_t workspace_bytes, void* stream) {
    if (rows < 0 || rows > kMaxRows)
        return set_error(W4G64_STATUS_INVALID_VALUE, "lm_head rows must be in [0, %d], got %lld", kMaxRows,
                         (long long)rows);
    if (hidden <= 0 || hidden % kBlockK || hidden > 8 * kHeadWaves * kBlockK)
        return set_error(W4G64_STATUS_INVALID_VALUE, "lm_head hidden must be a multiple of %d in [%d, %d], got %lld",
                         kBlockK, kBlockK, 8 * kHeadWaves * kBlockK, (long long)hidden);
    if (vocab <= 0 || vocab > 0x7FFFFFFF)
        return set_error(W4G64_STATUS_INVALID_VALUE, "lm_head vocab must be in [1, 2^31), got %lld", (long long)vocab);
    if (rows == 0) return clear_error();
    if (!x || !weight || !logits)
        return set_error(W4G64_STATUS_INVALID_VALUE, "x, weight and logits must be non-null device pointers");
    if ((((uintptr_t)x) & 15) || (((uintptr_t)weight) & 15))
        return set_error(W4G64_STATUS_INVALID_VALUE, "lm_head x and weight must be 16-byte aligned");
    LmHeadArgs a{};
    a.x = (const uint16_t*)x;
    a.w = (const uint16_t*)weight;
    a.logits = (uint16_t*)logits;
    a.rows = (int)rows;
    a.vocab = (int)vocab;
    a.hidden = (int)hidden;
    a.num_groups = (int)lm_head_groups(rows, vocab, hidden);
    if (argmax) {
        const int64_t need = qwen2_lm_head_workspace_bytes(rows, vocab, hidden);
        if (!workspace || workspace_bytes < need)
            return set_error(W4G64_STATUS_WORKSPACE, "lm_head argmax needs %lld workspace bytes, got %lld",
                             (long long)need, (long long)workspace_bytes);
        if (((uintptr_t)workspace) & 7)
            return set_error(W4G64_STATUS_INVALID_VALUE, "lm_head workspace must be 8-byte aligned");
        a.keys = (uint64_t*)workspace;
    }
    const int bpw = (int)((hidden / kBlockK + kHeadWaves - 1) / kHeadWaves);
    const int tiles = lm_head_tiles(rows, hidden);
    const hipStream_t s = (hipStream_t)stream;
    switch (bpw) {
        case 1: launch_lm_head<1>(a, tiles, s); break;
        case 2: launch_lm_head<2>(a, tiles, s); break;
        case 3: launch_lm_head<3>(a, tiles, s); break;
        case 4: launch_lm_head<4>(a, tiles, s); break;
        case 5: launch_lm_head<5>(a, tiles, s); break;
        case 6: launch_lm_head<6>(a, tiles, s); break;
        case 7: launch_lm_head<7>(a, tiles, s); break;
        default: launch_lm_head<8>(a, tiles, s); break;
    }
    hipError_t err = hipGetLastError();
    if (err == hipSuccess && argmax) {
        hipLaunchKernelGGL(lm_head_argmax_kernel, dim3((unsigned)rows), dim3(kReduceThreads), 0, s,
                           (const uint64_t*)a.keys, a.num_groups, argmax);
        err = hipGetLastError();
    }
    if (err != hipSuccess)
        return set_error(W4G64_STATUS_HIP_ERROR, "lm_head launch failed: %s", hipGetErrorString(err));
    return clear_error();
}

}  // extern "C"
