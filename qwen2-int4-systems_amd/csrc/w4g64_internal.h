// Internal launch interface between the C ABI (w4g64_capi.hip) and the
// kernel translation units.  Host code only; arguments are already validated.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4g64 {

struct LinearProblem {
    const void* x;
    int x_kind;  // XKind
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;  // 0 none, else XKind
    void* y;
    int64_t rows;
    int64_t out_features;
    int64_t in_features;
    int paired = 0;  // decode GEMV: paired gate|up epilogue writing SiLU-product planes
    // decode GEMV, x_kind kNormB / kNormF: x is the residual stream (bf16); the
    // activation is RMSNorm(x + delta) (weight, eps), and x + delta (bf16) is
    // stored to norm_out_sum by one workgroup
    const void* norm_delta = nullptr;
    const uint16_t* norm_weight = nullptr;
    float norm_eps = 0.0f;
    void* norm_out_sum = nullptr;
    int norm_delta_parts = 1;  // kNormP: fp32 partial sums [parts][rows][in_features] added in order
    // decode GEMV: write the fp32 split-K partial sums [splits][rows][out_features]
    // here (no bias, no reduction launch; one split: the fp32 result)
    float* partials_out = nullptr;
    // decode GEMV, x_kind kAttnM: x is the decode attention's partial results
    // (att_chunks chunks per (row, key/value head), att_group query heads per
    // key/value head, att_kv_heads key/value heads)
    int att_chunks = 0;
    int att_group = 0;
    int att_kv_heads = 0;
};

// Decode GEMV (rows <= kGemvMaxRows).
constexpr int kGemvMaxRows = 16;
// Largest out_features the decode path takes (its grid and index arithmetic
// stay within 32 bits).
constexpr int64_t kGemvMaxOutFeatures = int64_t(1) << 26;
// Workspace of a split-K GEMV call: the fp32 partial sums [splits][rows][out_features].
struct GemvPlan {
    int kind;              // 0: segmented kernel (any rows); 1: 9..16-row kernel (fp16/bf16)
    int waves;             // kind 1: waves per 16-feature block (they split its K range)
    int fblocks;           // kind 1: 16-feature blocks per workgroup
    int segments;          // K segments per wave (16 / output features per wave)
    int steps;             // group steps per lane (compile-time bucket >= groups_per_split / segments)
    int n_blocks;          // column blocks (kind 0: 4 * 16 / segments output features each; kind 1: 16)
    int splits;            // K splits across workgroups
    int groups_per_split;  // 64-wide K groups per split
    int tiles;             // 16-row MFMA A tiles (fp32 input uses 3 bf16 parts per row)
    int kparts = 1;        // kind 2: K parts per workgroup (its waves split K)
    int stage = 1;         // kind 2, 4: staging loads per lane
    int rbw = 1;           // kind 4: row blocks per wave
    int depth = 1;         // kind 4: steps of loads kept in flight
    int form = 0;          // kind 4: activation form (0 plain, 1 bf16 planes, 2 / 3 RMSNorm with bf16 / fp32-parts delta)
    int pair = 0;          // kind 4: paired gate|up epilogue (SiLU-product planes)
    int64_t lds_bytes;     // dynamic LDS per workgroup
    int64_t workspace_bytes;
};
GemvPlan plan_gemv(int64_t rows, int64_t out_features, int64_t in_features, int x_kind);
// Same, with the segment count and K split forced (> 0) -- for tuning sweeps.
GemvPlan plan_gemv(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, int force_segments,
                   int force_splits);
hipError_t launch_gemv(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                       hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Second kernel of a K-split GEMV call (either decode GEMV kernel): adds the
// fp32 partial sums [splits][M][N] in split order, adds the bias and stores
// out_kind values; paired (N = 2 I gate|up features): stores the three bf16
// planes of silu(bf16(gate)) * bf16(up) per (row, i).
hipError_t launch_split_reduce(const float* partials, const void* bias, int bias_kind, void* y, int M, int N,
                               int splits, bool paired, int out_kind, hipStream_t stream, hipEvent_t stop);
const char* gemv_kernel_name(const GemvPlan& plan, int x_kind);
// Plan of the paired gate|up GEMV (bf16, out_features = 2 I rows: gate then
// up): the segmented kernel with at most 8 segments, so that every wave holds
// whole (gate, up) pairs.
GemvPlan plan_gemv_paired(int64_t rows, int64_t out_features, int64_t in_features, int x_kind = 2 /* bf16 */);
// The 9..16-row kernel's plan with its shape forced (> 0: feature blocks per
// workgroup, waves per block, K splits) -- for tuning sweeps.  false if the
// rows or the shape do not fit it.
bool plan_rows16(int64_t rows, int64_t out_features, int64_t in_features, GemvPlan& plan, int force_fblocks,
                 int force_waves, int force_splits);
hipError_t launch_gemv16(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                         hipEvent_t start, hipEvent_t stop);

// Lean decode GEMV (one fp16/bf16 row, even group count, N G 2 and N P
// multiples of 16, at most three 16-byte weight loads per lane): whole rows
// per workgroup, no workspace.  plan.kind = 2; segments, fblocks (row blocks)
// and kparts (K parts) select the shape, stage the staging loads per lane.
bool plan_seg(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, GemvPlan& plan);
// Pointer alignment and forms the lean kernel takes (plain linear only).
bool seg_supported(const LinearProblem& p);
hipError_t launch_gemv_seg(const LinearProblem& p, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                           hipEvent_t stop);
// One-row RMSNorm + gate|up planes form of the lean kernel (plan.kind = 3):
// bf16 residual and delta, no bias, out_features / 2 a multiple of 8,
// in_features a multiple of 128 up to 1536, 16-byte aligned weights.
bool plan_seg_norm_planes(const LinearProblem& p, GemvPlan& plan);
hipError_t launch_gemv_seg_norm_planes(const LinearProblem& p, const GemvPlan& plan, hipStream_t stream);

// Pipelined decode GEMV (plan.kind = 4; 1..16 fp16/bf16 rows, in_features a
// multiple of 128): segments, tiles (A tiles), fblocks (wave rows), kparts
// (K parts per workgroup), rbw (row blocks per wave), steps (pair steps per
// wave), depth (steps in flight) and stage (staging loads per lane) select
// the kernel; finish_pipe_plan fills in the grid, K splits, LDS and
// workspace.  K splits store fp32 partial sums reduced by the split-reduce
// kernel (or, with partials_out, left to the caller).
bool finish_pipe_plan(int64_t rows, int64_t out_features, int64_t in_features, GemvPlan& plan);
bool plan_pipe(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, GemvPlan& plan);
// Activation forms of the pipelined kernel (GemvPlan::form); each may be
// paired (gate rows then up rows, SiLU-product planes out).
enum PipeForm : int {
    kPlain = 0,       // fp16 / bf16 rows
    kPlanes3 = 1,     // three bf16 planes [3][Mo][K] (hi + mid + lo), staged as 3 Mo rows, summed; fp32 out
    kNormBf16 = 2,    // RMSNorm(residual + bf16 delta), one row
    kNormParts = 3,   // RMSNorm(residual + sum of fp32 partial sums), one row
    kAttnMerge = 4,   // the decode attention's per-chunk partial results, merged; one row
    kGrouped = 5,     // fp16 / bf16 rows (up to 16), one quantization group per MFMA: all rows in one A tile
};

// The decode attention's workspace: arrival counters (256-byte aligned
// area), then fp32 partial results [batch * kv_heads][chunks][kAttnPartFloats],
// chunk c of a (sequence, key/value head) covering positions 64 c .. 64 c +
// 63: m[8] (score maximum per query head of the group), l[8] (sum of
// exp(score - m)), then the 8 heads' exp-weighted value sums [8][128].
constexpr int kAttnChunk = 64;
constexpr int kAttnMaxGroup = 8;
constexpr int kAttnHeadDim = 128;
constexpr int kAttnPartFloats = 2 * kAttnMaxGroup + kAttnMaxGroup * kAttnHeadDim;
inline int64_t attention_counter_bytes(int64_t batch, int64_t kv_heads) {
    return (batch * kv_heads * (int64_t)sizeof(unsigned) + 255) / 256 * 256;
}
// Chunks the attention-merge form of the pipelined GEMV takes (the cache's
// max_length up to 1024 positions): it loads every chunk's partial result.
constexpr int kAttnMergeMaxChunks = 16;
bool plan_pipe_fused(int form, bool paired, int64_t rows, int64_t out_features, int64_t in_features,
                     GemvPlan& plan);
bool pipe_supported(const LinearProblem& p);
bool pipe_plan_launchable(const GemvPlan& plan);
hipError_t launch_gemv_pipe(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                            hipEvent_t start = nullptr, hipEvent_t stop = nullptr);

// Prefill GEMM (rows > 16): a staging kernel writes the activations as fp16
// rows (scaled by a power of two per row; fp32-class kinds as hi|lo planes)
// into the workspace, the GEMM kernel multiplies them by the exact integer
// (code - zero) and applies each group's scale in fp32.  Tiles of a last,
// mostly empty round of workgroups (or all tiles, when there are fewer than
// the device's workgroup slots) are split along K; their fp32 partial sums
// live at the start of the workspace and a third kernel adds them up.
bool gemm_supported(const LinearProblem& p);
int64_t gemm_workspace_bytes(int64_t rows, int64_t out_features, int64_t in_features, int x_kind);
const char* gemm_kernel_name(int64_t rows, int64_t out_features, int64_t in_features, int x_kind);
hipError_t launch_gemm(const LinearProblem& p, void* workspace, hipStream_t stream, hipEvent_t start = nullptr,
                       hipEvent_t stop = nullptr);

// Launch a kernel; with events, hipExtLaunchKernelGGL records them at the
// kernel's own start and end (what a profiler reports as its duration).
template <typename F, typename... Args>
hipError_t launch_kernel(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, hipEvent_t start,
                         hipEvent_t stop, Args... args) {
    if (start || stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, start, stop, 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
    return hipGetLastError();
}

// Per-thread error string of the C ABI (defined with the w4g64_* entry
// points): set_error formats the message and returns `status`; clear_error
// empties it and returns 0.
int set_error(int status, const char* fmt, ...);
int clear_error();

// Primitives.
hipError_t launch_unpack(const uint8_t* packed, int8_t* out, int64_t elements, hipStream_t stream);
hipError_t launch_dequant(const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros, float* out,
                          int64_t out_features, int64_t in_features, hipStream_t stream);

#ifdef W4G64_TIMELINE
// The timeline buffer registered by w4g64_timeline_register (profiling builds).
extern unsigned long long* g_timeline_stamps;
extern int g_timeline_workgroups;
#endif

}  // namespace w4g64
