// Decode path: fused unpack + dequant + GEMV for 1..16 activation rows.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])   (+ bias[n])
// which is the reference's (x.float() @ W.t() + bias).to(x.dtype)
// (src/qwen_int4/backends.py:73-98) with the group scale applied once per
// 64-wide group in fp32.
//
// Mapping (one workgroup = 4 waves = 64 output features x one K split):
//   * each wave owns 16 consecutive output features n (MFMA B columns);
//     lane (n = lane % 16, q = lane / 16) loads 8 packed bytes per group
//     (q selects the 16-value quarter of the 64-value group), so a wave
//     instruction fetches 16 rows x 32 contiguous bytes;
//   * v_mfma_f32_16x16x32_{f16,bf16}: A = activations (16 rows, zero padded),
//     B = exact small-integer weights, two MFMAs per group;
//   * fp16 activations: B = (code - zero) built exactly with the 1024+n'
//     magic and one v_pk_add_f16 per pair; group scale applied to the MFMA
//     result in fp32;
//   * bf16 activations: B = 128 + n' (exact in bf16); the per-group result is
//     corrected by -(136 + zero) * sum_k x[m,k] before scaling;
//   * fp32 activations: each row is split exactly into three bf16 parts
//     (hi + mid + lo == x) that occupy three "virtual" A rows; the bf16 path
//     runs on them and the parts are summed in fp32.
//   * all weight loads of the wave's K range are issued before any math so
//     the whole split is in flight at once (HBM latency hiding by MLP).
//   * K splits across workgroups write fp32 partials to the workspace; the
//     last workgroup to arrive for a 64-column block (per-block atomic
//     counter) sums them in split order -- deterministic -- adds the bias,
//     converts and stores, then resets the counter to zero.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kWaves = 4;
constexpr int kBlockCols = kWaves * 16;       // output features per workgroup
constexpr int kMaxGroupsPerSplit = 12;        // 768 K values per split

struct GemvArgs {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;
    void* y;
    int M;      // activation rows
    int N;      // out_features
    int K;      // in_features
    int G;      // K / 64
    int gps;    // groups per split
    int splits;
    int mv;     // virtual A rows (M, or 3M for fp32 input)
    float* partials;     // [splits][M][N]
    unsigned* counters;  // [n_blocks]
};

template <int XK, int TILES>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ int s_last;
    constexpr int kParts = (XK == kF32) ? 3 : 1;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nb = blockIdx.x;
    const int split = blockIdx.y;
    const int g0 = split * a.gps;
    const int cnt = min(a.gps, a.G - g0);
    const int kbase = g0 * 64;
    const int row_stride = a.gps * 64 + 8;    // 16-bit elements, +16 B pad per row
    uint16_t* xs = (uint16_t*)smem;           // [mv][row_stride], slot-permuted
    float* sx = (float*)(smem + (size_t)a.mv * row_stride * 2);  // [gps][mv] group sums

    // ---- weights of this lane: issue every load of the split up front ----
    const int n = nb * kBlockCols + wave * 16 + (lane & 15);
    const int q = lane >> 4;
    const bool nvalid = n < a.N;
    u32x2 wq[kMaxGroupsPerSplit];
    float sc[kMaxGroupsPerSplit];
    int zr[kMaxGroupsPerSplit];
    // Branch-free: out-of-range rows/groups read row 0 / group 0 of the
    // split (always valid) and are zeroed afterwards, so every load of the
    // split is issued back to back.
    const int nrow = nvalid ? n : 0;
    const uint8_t* wrow = a.qweight + (int64_t)nrow * (a.K / 2) + (int64_t)g0 * 32 + 8 * q;
    const int64_t sbase = (int64_t)nrow * a.G + g0;
#pragma unroll
    for (int j = 0; j < kMaxGroupsPerSplit; ++j) {
        const int jj = j < cnt ? j : 0;
        wq[j] = __builtin_nontemporal_load((const u32x2*)(wrow + 32 * jj));
    }
#pragma unroll
    for (int j = 0; j < kMaxGroupsPerSplit; ++j) {
        const int jj = j < cnt ? j : 0;
        sc[j] = half_bits_to_float(a.scales[sbase + jj]);
        zr[j] = nibble_at(a.zeros, sbase + jj);
    }
    if (!nvalid) {
#pragma unroll
        for (int j = 0; j < kMaxGroupsPerSplit; ++j) {
            wq[j] = u32x2{0u, 0u};
            sc[j] = 0.0f;
            zr[j] = 0;
        }
    }

    // ---- stage this split's activations in LDS (slot order) ----
    const int items_per_row = cnt * 8;  // 8 values per item
    for (int it = tid; it < a.M * items_per_row; it += 256) {
        const int m = it / items_per_row;
        const int c = it - m * items_per_row;
        if constexpr (XK != kF32) {
            const u32x4 v = *(const u32x4*)((const uint16_t*)a.x + (int64_t)m * a.K + kbase + 8 * c);
            *(u32x4*)(xs + m * row_stride + 8 * c) = permute_slots(v);
        } else {
            const float* src = (const float*)a.x + (int64_t)m * a.K + kbase + 8 * c;
            const float4v f0 = *(const float4v*)src;
            const float4v f1 = *(const float4v*)(src + 4);
            uint16_t hi[8], mid[8], lo[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) split3_bf16(j < 4 ? f0[j] : f1[j - 4], hi[j], mid[j], lo[j]);
            u32x4 ph, pm, pl;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                ph[j] = (uint32_t)hi[2 * j] | ((uint32_t)hi[2 * j + 1] << 16);
                pm[j] = (uint32_t)mid[2 * j] | ((uint32_t)mid[2 * j + 1] << 16);
                pl[j] = (uint32_t)lo[2 * j] | ((uint32_t)lo[2 * j + 1] << 16);
            }
            *(u32x4*)(xs + m * row_stride + 8 * c) = permute_slots(ph);
            *(u32x4*)(xs + (a.M + m) * row_stride + 8 * c) = permute_slots(pm);
            *(u32x4*)(xs + (2 * a.M + m) * row_stride + 8 * c) = permute_slots(pl);
        }
    }
    __syncthreads();
    if constexpr (XK != kF16) {
        for (int idx = tid; idx < cnt * a.mv; idx += 256) {
            const int j = idx / a.mv;
            const int r = idx - j * a.mv;
            const uint16_t* src = xs + r * row_stride + 64 * j;
            float s = 0.0f;
            for (int k = 0; k < 64; ++k) s += bf16_bits_to_float(src[k]);
            sx[j * a.mv + r] = s;
        }
        __syncthreads();
    }

    // ---- MFMA over the split ----
    float4v acc[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[t] = float4v{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int j = 0; j < kMaxGroupsPerSplit; ++j) {
        if (j < cnt) {
            if constexpr (XK == kF16) {
                const _Float16 zl = (_Float16)(1032 + zr[j]);
                const _Float16 zh = (_Float16)(72 + zr[j]);
                const half8 b0 = dequant8_f16_int(wq[j][0], half2v{zl, zl}, half2v{zh, zh});
                const half8 b1 = dequant8_f16_int(wq[j][1], half2v{zl, zl}, half2v{zh, zh});
#pragma unroll
                for (int t = 0; t < TILES; ++t) {
                    const int row = 16 * t + (lane & 15);
                    half8 a0 = {}, a1 = {};
                    if (row < a.mv) {
                        const uint16_t* src = xs + row * row_stride + 64 * j + 16 * q;
                        a0 = *(const half8*)src;
                        a1 = *(const half8*)(src + 8);
                    }
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(sc[j], d[r], acc[t][r]);
                }
            } else {
                const bf16x8 b0 = dequant8_bf16_biased(wq[j][0]);
                const bf16x8 b1 = dequant8_bf16_biased(wq[j][1]);
                const float corr = 136.0f + (float)zr[j];
#pragma unroll
                for (int t = 0; t < TILES; ++t) {
                    const int row = 16 * t + (lane & 15);
                    bf16x8 a0 = {}, a1 = {};
                    if (row < a.mv) {
                        const uint16_t* src = xs + row * row_stride + 64 * j + 16 * q;
                        a0 = *(const bf16x8*)src;
                        a1 = *(const bf16x8*)(src + 8);
                    }
                    float4v d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int vr = 16 * t + 4 * q + r;
                        const float s_x = vr < a.mv ? sx[j * a.mv + vr] : 0.0f;
                        acc[t][r] = fmaf(sc[j], fmaf(-corr, s_x, d[r]), acc[t][r]);
                    }
                }
            }
        }
    }

    // ---- epilogue: gather the 16 x 64 tile(s), fold fp32 parts ----
    __syncthreads();  // xs / sx no longer read
    float* red = (float*)smem;  // [16 * TILES][64]
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(16 * t + 4 * q + r) * kBlockCols + wave * 16 + (lane & 15)] = acc[t][r];
    __syncthreads();

    const int col0 = nb * kBlockCols;
    for (int idx = tid; idx < a.M * kBlockCols; idx += 256) {
        const int m = idx / kBlockCols;
        const int c = idx - m * kBlockCols;
        const int nn = col0 + c;
        if (nn >= a.N) continue;
        float v = 0.0f;
#pragma unroll
        for (int p = 0; p < kParts; ++p) v += red[(p * a.M + m) * kBlockCols + c];
        if (a.splits == 1) {
            v += load_bias(a.bias, a.bias_kind, nn);
            store_out<XK>(a.y, (int64_t)m * a.N + nn, v);
        } else {
            __hip_atomic_store(a.partials + ((int64_t)split * a.M + m) * a.N + nn, v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (a.splits == 1) return;

    // ---- split-K: the last workgroup of this column block reduces ----
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + nb, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)a.splits - 1u);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = tid; idx < a.M * kBlockCols; idx += 256) {
        const int m = idx / kBlockCols;
        const int c = idx - m * kBlockCols;
        const int nn = col0 + c;
        if (nn >= a.N) continue;
        float v = 0.0f;
        for (int s = 0; s < a.splits; ++s)
            v += __hip_atomic_load(a.partials + ((int64_t)s * a.M + m) * a.N + nn, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        v += load_bias(a.bias, a.bias_kind, nn);
        store_out<XK>(a.y, (int64_t)m * a.N + nn, v);
    }
    if (tid == 0) __hip_atomic_store(a.counters + nb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int XK, int TILES>
hipError_t launch_typed(const GemvArgs& args, const GemvPlan& plan, size_t lds, hipStream_t stream,
                        hipEvent_t start, hipEvent_t stop) {
    return launch_kernel(gemv_kernel<XK, TILES>, dim3(plan.n_blocks, plan.splits), dim3(256), lds, stream, start,
                         stop, args);
}

}  // namespace

GemvPlan plan_gemv(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    GemvPlan plan{};
    const int64_t groups = in_features / 64;
    const int64_t parts = (x_kind == kF32) ? 3 : 1;
    plan.tiles = (int)((rows * parts + 15) / 16);
    plan.n_blocks = (int)((out_features + kBlockCols - 1) / kBlockCols);
    // Aim for ~4 workgroups per CU (256 CUs) while keeping the split-K
    // partial traffic (write + read, fp32) under 1/8 of the packed weight
    // bytes: 2 * S * rows * N * 4 <= N * K / 16  =>  S <= K / (128 * rows).
    int64_t target = (1024 + plan.n_blocks - 1) / plan.n_blocks;
    int64_t traffic_cap = in_features / (128 * rows);
    int64_t splits = target < traffic_cap ? target : traffic_cap;
    if (splits < 1) splits = 1;
    if (splits > groups) splits = groups;
    int64_t gps = (groups + splits - 1) / splits;
    if (gps > kMaxGroupsPerSplit) gps = kMaxGroupsPerSplit;
    // Activation staging (virtual rows x split width, 16-bit) plus the group
    // sums must fit a 60 KB dynamic-LDS budget (64 KB per workgroup).
    const int64_t mv = rows * parts;
    auto lds_for = [&](int64_t g) {
        int64_t bytes = mv * (g * 64 + 8) * 2 + g * mv * 4;
        const int64_t red = (int64_t)16 * plan.tiles * kBlockCols * 4;
        return bytes > red ? bytes : red;
    };
    while (gps > 1 && lds_for(gps) > 60 * 1024) --gps;
    splits = (groups + gps - 1) / gps;
    plan.lds_bytes = lds_for(gps);
    plan.splits = (int)splits;
    plan.groups_per_split = (int)((groups + splits - 1) / splits);
    plan.counter_bytes = splits > 1 ? kGemvCounterBytes : 0;
    plan.workspace_bytes = splits > 1 ? plan.counter_bytes + splits * rows * out_features * 4 : 0;
    return plan;
}

const char* gemv_kernel_name(const GemvPlan& plan, int x_kind) {
    static const char* names[3][3] = {
        {"gemv_kernel<f16,1>", "gemv_kernel<f16,2>", "gemv_kernel<f16,3>"},
        {"gemv_kernel<bf16,1>", "gemv_kernel<bf16,2>", "gemv_kernel<bf16,3>"},
        {"gemv_kernel<f32,1>", "gemv_kernel<f32,2>", "gemv_kernel<f32,3>"},
    };
    int t = plan.tiles < 1 ? 1 : (plan.tiles > 3 ? 3 : plan.tiles);
    return names[x_kind - 1][t - 1];
}

hipError_t launch_gemv(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
    GemvArgs args{};
    args.x = p.x;
    args.qweight = p.qweight;
    args.scales = p.scales;
    args.zeros = p.zeros;
    args.bias = p.bias;
    args.bias_kind = p.bias_kind;
    args.y = p.y;
    args.M = (int)p.rows;
    args.N = (int)p.out_features;
    args.K = (int)p.in_features;
    args.G = (int)(p.in_features / 64);
    args.gps = plan.groups_per_split;
    args.splits = plan.splits;
    args.mv = (int)(p.rows * (p.x_kind == kF32 ? 3 : 1));
    args.counters = (unsigned*)workspace;
    args.partials = workspace ? (float*)((char*)workspace + plan.counter_bytes) : nullptr;
    const size_t lds = (size_t)plan.lds_bytes;
    switch (p.x_kind) {
        case kF16:
            return launch_typed<kF16, 1>(args, plan, lds, stream, start, stop);
        case kBF16:
            return launch_typed<kBF16, 1>(args, plan, lds, stream, start, stop);
        default:
            if (plan.tiles == 1) return launch_typed<kF32, 1>(args, plan, lds, stream, start, stop);
            if (plan.tiles == 2) return launch_typed<kF32, 2>(args, plan, lds, stream, start, stop);
            return launch_typed<kF32, 3>(args, plan, lds, stream, start, stop);
    }
}

}  // namespace w4g64
