// Decode path for 9..16 activation rows (fp16 / bf16): fused unpack +
// dequant + GEMV with the K range split across the waves of a workgroup.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])   (+ bias[n])
// (src/qwen_int4/backends.py:73-98, group scale applied once per group in fp32).
//
// With 9..16 rows the activation rows fill the 16 A rows of
// v_mfma_f32_16x16x32_{f16,bf16} on their own, so:
//   * a workgroup owns one block of 16 output features (the 16 B columns);
//     its KW waves take the groups of its K range round robin (wave w takes
//     g0 + w, g0 + w + KW, ...), and their partial sums meet in LDS;
//   * every lane loads its A fragment straight from global memory (the
//     activations are small and stay in L2): row lane % 16, the 16 values
//     [16 q, 16 q + 16) of the group, q = lane / 16 -- the same K values as the
//     8 packed bytes it loads for its B column -- permuted into the slot
//     order the nibble decode produces.  No staging wave, no workgroup barrier
//     before the MFMAs;
//   * all scale, zero, weight and activation loads of a lane are issued
//     before the first MFMA (in that order), so the whole slice is in flight
//     at once and the MFMA of step t waits only for loads issued before its
//     own activations;
//   * fp16: B = (code - zero) exact (1024 + n' magic, one v_pk_add_f16 per
//     pair); bf16: B = 128 + n' exact, and the group result is corrected by
//     -(136 + zero) * sum_k x[m,k]; that row sum comes from one more MFMA pair
//     against an all-ones B, which leaves it in the accumulator's own layout.
//   * a K split across workgroups (when a wave would otherwise hold more than
//     18 group steps, or for long K with few column blocks: while a wave keeps
//     more than 6 steps and fewer than 256 workgroups run) uses the same
//     coherent last-arriver protocol as the segmented kernel.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

struct Gemv16Args {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;
    void* y;
    int M;       // activation rows, 9..16
    int N;       // out_features
    int K;       // in_features
    int G;       // K / 64
    int gps;     // groups per K split
    int splits;  // K splits across workgroups
    float* partials;     // [splits][M][N]
    unsigned* counters;  // [column blocks]
};

template <int XK, int STEPS, int KW>
__global__ __launch_bounds__(KW * 64) void gemv16_kernel(Gemv16Args a) {
    __shared__ float red[KW][16][16];  // [wave][row][feature]
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int nb = blockIdx.x;
    const int split = blockIdx.y;
    const int g0 = split * a.gps;
    const int cnt = min(a.gps, a.G - g0);

    const int j = lane & 15;  // B column = output feature, A row = activation row
    const int q = lane >> 4;  // 16-value quarter of the group
    const int n = nb * 16 + j;
    const bool nvalid = n < a.N;
    const int nrow = nvalid ? n : 0;
    const int mrow = j < a.M ? j : a.M - 1;  // rows past M load a valid row; their outputs are dropped
    const uint8_t* wrow = a.qweight + (int64_t)nrow * (a.K / 2) + 8 * q;
    const uint16_t* xrow = (const uint16_t*)a.x + (int64_t)mrow * a.K + 16 * q;
    const int64_t sbase = (int64_t)nrow * a.G;

    // Loads complete in order, so any use of a loaded value waits for every
    // load issued before it.  All scale and zero loads go first (their decode
    // may be scheduled early), then every weight load, then every activation
    // load; no use is scheduled before the last load is issued.
    // Long K ranges (more than 12 steps) load their activations in two
    // phases, the second after the first half of the MFMAs, to stay within 256
    // registers; the weights are always in flight at once.
    constexpr int kPhases = STEPS > 12 ? 2 : 1;
    constexpr int kChunk = (STEPS + kPhases - 1) / kPhases;
    u32x2 wq[STEPS];
    uint32_t sraw[STEPS];
    uint32_t zraw[STEPS];
    auto group_of = [&](int t) {
        const int gl = wave + KW * t;
        return gl < cnt ? g0 + gl : g0;  // past the range: re-read group g0, zero scale below
    };
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int64_t e = sbase + group_of(t);
        sraw[t] = a.scales[e];
        zraw[t] = (uint32_t)a.zeros[e >> 1] >> (4 * (e & 1));
    }
#pragma unroll
    for (int t = 0; t < STEPS; ++t)
        wq[t] = __builtin_nontemporal_load((const u32x2*)(wrow + (int64_t)group_of(t) * 32));

    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ph = 0; ph < kPhases; ++ph) {
        u32x4 xa[kChunk][2];
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
            const int t = ph * kChunk + c;
            if (t < STEPS) {
                xa[c][0] = *(const u32x4*)(xrow + (int64_t)group_of(t) * 64);
                xa[c][1] = *(const u32x4*)(xrow + (int64_t)group_of(t) * 64 + 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
            const int t = ph * kChunk + c;
            if (t >= STEPS) continue;
            const bool live = nvalid && wave + KW * t < cnt;
            const float sct = live ? half_bits_to_float((uint16_t)sraw[t]) : 0.0f;
            const int zn = (int)(zraw[t] & 0xF);
            const int zrt = zn - ((zn & 8) << 1);
            const u32x4 a0 = permute_slots(xa[c][0]);
            const u32x4 a1 = permute_slots(xa[c][1]);
            float4v d;
            if constexpr (XK == kF16) {
                const _Float16 zl = (_Float16)(1032 + zrt);
                const _Float16 zh = (_Float16)(72 + zrt);
                const half8 b0 = dequant8_f16_int(wq[t][0], half2v{zl, zl}, half2v{zh, zh});
                const half8 b1 = dequant8_f16_int(wq[t][1], half2v{zl, zl}, half2v{zh, zh});
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a0), b0,
                                                           float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a1), b1, d, 0, 0, 0);
            } else {
                const bf16x8 b0 = dequant8_bf16_biased(wq[t][0]);
                const bf16x8 b1 = dequant8_bf16_biased(wq[t][1]);
                const bf16x8 ones =
                    __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), b0,
                                                            float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), b1, d, 0, 0, 0);
                float4v sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), ones,
                                                                     float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), ones, sx, 0, 0, 0);
                const float corr = 136.0f + (float)zrt;
#pragma unroll
                for (int r = 0; r < 4; ++r) d[r] = fmaf(-corr, sx[r], d[r]);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r] = fmaf(sct, d[r], acc[r]);
        }
    }

    // ---- combine the waves' partial sums: D row = 4 q + r, column = j ----
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * q + r][j] = acc[r];
    __syncthreads();

    float v = 0.0f;
    const int m = tid >> 4;  // threads 0..255: (row, feature)
    const int c = tid & 15;
    const int nn = nb * 16 + c;
    const bool mine = tid < 256 && m < a.M && nn < a.N;
    if (tid < 256) {
#pragma unroll
        for (int w = 0; w < KW; ++w) v += red[w][m][c];  // fixed order: deterministic
    }
    if (a.splits == 1) {
        if (mine) store_out<XK>(a.y, (int64_t)m * a.N + nn, v + load_bias(a.bias, a.bias_kind, nn));
        return;
    }

    // ---- K split across workgroups: the last arrival of the block reduces ----
    // Partials travel through device-coherent (sc1) atomic stores and loads;
    // the wait completes this workgroup's partial stores before its arrival is
    // counted, and the reducer loads only after its counter update returned.
    if (mine)
        __hip_atomic_store(a.partials + ((int64_t)split * a.M + m) * a.N + nn, v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + nb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)a.splits - 1u);
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if (mine) {
        float s = 0.0f;
        for (int sp = 0; sp < a.splits; ++sp)
            s += __hip_atomic_load(a.partials + ((int64_t)sp * a.M + m) * a.N + nn, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        store_out<XK>(a.y, (int64_t)m * a.N + nn, s + load_bias(a.bias, a.bias_kind, nn));
    }
    if (tid == 0) __hip_atomic_store(a.counters + nb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int XK, int KW>
hipError_t launch_steps16(const Gemv16Args& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                          hipEvent_t stop) {
    const dim3 grid(plan.n_blocks, plan.splits);
    switch (plan.steps) {
        case 2: return launch_kernel(gemv16_kernel<XK, 2, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
        case 3: return launch_kernel(gemv16_kernel<XK, 3, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
        case 6: return launch_kernel(gemv16_kernel<XK, 6, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
        case 9: return launch_kernel(gemv16_kernel<XK, 9, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
        case 12: return launch_kernel(gemv16_kernel<XK, 12, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
        default: return launch_kernel(gemv16_kernel<XK, 18, KW>, grid, dim3(KW * 64), 0, stream, start, stop, args);
    }
}

}  // namespace

hipError_t launch_gemv16(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                         hipEvent_t start, hipEvent_t stop) {
    Gemv16Args args{};
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
    args.counters = (unsigned*)workspace;
    args.partials = workspace ? (float*)((char*)workspace + plan.counter_bytes) : nullptr;
    if (p.x_kind == kF16)
        return plan.waves == 8 ? launch_steps16<kF16, 8>(args, plan, stream, start, stop)
                               : launch_steps16<kF16, 4>(args, plan, stream, start, stop);
    return plan.waves == 8 ? launch_steps16<kBF16, 8>(args, plan, stream, start, stop)
                           : launch_steps16<kBF16, 4>(args, plan, stream, start, stop);
}

}  // namespace w4g64
