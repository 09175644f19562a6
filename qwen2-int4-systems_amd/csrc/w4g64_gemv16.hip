// Decode path for 9..16 activation rows (fp16 / bf16): fused unpack +
// dequant + GEMV, the activations staged once per workgroup in LDS.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])   (+ bias[n])
// (src/qwen_int4/backends.py:73-98, group scale applied once per group in fp32).
//
// With 9..16 rows the activation rows fill the 16 A rows of
// v_mfma_f32_16x16x32_{f16,bf16} on their own, so:
//   * a workgroup owns FB blocks of 16 output features (the 16 B columns of
//     a wave's MFMA); KW waves work on each block and take the groups of the
//     workgroup's K range round robin (wave kw takes g0 + kw, g0 + kw + KW,
//     ...); their partial sums meet in LDS at the end;
//   * the activations of the K range (rows x groups x 64 values) are staged
//     once per workgroup: every lane first issues its share of dense 16-byte
//     loads, then every weight, scale and zero load of its steps.  A wave's
//     loads return in issue order, so the activations arrive first; they go
//     to LDS in MFMA slot order (bf16: with the group sums for the zero
//     correction, reduced over 8 lanes), and a barrier over LDS alone lets
//     the MFMA steps start while the weights still stream in.  Staging
//     FB blocks' worth of features per workgroup divides the activation
//     traffic (M / 4 bytes of activations per weight byte per block) by FB;
//   * fp16: B = (code - zero) exact (1024 + n' magic, one v_pk_add_f16 per
//     pair); bf16: B = 128 + n' exact, and the group result is corrected by
//     -(136 + zero) * sum_{k in g} x[m,k].
//   * a K split across workgroups (long K: the staged range must fit LDS)
//     stores fp32 partial sums that the split-reduce kernel adds up, as for
//     the segmented kernel.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

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
    float* partials;  // [splits][M][N]
    W4G64_TIMELINE_FIELDS
};

// Activation items (8 values) a lane stages: 16 rows x KW STEPS groups x 8
// items over KW FB waves.
template <int STEPS, int FB>
constexpr int stage_items16() {
    return (2 * STEPS + FB - 1) / FB;
}

// Sum over the 8 lanes 8i..8i+7; every one of them gets the same bits.
__device__ __forceinline__ float sum8_lanes16(float s) {
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x4E, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x141, 0xF, 0xF, false));
    return s;
}

template <int XK, int STEPS, int KW, int FB>
__global__ __launch_bounds__(KW * FB * 64) void gemv16_kernel(Gemv16Args a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    __shared__ float red[KW * FB][16][16];  // [wave][row][feature]
    constexpr int kThreads16 = KW * FB * 64;
    constexpr int kStage = stage_items16<STEPS, FB>();
    constexpr int kCols = 16 * FB;  // output features per workgroup

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);
    const int fb = wave % FB;  // this wave's 16-feature block
    const int kw = wave / FB;  // this wave's share of the groups
    const int nb = blockIdx.x;
    const int split = blockIdx.y;
    const int g0 = split * a.gps;
    const int cnt = min(a.gps, a.G - g0);
    const int row_stride = a.gps * 64 + 8;  // 16-bit elements per staged row (+16 B pad)
    uint16_t* xs = (uint16_t*)smem;         // [M][row_stride], slot order
    float* sx = (float*)(smem + (size_t)a.M * row_stride * 2);  // [M][gps] group sums (bf16)

    const int j = lane & 15;  // B column = output feature, A row = activation row
    const int q = lane >> 4;  // 16-value quarter of the group
    const int n = nb * kCols + fb * 16 + j;
    const bool nvalid = n < a.N;
    const int nrow = nvalid ? n : 0;
    const uint8_t* wrow = a.qweight + (int64_t)nrow * (a.K / 2) + 8 * q;

    // ---- 1. activation loads: item it = kThreads16 u + tid (8 values of row m) ----
    // Lanes past the last item take the item at the same place in the last
    // group, so they load, sum and store exactly what that group's own lanes
    // do: no branch anywhere before the MFMA loop.
    const int kbase = g0 * 64;
    const int items_per_row = cnt * 8;
    const int total = a.M * items_per_row;
    const float inv_items = 1.0f / (float)items_per_row;
    auto item_rc = [&](int it, int& m, int& c) {  // branch-free; it < 2^24
        m = (int)((float)it * inv_items);
        c = it - m * items_per_row;
        const int adj = (int)(c >= items_per_row) - (int)(c < 0);
        m += adj;
        c -= adj * items_per_row;
    };
    u32x4 v[kStage];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
        const int it = kThreads16 * u + tid;
        int m, c;
        item_rc(it < total ? it : total - 8 + (tid & 7), m, c);
        v[u] = *(const u32x4*)((const uint16_t*)a.x + (int64_t)m * a.K + kbase + 8 * c);
    }
    // ---- 1b. scale and zero-point runs of the workgroup's features over its K range ----
    // Feature slot f (n = nb kCols + f, clamped to N - 1) has its scales at
    // bytes [2 (n G + g0), + 2 cnt) and its zero nibbles at elements
    // [n G + g0, + cnt); each run is staged in 16-byte chunks from the
    // aligned-down start, one scale chunk and one zero chunk per thread
    // (clamped thread indices repeat the last chunk); bytes past an
    // array's end read 0.
    constexpr int kScChunks = (2 * KW * STEPS + 15) / 16 + 1;
    constexpr int kZbChunks = (KW * STEPS / 2 + 1 + 15) / 16 + 1;
    static_assert(16 * FB * kScChunks <= kThreads16 && 16 * FB * kZbChunks <= kThreads16, "one chunk per thread");
    __shared__ __attribute__((aligned(16))) unsigned char scl[kCols][kScChunks * 16];
    __shared__ __attribute__((aligned(16))) unsigned char zbl[kCols][kZbChunks * 16];
    auto run_start = [&](int nf, bool zeros) {
        const uint32_t e = (uint32_t)nf * (uint32_t)a.G + (uint32_t)g0;
        return zeros ? (e >> 1) & ~15u : (2u * e) & ~15u;
    };
    const int ts = min(tid, kCols * kScChunks - 1), tz = min(tid, kCols * kZbChunks - 1);
    const int fs = ts / kScChunks, cs = ts - fs * kScChunks;
    const int fz = tz / kZbChunks, cz = tz - fz * kZbChunks;
    u32x4 svec, zvec;
    {
        const uint32_t ng = (uint32_t)a.N * (uint32_t)a.G;
        const __amdgpu_buffer_rsrc_t s_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, 0, (int)(2u * ng), 0x00020000);
        const __amdgpu_buffer_rsrc_t z_rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.zeros, 0, (int)((ng + 1u) >> 1), 0x00020000);
        svec = load16_bounded(s_rsrc, run_start(min(nb * kCols + fs, a.N - 1), false) + 16u * cs, 2u * ng);
        zvec = load16_bounded(z_rsrc, run_start(min(nb * kCols + fz, a.N - 1), true) + 16u * cz, (ng + 1u) >> 1);
    }
    // (the empty asm statements with a memory clobber fix the issue order)
    asm volatile("" ::: "memory");
    // Every wave's activation loads are issued before any wave's weight
    // loads: a CU returns vector memory data in issue order, so a wave whose
    // activation loads queue behind another wave's weight stream receives
    // them (measured) 1.3-1.5 us late for every wave ahead of it on its SIMD.
    // The barrier waits for no memory.
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // ---- 2. weight loads of every step, in step order ----
    // Steps past the K range re-read group g0 and get a zero scale.
    u32x2 wq[STEPS];
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int gl = kw + KW * t;
        const int g = gl < cnt ? g0 + gl : g0;
        wq[t] = __builtin_nontemporal_load((const u32x2*)(wrow + (int64_t)g * 32));
        asm volatile("" ::: "memory");
    }
    // Nothing that uses the activations may move above the last load issue.
#pragma unroll
    for (int u = 0; u < kStage; ++u) asm volatile("" : "+v"(v[u]));
    asm volatile("" : "+v"(svec), "+v"(zvec));
    *(u32x4*)&scl[fs][16 * cs] = svec;
    *(u32x4*)&zbl[fz][16 * cz] = zvec;
    W4G64_STAMP(1);

    // ---- 3. activations into LDS (slot order); bf16 group sums ----
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
        const int it = kThreads16 * u + tid;
        int m, c;
        item_rc(it < total ? it : total - 8 + (tid & 7), m, c);
        *(u32x4*)(xs + m * row_stride + 8 * c) = permute_slots(v[u]);
        if constexpr (XK == kBF16) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                s += __builtin_bit_cast(float, v[u][e] << 16) + __builtin_bit_cast(float, v[u][e] & 0xFFFF0000u);
            s = sum8_lanes16(s);
            sx[m * a.gps + (c >> 3)] = s;
        }
    }
    W4G64_STAMP(2);
    // A barrier over LDS alone: the weight loads stay in flight through it.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    W4G64_STAMP(3);

    // ---- 4. MFMA over the steps: A row = activation row (rows past M read row M - 1) ----
    // this lane's scale bits and zero nibbles of every step (feature row as
    // staged, clamped to N - 1), read from LDS together
    uint32_t sreg[STEPS], zreg[STEPS];
    {
        const int nrowc = min(n, a.N - 1);
        const uint32_t s_run = run_start(nrowc, false), z_run = run_start(nrowc, true);
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int gl = kw + KW * t;
            const uint32_t e_sz = (uint32_t)nrowc * (uint32_t)a.G + (uint32_t)(gl < cnt ? g0 + gl : g0);
            sreg[t] = *(const uint16_t*)&scl[fb * 16 + j][2u * e_sz - s_run];
            const uint32_t zb = zbl[fb * 16 + j][(e_sz >> 1) - z_run];
            zreg[t] = (e_sz & 1) ? zb >> 4 : zb & 0xFu;
        }
    }
    const int mrow = min(j, a.M - 1);
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int gl = kw + KW * t;
        const int glc = min(gl, cnt - 1);
        const uint16_t* src = xs + mrow * row_stride + 64 * glc + 16 * q;
        const u16x8 a0 = *(const u16x8*)src;
        const u16x8 a1 = *(const u16x8*)(src + 8);
        // wait for this step's weight, scale and zero alone; the empty asm keeps
        // their decoding here
        asm volatile("" : "+v"(wq[t]));
        const float sct = (nvalid && gl < cnt) ? half_bits_to_float((uint16_t)sreg[t]) : 0.0f;
        const int zn = (int)zreg[t];
        const int zrt = zn - ((zn & 8) << 1);
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
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0), b0,
                                                        float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1), b1, d, 0, 0, 0);
            // D row 4 q + r = activation row; its group sum over this step's group
            const float corr = 136.0f + (float)zrt;
#pragma unroll
            for (int r = 0; r < 4; ++r) d[r] = fmaf(-corr, sx[min(4 * q + r, a.M - 1) * a.gps + glc], d[r]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(sct, d[r], acc[r]);
    }

    W4G64_STAMP(4);
    // ---- 5. combine the KW waves of each block: D row = 4 q + r, column = j ----
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][4 * q + r][j] = acc[r];
    __syncthreads();
    W4G64_STAMP(5);

    const int col0 = nb * kCols;
    for (int idx = tid; idx < a.M * kCols; idx += kThreads16) {
        const int m = idx / kCols;
        const int c = idx - m * kCols;
        const int nn = col0 + c;
        if (nn >= a.N) continue;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) s += red[w * FB + c / 16][m][c % 16];  // fixed order: deterministic
        if (a.splits == 1)
            store_out<XK>(a.y, (int64_t)m * a.N + nn, s + load_bias(a.bias, a.bias_kind, nn));
        else
            a.partials[((int64_t)split * a.M + m) * a.N + nn] = s;
    }
    W4G64_STAMP(6);
    W4G64_TIMELINE_STORE(a);
}

template <int XK, int STEPS, int KW, int FB>
hipError_t launch16(const Gemv16Args& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                    hipEvent_t stop) {
    // the staging capacity of this instantiation (the planner never exceeds it)
    if ((int64_t)args.M * args.gps * 8 > (int64_t)stage_items16<STEPS, FB>() * KW * FB * 64 || args.gps > KW * STEPS)
        return hipErrorInvalidValue;
    const bool split = plan.splits > 1;
    const hipError_t err = launch_kernel(gemv16_kernel<XK, STEPS, KW, FB>, dim3(plan.n_blocks, plan.splits),
                                         dim3(KW * FB * 64), (size_t)plan.lds_bytes, stream, start,
                                         split ? nullptr : stop, args);
    if (err != hipSuccess || !split) return err;
    return launch_split_reduce(args.partials, args.bias, args.bias_kind, args.y, args.M, args.N, args.splits, false,
                               XK, stream, stop);
}

template <int XK, int KW, int FB>
hipError_t launch_steps16(const Gemv16Args& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                          hipEvent_t stop) {
    switch (plan.steps) {
        case 2: return launch16<XK, 2, KW, FB>(args, plan, stream, start, stop);
        case 3: return launch16<XK, 3, KW, FB>(args, plan, stream, start, stop);
        case 6: return launch16<XK, 6, KW, FB>(args, plan, stream, start, stop);
        case 9: return launch16<XK, 9, KW, FB>(args, plan, stream, start, stop);
        case 12: return launch16<XK, 12, KW, FB>(args, plan, stream, start, stop);
        default: return launch16<XK, 18, KW, FB>(args, plan, stream, start, stop);
    }
}

template <int XK>
hipError_t launch_shape16(const Gemv16Args& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                          hipEvent_t stop) {
    // (KW, FB) pairs the planner produces
    if (plan.fblocks == 1 && plan.waves == 4) return launch_steps16<XK, 4, 1>(args, plan, stream, start, stop);
    if (plan.fblocks == 1 && plan.waves == 8) return launch_steps16<XK, 8, 1>(args, plan, stream, start, stop);
    if (plan.fblocks == 2 && plan.waves == 2) return launch_steps16<XK, 2, 2>(args, plan, stream, start, stop);
    if (plan.fblocks == 2 && plan.waves == 4) return launch_steps16<XK, 4, 2>(args, plan, stream, start, stop);
    if (plan.fblocks == 3 && plan.waves == 4) return launch_steps16<XK, 4, 3>(args, plan, stream, start, stop);
    if (plan.fblocks == 4 && plan.waves == 1) return launch_steps16<XK, 1, 4>(args, plan, stream, start, stop);
    if (plan.fblocks == 4 && plan.waves == 2) return launch_steps16<XK, 2, 4>(args, plan, stream, start, stop);
    return hipErrorInvalidValue;
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
    args.partials = (float*)workspace;
    W4G64_TIMELINE_SET(args);
    if (p.x_kind == kF16) return launch_shape16<kF16>(args, plan, stream, start, stop);
    return launch_shape16<kBF16>(args, plan, stream, start, stop);
}

}  // namespace w4g64
