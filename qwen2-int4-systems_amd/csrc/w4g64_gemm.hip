// Prefill path: W4G64 GEMM on MFMA for more than 16 activation rows.
//
// y[M, N] = x[M, K] @ W^T (+ bias), W[n,k] = (code - zero) * scale.
// One workgroup computes a BM x BN output tile; the K loop walks the 64-wide
// quantization groups (BK = 64 = one group, so each weight row has a single
// scale and zero per K step).  Per step:
//   * the activation tile (BM x 64) is copied to LDS in MFMA slot order
//     ([k0 k4 k1 k5 k2 k6 k3 k7] within each 8-block); fp32 activations are
//     split into two bf16 parts (hi + lo, 16 significant bits) that form two
//     A operands;
//   * the packed weight tile (BN x 32 bytes) is read once, dequantized with
//     the scale folded in -- fp16: RNE((code - zero) * scale) in fp16, bf16:
//     RNE((code - zero) * scale) from the exact fp32 product -- and written
//     to LDS in the same slot order;
//   * 4 waves (2 x 2) each run 2 x 2 v_mfma_f32_32x32x16 blocks per 16-wide
//     K sub-step, accumulating in fp32.
// Tiles are double buffered: the global loads of step g+1 are issued before
// the MFMAs of step g and written to the other LDS buffer afterwards.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int LDK = 64 + 8;  // 16-bit elements per LDS row (+16 B pad)

struct GemmArgs {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;
    void* y;
    int M;
    int N;
    int K;
    int G;
};

// Register-staged global data of one K step for one thread.
template <int XK>
struct Stage {
    static constexpr int kParts = (XK == kF32) ? 2 : 1;
    u32x4 a[4][kParts];  // 4 activation items (8 values each) per thread, slot order
    u32x4 w;             // 16 packed bytes (32 weights)
    float s;
    int z;
};

template <int XK>
__device__ __forceinline__ void load_stage(const GemmArgs& a, int g, int64_t m0, int64_t n0, int tid,
                                           Stage<XK>& st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int it = tid + 256 * i;  // BM * 8 = 1024 items
        const int r = it >> 3;
        const int c = it & 7;
        const int64_t m = m0 + r;
        if (m < a.M) {
            if constexpr (XK != kF32) {
                st.a[i][0] = *(const u32x4*)((const uint16_t*)a.x + m * a.K + (int64_t)g * 64 + 8 * c);
            } else {
                const float* src = (const float*)a.x + m * a.K + (int64_t)g * 64 + 8 * c;
                const float4v f0 = *(const float4v*)src;
                const float4v f1 = *(const float4v*)(src + 4);
                uint16_t hi[8], lo[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) split2_bf16(j < 4 ? f0[j] : f1[j - 4], hi[j], lo[j]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    st.a[i][0][j] = (uint32_t)hi[2 * j] | ((uint32_t)hi[2 * j + 1] << 16);
                    st.a[i][1][j] = (uint32_t)lo[2 * j] | ((uint32_t)lo[2 * j + 1] << 16);
                }
            }
        } else {
#pragma unroll
            for (int p = 0; p < Stage<XK>::kParts; ++p) st.a[i][p] = u32x4{0u, 0u, 0u, 0u};
        }
    }
    const int r = tid >> 1;
    const int h = tid & 1;
    const int64_t n = n0 + r;
    if (n < a.N) {
        st.w = *(const u32x4*)(a.qweight + n * (a.K / 2) + (int64_t)g * 32 + 16 * h);
        st.s = half_bits_to_float(a.scales[n * a.G + g]);
        st.z = nibble_at(a.zeros, n * a.G + g);
    } else {
        st.w = u32x4{0u, 0u, 0u, 0u};
        st.s = 0.0f;
        st.z = 0;
    }
}

template <int XK>
__device__ __forceinline__ void store_stage(const Stage<XK>& st, uint16_t* As, uint16_t* Bs, int tid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int it = tid + 256 * i;
        const int r = it >> 3;
        const int c = it & 7;
#pragma unroll
        for (int p = 0; p < Stage<XK>::kParts; ++p)
            *(u32x4*)(As + p * BM * LDK + r * LDK + 8 * c) = permute_slots(st.a[i][p]);
    }
    const int r = tid >> 1;
    const int h = tid & 1;
    const _Float16 zl = (_Float16)(1032 + st.z);
    const _Float16 zh = (_Float16)(72 + st.z);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const half8 ints = dequant8_f16_int(st.w[j], half2v{zl, zl}, half2v{zh, zh});
        u32x4 out;
        if constexpr (XK == kF16) {
            const _Float16 s16 = (_Float16)st.s;  // exact: the stored fp16 scale
            const half8 v = ints * half8{s16, s16, s16, s16, s16, s16, s16, s16};
            out = __builtin_bit_cast(u32x4, v);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = (float)ints[2 * e] * st.s;      // exact in fp32
                const float hi = (float)ints[2 * e + 1] * st.s;
                out[e] = (uint32_t)float_to_bf16_bits(lo) | ((uint32_t)float_to_bf16_bits(hi) << 16);
            }
        }
        *(u32x4*)(Bs + r * LDK + 32 * h + 8 * j) = out;
    }
}

template <int XK>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a) {
    constexpr int kParts = Stage<XK>::kParts;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][kParts * BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;
    const int64_t m0 = (int64_t)blockIdx.y * BM;
    const int64_t n0 = (int64_t)blockIdx.x * BN;

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = float16v{};

    Stage<XK> st;
    load_stage<XK>(a, 0, m0, n0, tid, st);
    store_stage<XK>(st, As[0], Bs[0], tid);
    __syncthreads();

    const int i32 = lane & 31;
    const int q = lane >> 5;
    for (int g = 0; g < a.G; ++g) {
        const int buf = g & 1;
        const bool more = g + 1 < a.G;
        if (more) load_stage<XK>(a, g + 1, m0, n0, tid, st);
        const uint16_t* Ab = As[buf];
        const uint16_t* Bb = Bs[buf];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            half8 bfr[2];
#pragma unroll
            for (int bj = 0; bj < 2; ++bj)
                bfr[bj] = *(const half8*)(Bb + (wn + 32 * bj + i32) * LDK + 16 * kk + 8 * q);
#pragma unroll
            for (int p = 0; p < kParts; ++p) {
#pragma unroll
                for (int bi = 0; bi < 2; ++bi) {
                    const half8 afr = *(const half8*)(Ab + p * BM * LDK + (wm + 32 * bi + i32) * LDK + 16 * kk + 8 * q);
#pragma unroll
                    for (int bj = 0; bj < 2; ++bj) {
                        if constexpr (XK == kF16) {
                            acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr, bfr[bj], acc[bi][bj], 0, 0, 0);
                        } else {
                            acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                __builtin_bit_cast(bf16x8, afr), __builtin_bit_cast(bf16x8, bfr[bj]), acc[bi][bj], 0,
                                0, 0);
                        }
                    }
                }
            }
        }
        if (more) store_stage<XK>(st, As[buf ^ 1], Bs[buf ^ 1], tid);
        __syncthreads();
    }

    // Epilogue.  32x32 accumulator layout: column = lane % 32,
    // row = 8 * (r / 4) + 4 * (lane / 32) + r % 4 for register r.
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            const int64_t n = n0 + wn + 32 * bj + i32;
            if (n >= a.N) continue;
            const float b = load_bias(a.bias, a.bias_kind, n);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t m = m0 + wm + 32 * bi + 8 * (r / 4) + 4 * q + (r % 4);
                if (m < a.M) store_out<XK>(a.y, m * a.N + n, acc[bi][bj][r] + b);
            }
        }
    }
}

}  // namespace

hipError_t launch_gemm(const LinearProblem& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    GemmArgs args{};
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
    dim3 grid((unsigned)((p.out_features + BN - 1) / BN), (unsigned)((p.rows + BM - 1) / BM));
    switch (p.x_kind) {
        case kF16:
            return launch_kernel(gemm_kernel<kF16>, grid, dim3(256), 0, stream, start, stop, args);
        case kBF16:
            return launch_kernel(gemm_kernel<kBF16>, grid, dim3(256), 0, stream, start, stop, args);
        default:
            return launch_kernel(gemm_kernel<kF32>, grid, dim3(256), 0, stream, start, stop, args);
    }
}

const char* gemm_kernel_name(int64_t, int64_t, int64_t, int x_kind) {
    if (x_kind == kF16) return "gemm2_kernel<f16,128>";
    if (x_kind == kBF16) return "gemm2_kernel<bf16,128>";
    return "gemm_kernel<f32>";
}

}  // namespace w4g64
