// Prefill path v2: pipelined W4G64 GEMM for fp16 / bf16 activations.
//
// y[M, N] = x[M, K] @ W^T (+ bias), W[n,k] = (code - zero) * scale, fp32
// accumulation in v_mfma_f32_32x32x16_{f16,bf16}.
//
// Workgroup = 4 waves, output tile BM x 256: wave w owns all BM rows of the
// 64 output features [n0 + 64 w, n0 + 64 w + 64).  One K step = one 64-wide
// quantization group.
//   * Every load is a gfx950 direct global->LDS load into a ring of S = 3
//     stages, issued S-1 steps ahead: the activation tile (16-byte loads)
//     and, per wave, its packed weight columns, scales and zero bytes.  Every 1 KB a wave instruction writes holds 8 tile rows; the 16 B
//     chunks of a row are XOR-swizzled by (row & 7), which the fragment reads
//     undo, so the 32 rows of a fragment read hit distinct banks.
//   * Weights (B): each wave reads back its own packed columns (16 B = 32
//     consecutive K values per lane and column block) and dequantizes only
//     its own columns:
//     (code - zero) built exactly in fp16 with the magic-number trick in
//     natural K order (v_perm + v_bitop3), then times the scale: fp16 weights
//     are RNE((code - zero) * scale) in fp16; bf16 weights are
//     RNE(fp32((code - zero) * scale)).
//   * MFMA K slots: lane group q (of 2) takes K values [32q, 32q + 32) of the
//     group, sub-step kk uses [32q + 8kk, 32q + 8kk + 8); A and B fragments
//     use the same slots, so the contraction is unchanged.
//   * Waits are explicit: every step issues the same number of vector memory
//     operations (prefetches past the last step re-load the last step), so
//     "this step's data has landed" is vmcnt <= (S - 2) * ops_per_step.  All
//     loads are drained before the workgroup exits.
//   * Tiles are assigned so that the workgroups of one XCD (ids congruent
//     mod 8) cover consecutive tiles of one row band: they share the
//     activation band in their L2.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kStages = 3;
constexpr int kBN = 256;  // 4 waves x 64 output features
constexpr int kXcds = 8;

struct Gemm2Args {
    const uint16_t* x;
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
    int tiles_m;
    int tiles_n;
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Natural-order fp16 (code - zero) pairs of one packed dword:
// pair b = (k = 2b, k = 2b + 1).  Byte b is replicated by v_perm; the mask
// keeps its low nibble at bits 0-3 (fp16 1024 + n') and its high nibble at
// bits 20-23 (fp16 64 + n' in the upper half); the XOR by 8 and the magic
// exponents are folded into the same bitwise select.
__device__ __forceinline__ uint32_t nib_pair_natural(uint32_t w, int b) {
    const uint32_t rep = __builtin_amdgcn_perm(w, w, 0x01010101u * (uint32_t)b);
    constexpr uint32_t kMask = 0x00F0000Fu;
    constexpr uint32_t kSel = 0x54806408u;  // (mask & 0x88888888) | (~mask & 0x54006400)
    return ((rep ^ kSel) & kMask) | (kSel & ~kMask);
}

template <int XK>
__device__ __forceinline__ u32x4 dequant_natural(uint32_t w, uint32_t zc_bits, float s, uint32_t s2_bits) {
    u32x4 out;
    if constexpr (XK == kF16) {
        const half2v zc = __builtin_bit_cast(half2v, zc_bits);   // (1032 + z, 72 + z)
        const half2v s2 = __builtin_bit_cast(half2v, s2_bits);   // (scale, scale)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half2v v = (__builtin_bit_cast(half2v, nib_pair_natural(w, b)) - zc) * s2;
            out[b] = __builtin_bit_cast(uint32_t, v);
        }
    } else {
        const half2v zc = __builtin_bit_cast(half2v, zc_bits);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half2v d = __builtin_bit_cast(half2v, nib_pair_natural(w, b)) - zc;  // exact ints
            const float lo = (float)d[0] * s;  // exact in fp32
            const float hi = (float)d[1] * s;
            out[b] = (uint32_t)float_to_bf16_bits(lo) | ((uint32_t)float_to_bf16_bits(hi) << 16);
        }
    }
    return out;
}

template <int XK, int BM>
__global__ __launch_bounds__(256) void gemm2_kernel(Gemm2Args a) {
    constexpr int MB = BM / 32;                 // 32-row MFMA blocks per wave
    constexpr int kABytes = BM * 128;           // BM rows x 64 fp16/bf16 values
    constexpr int kWBytes = 4 * 2 * 1024;       // 4 waves x 2 column blocks x (32 columns x 32 B)
    // Sub-dword global->LDS loads write one zero-extended dword per lane.
    constexpr int kSBytes = 4 * 64 * 4;         // one fp16 scale per column (in a dword)
    constexpr int kZBytes = 4 * 64 * 4;         // the byte holding each column's zero nibble (in a dword)
    constexpr int kStageBytes = kABytes + kWBytes + kSBytes + kZBytes;
    constexpr int kDma = BM / 32;               // 1 KB activation DMA instructions per wave
    constexpr int kOpsPerStep = kDma + 2 + 1 + 1;  // + weight blocks, scales, zeros
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kStages][kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- XCD-aware tile assignment ----
    // Workgroup ids are dealt to the XCDs round robin (id % 8); give XCD x the
    // contiguous tile range [start_x, start_x + count_x) -- a bijection.
    const int tiles = a.tiles_m * a.tiles_n;
    const int bid = blockIdx.x;
    const int xcd = bid % kXcds;
    const int base = tiles / kXcds;
    const int extra = tiles % kXcds;
    const int t = xcd * base + (xcd < extra ? xcd : extra) + bid / kXcds;
    const int tile_m = t / a.tiles_n;
    const int tile_n = t - tile_m * a.tiles_n;
    const int64_t m0 = (int64_t)tile_m * BM;
    const int64_t nw = (int64_t)tile_n * kBN + 64 * wave;  // this wave's first output feature

    // ---- per-lane DMA sources ----
    // activations: instruction d writes tile rows [8 (wave kDma + d), +8), 16 B per lane
    const uint16_t* a_src[kDma];
#pragma unroll
    for (int d = 0; d < kDma; ++d) {
        const int r = 8 * (wave * kDma + d) + (lane >> 3);
        const int chunk = (lane & 7) ^ (r & 7);
        int64_t m = m0 + r;
        m = m < a.M ? m : a.M - 1;  // rows past M load a valid row; their outputs are not stored
        a_src[d] = a.x + m * a.K + 8 * chunk;
    }
    // weights: block bj, lane (j = lane % 32, q = lane / 32) -> column nw + 32 bj + j, bytes [16q, 16q + 16)
    const int j = lane & 31;
    const int q = lane >> 5;
    const uint8_t* w_src[2];
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        int64_t n = nw + 32 * bj + j;
        n = n < a.N ? n : a.N - 1;
        w_src[bj] = a.qweight + n * (a.K / 2) + 16 * q;
    }
    // scale / zero of column nw + lane
    int64_t ncol = nw + lane;
    ncol = ncol < a.N ? ncol : a.N - 1;
    const int64_t s_row = ncol * a.G;

    auto issue = [&](int g) {
        const int gg = g < a.G ? g : a.G - 1;  // past the end: re-load the last step (uniform op count)
        unsigned char* st = smem[g % kStages];
#pragma unroll
        for (int d = 0; d < kDma; ++d)
            __builtin_amdgcn_global_load_lds((const void*)(a_src[d] + (int64_t)gg * 64),
                                             (lds_ptr_t)(st + 1024 * (wave * kDma + d)), 16, 0, 0);
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
            __builtin_amdgcn_global_load_lds((const void*)(w_src[bj] + (int64_t)gg * 32),
                                             (lds_ptr_t)(st + kABytes + 2048 * wave + 1024 * bj), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(a.scales + s_row + gg),
                                         (lds_ptr_t)(st + kABytes + kWBytes + 256 * wave), 2, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(a.zeros + ((s_row + gg) >> 1)),
                                         (lds_ptr_t)(st + kABytes + kWBytes + kSBytes + 256 * wave), 1, 0, 0);
    };

    float16v acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) acc[i][bj] = float16v{};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(s);

    const int fr = lane & 31;
    constexpr int kWait = kOpsPerStep * (kStages - 2);  // loads issued after this step's
    static_assert(kWait < 64, "vmcnt is 6 bits");
    constexpr int kWaitImm = (kWait & 0xF) | ((kWait >> 4) << 14) | (0x7 << 4) | (0xF << 8);

    for (int g = 0; g < a.G; ++g) {
        // This wave's loads for step g have landed (loads complete in order and
        // kWait loads were issued after them); the barrier extends that to all
        // waves and guarantees nobody still reads the stage refilled below
        // (every wave consumed its LDS reads of step g-1 in that step's MFMAs).
        // A bare s_barrier: __syncthreads() would add a release fence that
        // drains the prefetches still in flight.
        __builtin_amdgcn_s_waitcnt(kWaitImm);
        __builtin_amdgcn_s_barrier();
        issue(g + kStages - 1);

        const unsigned char* st = smem[g % kStages];
        // ---- dequantize this wave's B fragments ----
        u32x4 bfrag[2][4];
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            const u32x4 w = *(const u32x4*)(st + kABytes + 2048 * wave + 1024 * bj + 16 * lane);
            const int c = 32 * bj + j;  // column within the wave
            const uint16_t sbits = *(const uint16_t*)(st + kABytes + kWBytes + 256 * wave + 4 * c);
            const int zb = st[kABytes + kWBytes + kSBytes + 256 * wave + 4 * c];
            const int64_t e = (nw + c < a.N ? nw + c : a.N - 1) * a.G + g;
            int zn = (e & 1) ? (zb >> 4) : (zb & 0xF);
            zn -= (zn & 8) << 1;
            const uint32_t zlo = 0x6408u + (uint32_t)zn;       // fp16 bits of 1032 + z
            const uint32_t zhi = 0x5480u + 16u * (uint32_t)zn;  // fp16 bits of 72 + z
            const uint32_t zc = (zlo & 0xFFFFu) | ((zhi & 0xFFFFu) << 16);
            const float s = half_bits_to_float(sbits);
            const uint32_t s2 = (uint32_t)sbits * 0x00010001u;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) bfrag[bj][kk] = dequant_natural<XK>(w[kk], zc, s, s2);
        }
        // ---- MFMA: A fragments from the swizzled stage ----
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int bi = 0; bi < MB; ++bi) {
                const int r = 32 * bi + fr;
                const int chunk = (4 * q + kk) ^ (r & 7);
                const u32x4 afr = *(const u32x4*)(st + r * 128 + chunk * 16);
#pragma unroll
                for (int bj = 0; bj < 2; ++bj) {
                    if constexpr (XK == kF16) {
                        acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(half8, afr), __builtin_bit_cast(half8, bfrag[bj][kk]), acc[bi][bj],
                            0, 0, 0);
                    } else {
                        acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, afr), __builtin_bit_cast(bf16x8, bfrag[bj][kk]),
                            acc[bi][bj], 0, 0, 0);
                    }
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // no DMA may still target this workgroup's LDS at exit

    // ---- epilogue: 32x32 accumulator layout: column = lane % 32,
    // row = 8 (r / 4) + 4 (lane / 32) + r % 4 ----
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        const int64_t n = nw + 32 * bj + j;
        if (n >= a.N) continue;
        const float b = load_bias(a.bias, a.bias_kind, n);
#pragma unroll
        for (int bi = 0; bi < MB; ++bi) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t m = m0 + 32 * bi + 8 * (r / 4) + 4 * q + (r % 4);
                if (m < a.M) store_out<XK>(a.y, m * a.N + n, acc[bi][bj][r] + b);
            }
        }
    }
}

}  // namespace

bool gemm2_supported(const LinearProblem& p) {
    return (p.x_kind == kF16 || p.x_kind == kBF16);
}

hipError_t launch_gemm2(const LinearProblem& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    Gemm2Args args{};
    args.x = (const uint16_t*)p.x;
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
    const bool big = p.rows > 128;
    const int bm = big ? 256 : 128;
    args.tiles_m = (int)((p.rows + bm - 1) / bm);
    args.tiles_n = (int)((p.out_features + kBN - 1) / kBN);
    dim3 grid((unsigned)(args.tiles_m * args.tiles_n));
    if (p.x_kind == kF16) {
        return big ? launch_kernel(gemm2_kernel<kF16, 256>, grid, dim3(256), 0, stream, start, stop, args)
                   : launch_kernel(gemm2_kernel<kF16, 128>, grid, dim3(256), 0, stream, start, stop, args);
    }
    return big ? launch_kernel(gemm2_kernel<kBF16, 256>, grid, dim3(256), 0, stream, start, stop, args)
               : launch_kernel(gemm2_kernel<kBF16, 128>, grid, dim3(256), 0, stream, start, stop, args);
}

}  // namespace w4g64
