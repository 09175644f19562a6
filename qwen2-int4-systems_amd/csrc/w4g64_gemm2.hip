// Prefill path v2: pipelined W4G64 GEMM for fp16 / bf16 activations.
//
// y[M, N] = x[M, K] @ W^T (+ bias), W[n,k] = (code - zero) * scale, fp32
// accumulation in v_mfma_f32_32x32x16_{f16,bf16}.
//
// Workgroup = 4 waves, output tile BM x 256 (BM = 128): wave w owns all BM
// rows of the 64 output features [n0 + 64 w, n0 + 64 w + 64).  One K step =
// one 64-wide quantization group.  Two workgroups share a CU (78 KB of LDS
// and 256 registers per lane each), so the MFMA pipes stay busy while one of
// them waits at its per-step barrier.
//   * Every load is a gfx950 direct global->LDS load into a ring of S = 3
//     stages, issued up to S steps ahead (a stage is refilled as soon as
//     every wave has finished reading it): the activation tile (16-byte loads)
//     and, per wave, its packed weight columns, scales and zero bytes.
//     Every 1 KB a wave instruction writes holds 8 tile rows; the 16 B
//     chunks of a row are XOR-swizzled by a_swizzle(row), which the fragment
//     reads undo: any 8 or 16 consecutive rows of one logical chunk land in
//     distinct 16-byte bank groups, so fragment reads are conflict-free.
//   * Weights (B): each wave reads back its own packed columns (16 B = 32
//     consecutive K values per lane and column block) and dequantizes only
//     its own columns, one MFMA sub-step ahead of their use, into exact
//     weights: w = (code - zero) * scale has at most 15 significant bits, so
//     it is exact in fp32, and it is split into hi = RNE(w) in the MFMA type
//     and lo = w - hi, which that type also holds exactly (bf16: at most 8
//     bits remain; fp16: lo is a multiple of the scale's last bit, itself a
//     multiple of 2^-24, with at most 5 significant bits).  Every B fragment
//     is multiplied twice, x * hi + x * lo == x * w: the products are those
//     of the exact fp32 weights, as in a dequantize-then-fp32-matmul, and
//     only the fp32 accumulation order differs.  (fp16 weights with |w| >
//     65504 overflow hi; fp16 outputs of such a product would overflow too.)
//   * MFMA K slots: lane group q (of 2) takes K values [32q, 32q + 32) of the
//     group, sub-step kk uses [32q + 8kk, 32q + 8kk + 8); A and B fragments
//     use the same slots, so the contraction is unchanged.
//   * Waits are explicit: every step issues the same number of vector memory
//     operations, so "step s has landed" is a vmcnt bound known at compile
//     time for each position in the loop (steps past the end are not issued;
//     the waits near the end tighten accordingly).  All loads are drained
//     before the workgroup exits.
//   * Tiles are assigned so that the workgroups of one XCD (ids congruent
//     mod 8) cover consecutive tiles of one row band: they share the
//     activation band in their L2.
//   * fp32 activations: a first kernel splits each row into two bf16 planes,
//     hi = RNE(x) and lo = RNE(x - hi) (16 significant bits, |x - hi - lo| <=
//     2^-17 |x|), laid out as one row [hi | lo] of 2K values in the
//     workspace; the GEMM then runs over K' = 2K with weight group g mod G,
//     so both planes meet the same exact weights, and stores fp32 outputs.
#include <type_traits>

#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kStages = 3;
constexpr int kBN = 256;  // 4 waves x 64 output features
constexpr int kBM = 128;  // rows per tile: two workgroups fit one CU (LDS and registers)
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
    int K;   // activation row length (2 in_features for fp32 activations)
    int G;   // activation groups, K / 64
    int wg;  // weight groups (in_features / 64): the K' step g reads weight group g mod wg
    int tiles_m;
    int tiles_n;
    int vec_out;    // y is 16-byte aligned and N % 8 == 0: 16-byte output stores
    int dp_tiles;   // tiles [0, dp_tiles): one workgroup each over the whole K range
    int splits;     // tiles [dp_tiles, tiles): `splits` workgroups each, one K range apiece
    int gps;        // groups per K range of a split tile
    float* partials;  // [(tile - dp_tiles) * splits + piece][BM][kBN] fp32
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt with only the vector memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
// Physical 16-byte chunk offset of tile row r (rows are 128 B = 8 chunks).
// Row r's chunks start at bank group 8 (r & 1) (mod 16 groups of 4 banks);
// the XOR term takes 8 distinct values over any 8 consecutive rows and over
// the 8 rows of either parity among 16 consecutive rows.
__device__ __forceinline__ int a_swizzle(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// Scheduling shape of one sub-step: each of the MB A-fragment reads is
// followed by 2 P MFMAs, with up to V other VALU instructions after each
// MFMA, and no instruction crosses the end of the sub-step.
template <int MB, int P, int V>
__device__ __forceinline__ void sched_interleave() {
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
        for (int p = 0; p < 2 * P; ++p) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            if constexpr (V > 0) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);  // VALU
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }
// Workgroup execution barrier without a memory fence (a fence would drain the
// loads still in flight); the empty asm statements keep the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

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

// Per-group constants of one column's dequantization.
struct BConst {
    uint32_t zc;  // fp16: bits of (1032 + z, 72 + z)
    uint32_t s2;  // fp16: bits of (scale, scale)
    float s;      // bf16: the scale
    float cs_lo;  // bf16: (1032 + z) * scale, exact (11-bit by 11-bit product)
    float cs_hi;  // bf16: (72 + z) * scale, exact
};

// Exact weights of one packed dword (8 consecutive K values of one column)
// as the hi and lo B fragments (4 natural-order pairs each).
//   fp16: d = (m - c) is exact in fp16 (m = magic value, c = magic offset +
//         zero); hi = RNE(d * scale) by one packed fp16 multiply; lo = d *
//         scale - hi by an fp32 FMA of the fp16 operands (exact product,
//         exact difference), exact in fp16.
//   bf16: w = d * s = m * s - c * s, and both products fit in 22 bits, so
//         one fp32 FMA against the precomputed exact c * s yields w exactly;
//         hi = RNE(w) in bf16 and lo = RNE(w - hi) = w - hi.
template <int XK>
__device__ __forceinline__ void dequant_hl(uint32_t w, const BConst& c, u32x4& hi, u32x4& lo) {
    if constexpr (XK == kF16) {
        const half2v zc = __builtin_bit_cast(half2v, c.zc);
        const half2v s2 = __builtin_bit_cast(half2v, c.s2);
        const float s = (float)s2[0];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half2v d = __builtin_bit_cast(half2v, nib_pair_natural(w, b)) - zc;
            const half2v h = d * s2;
            const half2v l = {(_Float16)__builtin_fmaf((float)d[0], s, -(float)h[0]),
                              (_Float16)__builtin_fmaf((float)d[1], s, -(float)h[1])};
            hi[b] = __builtin_bit_cast(uint32_t, h);
            lo[b] = __builtin_bit_cast(uint32_t, l);
        }
    } else {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const half2v m = __builtin_bit_cast(half2v, nib_pair_natural(w, b));  // (1024 + n', 64 + n')
            const float w0 = __builtin_fmaf((float)m[0], c.s, -c.cs_lo);
            const float w1 = __builtin_fmaf((float)m[1], c.s, -c.cs_hi);
            const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{w0, w1}, bf16x2v));
            const float h0 = __builtin_bit_cast(float, hb << 16);
            const float h1 = __builtin_bit_cast(float, hb & 0xFFFF0000u);
            hi[b] = hb;
            lo[b] = __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{w0 - h0, w1 - h1}, bf16x2v));
        }
    }
}

template <int XK, int BM, int OUTK>
__global__ __launch_bounds__(256, 2) void gemm2_kernel(Gemm2Args a) {
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

    // ---- tile and K range of this workgroup ----
    // Data-parallel tiles: workgroup ids are dealt to the XCDs round robin
    // (id % 8); XCD x gets the contiguous tile range [start_x, start_x +
    // count_x) -- a bijection on [0, dp_tiles) -- so an XCD's workgroups share
    // activation row bands in their L2.  Split tiles follow: `splits`
    // consecutive workgroups per tile, each over its own K range, writing fp32
    // partial sums that a second kernel adds up in range order.
    const int bid = blockIdx.x;
    int t, gbeg, gcnt, slot = -1;
    if (bid < a.dp_tiles) {
        const int xcd = bid % kXcds;
        const int base = a.dp_tiles / kXcds;
        const int extra = a.dp_tiles % kXcds;
        t = xcd * base + (xcd < extra ? xcd : extra) + bid / kXcds;
        gbeg = 0;
        gcnt = a.G;
    } else {
        slot = bid - a.dp_tiles;
        t = a.dp_tiles + slot / a.splits;
        gbeg = (slot % a.splits) * a.gps;
        gcnt = min(a.gps, a.G - gbeg);
    }
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
        const int chunk = (lane & 7) ^ a_swizzle(r);
        int64_t m = m0 + r;
        m = m < a.M ? m : a.M - 1;  // rows past M load a valid row; their outputs are not stored
        a_src[d] = a.x + m * a.K + (int64_t)gbeg * 64 + 8 * chunk;
    }
    // weights: block bj, lane (j = lane % 32, q = lane / 32) -> column nw + 32 bj + j, bytes [16q, 16q + 16)
    const int j = lane & 31;
    const int q = lane >> 5;
    const uint8_t* w_src[2];
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        int64_t n = nw + 32 * bj + j;
        n = n < a.N ? n : a.N - 1;
        w_src[bj] = a.qweight + n * ((int64_t)a.wg * 32) + 16 * q;
    }
    // scale / zero of column nw + lane
    int64_t ncol = nw + lane;
    ncol = ncol < a.N ? ncol : a.N - 1;
    const int64_t s_row = ncol * a.wg;  // scale / zero element of weight group 0
    // weight group of this workgroup's K step gg (one wrap at most: K' <= 2 in_features)
    auto wgroup = [&](int gg) {
        const int gabs = gbeg + gg;
        return gabs >= a.wg ? gabs - a.wg : gabs;
    };

    auto issue = [&](int gg) {  // callers pass gg < G only
        unsigned char* st = smem[gg % kStages];
        const int gw = wgroup(gg);
#pragma unroll
        for (int d = 0; d < kDma; ++d)
            __builtin_amdgcn_global_load_lds((const void*)(a_src[d] + (int64_t)gg * 64),
                                             (lds_ptr_t)(st + 1024 * (wave * kDma + d)), 16, 0, 0);
#pragma unroll
        for (int bj = 0; bj < 2; ++bj)
            __builtin_amdgcn_global_load_lds((const void*)(w_src[bj] + (int64_t)gw * 32),
                                             (lds_ptr_t)(st + kABytes + 2048 * wave + 1024 * bj), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(a.scales + s_row + gw),
                                         (lds_ptr_t)(st + kABytes + kWBytes + 256 * wave), 2, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(a.zeros + ((s_row + gw) >> 1)),
                                         (lds_ptr_t)(st + kABytes + kWBytes + kSBytes + 256 * wave), 1, 0, 0);
    };

    float16v acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) acc[i][bj] = float16v{};

    // parity of each of this lane's two dequant columns' zero element index at weight group 0
    int zpar[2];
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        const int64_t n = nw + 32 * bj + j;
        zpar[bj] = (int)(((n < a.N ? n : a.N - 1) * a.wg) & 1);
    }

    // Packed weights of step g, column block bj, read back from the stage:
    // dword kk holds K values [32q + 8kk, +8) of column nw + 32 bj + j.
    struct BRaw {
        u32x4 w;
        uint32_t sbits;
        uint32_t zb;
    };
    auto read_b = [&](int g, int bj) {
        const unsigned char* st = smem[g % kStages];
        const int c = 32 * bj + j;  // column within the wave
        BRaw r;
        r.w = *(const u32x4*)(st + kABytes + 2048 * wave + 1024 * bj + 16 * lane);
        r.sbits = *(const uint16_t*)(st + kABytes + kWBytes + 256 * wave + 4 * c);
        r.zb = st[kABytes + kWBytes + kSBytes + 256 * wave + 4 * c];
        return r;
    };
    auto group_const = [&](int g, int bj, const BRaw& r) {
        int zn = (int)(((zpar[bj] ^ wgroup(g)) & 1) ? (r.zb >> 4) : (r.zb & 0xF));
        zn -= (zn & 8) << 1;
        BConst c;
        const uint32_t zlo = 0x6408u + (uint32_t)zn;       // fp16 bits of 1032 + z
        const uint32_t zhi = 0x5480u + 16u * (uint32_t)zn;  // fp16 bits of 72 + z
        c.zc = (zlo & 0xFFFFu) | ((zhi & 0xFFFFu) << 16);
        c.s2 = (r.sbits & 0xFFFFu) * 0x00010001u;
        c.s = half_bits_to_float((uint16_t)r.sbits);
        c.cs_lo = (float)(1032 + zn) * c.s;
        c.cs_hi = (float)(72 + zn) * c.s;
        return c;
    };
    // A fragments of sub-step kk from the swizzled stage.
    const int fr = lane & 31;
    auto read_a = [&](const unsigned char* st, int kk, u32x4 (&af)[MB]) {
#pragma unroll
        for (int bi = 0; bi < MB; ++bi) {
            const int r = 32 * bi + fr;
            const int chunk = (4 * q + kk) ^ a_swizzle(r);
            af[bi] = *(const u32x4*)(st + r * 128 + chunk * 16);
        }
    };
    // B fragments of one sub-step: [column block][hi, lo]
    struct BFrag {
        u32x4 v[2][2];
    };
    auto dequant = [&](const u32x4 (&w)[2], const BConst (&c)[2], int kk) {
        BFrag f;
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) dequant_hl<XK>(w[bj][kk], c[bj], f.v[bj][0], f.v[bj][1]);
        return f;
    };
    // every hi product, then every lo product: 2 MB independent MFMAs
    // separate the two that update one accumulator
    auto mma = [&](const u32x4 (&af)[MB], const BFrag& bf) {
#pragma unroll
        for (int hl = 0; hl < 2; ++hl)
#pragma unroll
            for (int bi = 0; bi < MB; ++bi)
#pragma unroll
                for (int bj = 0; bj < 2; ++bj) {
                    if constexpr (XK == kF16) {
                        acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(half8, af[bi]), __builtin_bit_cast(half8, bf.v[bj][hl]), acc[bi][bj],
                            0, 0, 0);
                    } else {
                        acc[bi][bj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, af[bi]), __builtin_bit_cast(bf16x8, bf.v[bj][hl]),
                            acc[bi][bj], 0, 0, 0);
                    }
                }
    };
    constexpr int kV = XK == kF16 ? 4 : 6;  // dequant VALU instructions placed after each MFMA

    // ---- rotated software pipeline ----
    // Step g, four sub-steps of 4 MB MFMAs each (hi and lo weights):
    //   kk = 0: read this wave's packed B data of step g + 1 and the A
    //           fragments of kk = 1; dequantize B of step g, kk = 1;
    //   kk = 1: read the A fragments of kk = 2; dequantize B of kk = 2;
    //   kk = 2: read the A fragments of kk = 3; dequantize B of kk = 3 and
    //           form step g + 1's scale and zero constants;
    //   kk = 3: workgroup barrier (every wave has finished reading stage g and
    //           all of step g + 1 has landed), refill stage g with step g + 3,
    //           read the A fragments of step g + 1, kk = 0, and dequantize
    //           its B of kk = 0.
    // "Step s has landed" for this wave = its vector memory counter is at most
    // the number of operations issued after step s's (in-order completion).
    // Steps g + 3 < G run the branch-free body; the last (up to) three steps
    // the same body with the tighter waits and without refills.
    const int G = gcnt;  // steps of this workgroup's K range
    issue(0);
    if (G > 1) issue(1);
    if (G > 2) issue(2);
    if (G > 2) wait_vmcnt<2 * kOpsPerStep>();
    else if (G > 1) wait_vmcnt<kOpsPerStep>();
    else wait_vmcnt<0>();
    block_barrier();

    u32x4 wcur[2];
    BConst ccur[2];
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        const BRaw r = read_b(0, bj);
        wcur[bj] = r.w;
        ccur[bj] = group_const(0, bj, r);
    }
    BFrag bcur = dequant(wcur, ccur, 0);
    u32x4 a0[MB], a1[MB];
    read_a(smem[0], 0, a0);

    auto step = [&](int g, auto tail_tag) {
        constexpr bool kTail = decltype(tail_tag)::value;
        const unsigned char* st = smem[g % kStages];
        const int gn = (kTail && g + 1 >= G) ? g : g + 1;  // last step: re-read its own (valid) stage
        // ---- kk = 0 ----
        if constexpr (kTail) wait_vmcnt<0>();
        else wait_vmcnt<kOpsPerStep>();  // this wave's loads of step g + 1
        const BRaw rn0 = read_b(gn, 0);
        const BRaw rn1 = read_b(gn, 1);
        read_a(st, 1, a1);
        const BFrag b1 = dequant(wcur, ccur, 1);
        mma(a0, bcur);
        sched_interleave<MB, 2, kV>();
        // ---- kk = 1 ----
        read_a(st, 2, a0);
        const BFrag b2 = dequant(wcur, ccur, 2);
        mma(a1, b1);
        sched_interleave<MB, 2, kV>();
        // ---- kk = 2 ----
        read_a(st, 3, a1);
        const BFrag b3 = dequant(wcur, ccur, 3);
        const u32x4 wnext[2] = {rn0.w, rn1.w};
        const BConst cnext[2] = {group_const(gn, 0, rn0), group_const(gn, 1, rn1)};
        mma(a0, b2);
        sched_interleave<MB, 2, kV>();
        // ---- kk = 3 ----
        if (!kTail || g + 1 < G) {
            wait_lgkmcnt0();
            block_barrier();
            if (!kTail) issue(g + 3);
        }
        read_a(smem[(g + 1) % kStages], 0, a0);
        bcur = dequant(wnext, cnext, 0);
        mma(a1, b3);
        sched_interleave<MB, 2, kV>();
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            wcur[bj] = wnext[bj];
            ccur[bj] = cnext[bj];
        }
    };
    int g = 0;
    for (; g + 3 < G; ++g) step(g, std::false_type{});
    for (; g < G; ++g) step(g, std::true_type{});
    wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS at exit

    // ---- split tile: fp32 partial sums, added up by gemm2_reduce_kernel ----
    // 32x32 accumulator layout (below); a store instruction writes two full
    // 128-byte row segments.
    if (slot >= 0) {
        float* part = a.partials + (int64_t)slot * (BM * kBN) + 64 * wave + j;
#pragma unroll
        for (int bi = 0; bi < MB; ++bi)
#pragma unroll
            for (int bj = 0; bj < 2; ++bj)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    part[(32 * bi + 8 * (r / 4) + 4 * q + (r % 4)) * kBN + 32 * bj] = acc[bi][bj][r];
        return;
    }

    // ---- epilogue ----
    // 32x32 accumulator layout: column = lane % 32, row = 8 (r / 4) +
    // 4 (lane / 32) + r % 4.  Each wave stages its 64 output columns through
    // LDS, half of its rows at a time, and writes 8 consecutive outputs
    // (16 B) per lane: 8 full 128-byte row segments per store instruction.
    // Row stride 144 B: the two lane halves (rows 4 apart) write disjoint
    // banks and the 16-byte reads stay aligned.
    block_barrier();  // every wave has finished reading the pipeline stages
    if constexpr (OUTK == kF32) {
        // fp32 outputs: the same staging with 4-byte values (row stride 272 B)
        // and 16-byte stores of 4 outputs per lane
        constexpr int kOutStride32 = 272;
        constexpr int kHalfRows32 = BM / 2;
        static_assert(4 * kHalfRows32 * kOutStride32 <= kStages * kStageBytes, "output staging exceeds LDS");
        unsigned char* ost = &smem[0][0] + wave * kHalfRows32 * kOutStride32;
        float bias_v[2];
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
            const int64_t n = nw + 32 * bj + j;
            bias_v[bj] = n < a.N ? load_bias(a.bias, a.bias_kind, n) : 0.0f;
        }
        float* y = (float*)a.y;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int bi = 0; bi < MB / 2; ++bi)
#pragma unroll
                for (int bj = 0; bj < 2; ++bj)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = 32 * bi + 8 * (r / 4) + 4 * q + (r % 4);
                        *(float*)(ost + row * kOutStride32 + 4 * (32 * bj + j)) =
                            acc[h * (MB / 2) + bi][bj][r] + bias_v[bj];
                    }
            asm volatile("" ::: "memory");
#pragma unroll
            for (int i = 0; i < kHalfRows32 / 4; ++i) {
                const int row = 4 * i + (lane >> 4);
                const int c4 = lane & 15;
                const u32x4 v = *(const u32x4*)(ost + row * kOutStride32 + 16 * c4);
                const int64_t m = m0 + h * kHalfRows32 + row;
                const int64_t n = nw + 4 * c4;
                if (m < a.M) {
                    if (a.vec_out && n + 4 <= a.N) {
                        *(u32x4*)(y + m * a.N + n) = v;
                    } else {
#pragma unroll 1
                        for (int e = 0; e < 4; ++e)
                            if (n + e < a.N) y[m * a.N + n + e] = __builtin_bit_cast(float, (uint32_t)v[e]);
                    }
                }
            }
            asm volatile("" ::: "memory");
        }
        return;
    }
    constexpr int kOutStride = 144;
    constexpr int kHalfRows = BM / 2;
    static_assert(4 * kHalfRows * kOutStride <= kStages * kStageBytes, "output staging exceeds LDS");
    unsigned char* ost = &smem[0][0] + wave * kHalfRows * kOutStride;
    float bias_v[2];
#pragma unroll
    for (int bj = 0; bj < 2; ++bj) {
        const int64_t n = nw + 32 * bj + j;
        bias_v[bj] = n < a.N ? load_bias(a.bias, a.bias_kind, n) : 0.0f;
    }
    uint16_t* y = (uint16_t*)a.y;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int bi = 0; bi < MB / 2; ++bi) {
#pragma unroll
            for (int bj = 0; bj < 2; ++bj) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = 32 * bi + 8 * (r / 4) + 4 * q + (r % 4);
                    const float v = acc[h * (MB / 2) + bi][bj][r] + bias_v[bj];
                    *(uint16_t*)(ost + row * kOutStride + 2 * (32 * bj + j)) =
                        XK == kF16 ? float_to_half_bits(v) : float_to_bf16_bits(v);
                }
            }
        }
        // LDS accesses of one wave complete in order; the empty asm keeps the
        // compiler from reordering the staging writes and reads.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < kHalfRows / 8; ++i) {
            const int row = 8 * i + (lane >> 3);
            const int c8 = lane & 7;
            const u32x4 v = *(const u32x4*)(ost + row * kOutStride + 16 * c8);
            const int64_t m = m0 + h * kHalfRows + row;
            const int64_t n = nw + 8 * c8;
            if (m < a.M) {
                if (a.vec_out && n + 8 <= a.N) {
                    *(u32x4*)(y + m * a.N + n) = v;
                } else {
#pragma unroll 1
                    for (int e = 0; e < 8; ++e)
                        if (n + e < a.N) y[m * a.N + n + e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
                }
            }
        }
        asm volatile("" ::: "memory");
    }
}

// Sum of the K-range partials of every split tile, in range order
// (deterministic), plus bias, rounded to the output type.  One thread: 8
// consecutive outputs of one tile row.
template <int OUTK>
__global__ __launch_bounds__(256) void gemm2_reduce_kernel(Gemm2Args a) {
    constexpr int kPerTile = kBM * kBN / (256 * 8);  // workgroups per tile
    const int idx = blockIdx.x / kPerTile;           // split tile index
    const int e = ((blockIdx.x % kPerTile) * 256 + threadIdx.x) * 8;
    const int row = e / kBN;
    const int col = e % kBN;
    const int t = a.dp_tiles + idx;
    const int tile_m = t / a.tiles_n;
    const int tile_n = t - tile_m * a.tiles_n;
    const int64_t m = (int64_t)tile_m * kBM + row;
    const int64_t n = (int64_t)tile_n * kBN + col;
    if (m >= a.M || n >= a.N) return;
    const float* src = a.partials + (int64_t)idx * a.splits * (kBM * kBN) + row * kBN + col;
    float4v s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    int piece = 0;
    for (; piece + 4 <= a.splits; piece += 4) {  // four pieces' loads in flight, added in order
        float4v v[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            v[u][0] = *(const float4v*)(src + (int64_t)(piece + u) * (kBM * kBN));
            v[u][1] = *(const float4v*)(src + (int64_t)(piece + u) * (kBM * kBN) + 4);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            s0 += v[u][0];
            s1 += v[u][1];
        }
    }
    for (; piece < a.splits; ++piece) {
        s0 += *(const float4v*)(src + (int64_t)piece * (kBM * kBN));
        s1 += *(const float4v*)(src + (int64_t)piece * (kBM * kBN) + 4);
    }
    float out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int64_t nn = n + i < a.N ? n + i : a.N - 1;
        out[i] = (i < 4 ? s0[i] : s1[i - 4]) + load_bias(a.bias, a.bias_kind, nn);
    }
    if constexpr (OUTK == kF32) {
        float* y = (float*)a.y;
        if (a.vec_out && n + 8 <= a.N) {
            *(float4v*)(y + m * a.N + n) = float4v{out[0], out[1], out[2], out[3]};
            *(float4v*)(y + m * a.N + n + 4) = float4v{out[4], out[5], out[6], out[7]};
        } else {
            for (int i = 0; i < 8 && n + i < a.N; ++i) y[m * a.N + n + i] = out[i];
        }
        return;
    }
    uint16_t* y = (uint16_t*)a.y;
    if (a.vec_out && n + 8 <= a.N) {
        u32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = OUTK == kF16 ? float_to_half_bits(out[2 * i]) : float_to_bf16_bits(out[2 * i]);
            const uint32_t hi = OUTK == kF16 ? float_to_half_bits(out[2 * i + 1]) : float_to_bf16_bits(out[2 * i + 1]);
            v[i] = lo | (hi << 16);
        }
        *(u32x4*)(y + m * a.N + n) = v;
    } else {
        for (int i = 0; i < 8 && n + i < a.N; ++i) store_out<OUTK>(a.y, m * a.N + n + i, out[i]);
    }
}

struct Gemm2Plan {
    int tiles_m, tiles_n, dp_tiles, splits, gps, split_tiles;
    int64_t partial_bytes;
};

// Workgroup slots of the device (two per CU), queried once per device.
int gemm2_slots() {
    static int slots[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (slots[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        slots[dev] = 2 * cus;
    }
    return slots[dev];
}

// Choose data-parallel tiles and K splits.  Measured on MI355X: a K step
// costs ~1.0 us with one workgroup per CU and ~1.54 us for the two that
// share a CU; a round of workgroups costs ~6 us fixed (launch, pipeline
// fill, epilogue); the reduction kernel ~2 us plus its partial-sum reads at
// ~5 TB/s.  Full rounds of tiles stay data-parallel; the tiles of a last,
// less than half full round -- or all tiles, when there are fewer than the
// workgroup slots -- are split into the K-range count with the lowest
// modelled time.
Gemm2Plan plan_gemm2(int64_t rows, int64_t out_features, int64_t in_features) {
    Gemm2Plan pl{};
    pl.tiles_m = (int)((rows + kBM - 1) / kBM);
    pl.tiles_n = (int)((out_features + kBN - 1) / kBN);
    const int tiles = pl.tiles_m * pl.tiles_n;
    const int G = (int)(in_features / 64);
    const int slots = gemm2_slots();
    const int cus = slots / 2;
    int rem = tiles % slots;
    if (tiles >= slots && (rem == 0 || 2 * rem > slots)) rem = 0;
    pl.dp_tiles = tiles - rem;
    pl.split_tiles = rem;
    pl.splits = 1;
    pl.gps = G;
    if (rem > 0) {
        auto step_us = [&](int wgs) { return wgs <= cus ? 1.0 : 1.54; };
        double best = 6.0 + G * step_us(rem);  // unsplit
        for (int sp = 2; sp <= G && rem * sp <= slots; ++sp) {
            const int gps = (G + sp - 1) / sp;
            const int used = (G + gps - 1) / gps;
            const double t = 6.0 + gps * step_us(rem * used) + 2.0 + (double)rem * used * kBM * kBN * 4 / 5e6;
            if (t < best) {
                best = t;
                pl.splits = used;
                pl.gps = gps;
            }
        }
    }
    if (pl.splits == 1) {
        pl.dp_tiles = tiles;
        pl.split_tiles = 0;
        pl.gps = G;
    }
    pl.partial_bytes = (int64_t)pl.split_tiles * pl.splits * kBM * kBN * 4;
    return pl;
}

// Split of every fp32 activation row into [hi | lo] bf16 planes: one
// thread per 8 consecutive values.  XK = kF32: x is fp32 [M, K]; XK =
// kSwiGLU: x is [M, 2K] bf16 (gate | up) and the activation is silu(gate) *
// up in fp32, silu(g) = g / (1 + exp(-g)) (src/qwen_int4/model.py:133-136).
template <int XK>
__global__ __launch_bounds__(256) void split_planes_kernel(const void* x, uint16_t* planes, int64_t items, int K) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= items) return;
    const int64_t e = i * 8;
    const int64_t m = e / K;
    const int64_t c = e - m * K;
    float4v f0, f1;
    if constexpr (XK == kSwiGLU) {
        const uint16_t* gu = (const uint16_t*)x + m * 2 * K + c;
        const u32x4 gv = *(const u32x4*)gu;
        const u32x4 uv = *(const u32x4*)(gu + K);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t gw = gv[t / 2], uw = uv[t / 2];
            const float g = bf16_bits_to_float(t & 1 ? gw >> 16 : gw & 0xFFFFu);
            const float u = bf16_bits_to_float(t & 1 ? uw >> 16 : uw & 0xFFFFu);
            const float h = (g / (1.0f + expf(-g))) * u;
            if (t < 4) f0[t] = h; else f1[t - 4] = h;
        }
    } else {
        f0 = *(const float4v*)((const float*)x + e);
        f1 = *(const float4v*)((const float*)x + e + 4);
    }
    u32x4 hi, lo;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float x0 = k < 2 ? f0[2 * k] : f1[2 * k - 4];
        const float x1 = k < 2 ? f0[2 * k + 1] : f1[2 * k - 3];
        const uint16_t h0 = float_to_bf16_bits(x0), h1 = float_to_bf16_bits(x1);
        const uint16_t l0 = float_to_bf16_bits(x0 - bf16_bits_to_float(h0));
        const uint16_t l1 = float_to_bf16_bits(x1 - bf16_bits_to_float(h1));
        hi[k] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        lo[k] = (uint32_t)l0 | ((uint32_t)l1 << 16);
    }
    *(u32x4*)(planes + m * 2 * K + c) = hi;
    *(u32x4*)(planes + m * 2 * K + K + c) = lo;
}

// Workspace: [split-tile partials][fp32 activations: bf16 planes, 256-byte aligned]
int64_t planes_offset(const Gemm2Plan& pl) { return (pl.partial_bytes + 255) / 256 * 256; }

}  // namespace

int64_t gemm2_workspace_bytes(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    const bool f32 = x_kind == kF32 || x_kind == kSwiGLU;
    const Gemm2Plan pl = plan_gemm2(rows, out_features, f32 ? 2 * in_features : in_features);
    if (f32) return planes_offset(pl) + rows * in_features * 4;
    return pl.partial_bytes;
}

bool gemm2_supported(const LinearProblem& p) {
    return p.x_kind == kF16 || p.x_kind == kBF16 || p.x_kind == kF32 || p.x_kind == kSwiGLU;
}

const char* gemm_kernel_name(int64_t, int64_t, int64_t, int x_kind) {
    if (x_kind == kF16) return "gemm2_kernel<f16,128>";
    if (x_kind == kBF16) return "gemm2_kernel<bf16,128>";
    if (x_kind == kSwiGLU) return "gemm2_kernel<bf16 hi|lo planes of silu(gate)*up,128>";
    return "gemm2_kernel<bf16 hi|lo planes of f32,128>";
}

hipError_t launch_gemm2(const LinearProblem& p, void* workspace, hipStream_t stream, hipEvent_t start,
                        hipEvent_t stop) {
    const bool f32 = p.x_kind == kF32 || p.x_kind == kSwiGLU;
    const int64_t k_act = f32 ? 2 * p.in_features : p.in_features;  // activation row length
    const Gemm2Plan pl = plan_gemm2(p.rows, p.out_features, k_act);
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
    args.K = (int)k_act;
    args.G = (int)(k_act / 64);
    args.wg = (int)(p.in_features / 64);
    args.tiles_m = pl.tiles_m;
    args.tiles_n = pl.tiles_n;
    args.vec_out = (((uintptr_t)p.y & 15) == 0) && (p.out_features % (f32 ? 4 : 8) == 0);
    args.dp_tiles = pl.dp_tiles;
    args.splits = pl.splits;
    args.gps = pl.gps;
    args.partials = pl.split_tiles ? (float*)workspace : nullptr;
    const dim3 grid((unsigned)(pl.dp_tiles + pl.split_tiles * pl.splits));
    const bool two = pl.split_tiles > 0;
    constexpr int kPerTile = kBM * kBN / (256 * 8);
    const dim3 rgrid((unsigned)(pl.split_tiles * kPerTile));
    hipError_t err;
    if (p.x_kind == kF16) {
        err = launch_kernel(gemm2_kernel<kF16, kBM, kF16>, grid, dim3(256), 0, stream, start, two ? nullptr : stop,
                            args);
        if (err == hipSuccess && two)
            err = launch_kernel(gemm2_reduce_kernel<kF16>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    } else if (p.x_kind == kBF16) {
        err = launch_kernel(gemm2_kernel<kBF16, kBM, kBF16>, grid, dim3(256), 0, stream, start, two ? nullptr : stop,
                            args);
        if (err == hipSuccess && two)
            err = launch_kernel(gemm2_reduce_kernel<kBF16>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    } else {
        // fp32 (or silu(gate) * up): [hi | lo] bf16 planes into the workspace, then the bf16 GEMM over 2K
        // with fp32 output
        uint16_t* planes = (uint16_t*)((char*)workspace + planes_offset(pl));
        const int64_t items = p.rows * p.in_features / 8;
        const dim3 sgrid((unsigned)((items + 255) / 256));
        if (p.x_kind == kSwiGLU)
            err = launch_kernel(split_planes_kernel<kSwiGLU>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, planes,
                                items, (int)p.in_features);
        else
            err = launch_kernel(split_planes_kernel<kF32>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, planes,
                                items, (int)p.in_features);
        args.x = planes;
        if (err == hipSuccess)
            err = launch_kernel(gemm2_kernel<kBF16, kBM, kF32>, grid, dim3(256), 0, stream, nullptr,
                                two ? nullptr : stop, args);
        if (err == hipSuccess && two)
            err = launch_kernel(gemm2_reduce_kernel<kF32>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    }
    return err;
}

}  // namespace w4g64
