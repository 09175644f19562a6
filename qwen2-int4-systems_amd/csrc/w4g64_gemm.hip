// Prefill path: pipelined W4G64 GEMM, rows > 16.
//
// y[M, N] = x[M, K] @ W^T (+ bias), W[n, k] = (code - zero) * scale -- the
// reference's dequantize-then-fp32-matmul (src/qwen_int4/backends.py:73-98),
// evaluated as
//     y[m, n] = rowscale[m] * sum_g scale[n, g] * D_g[m, n]  (+ bias[n]),
//     D_g[m, n] = sum_{k in g} a[m, k] * (code[n, k] - zero[n, g]),
// where D_g is one 64-wide group's contraction on the matrix cores
// (v_mfma_f32_16x16x32_f16, fp32 accumulation) and the group scale is
// applied to it in fp32 (one FMA per output per group).
//   * B = (code - zero) is an integer in [-15, 15]: exact in fp16, built from
//     the packed nibbles by one bitwise select and one v_pk_add_f16 per pair.
//     Every product a * (code - zero) is exact, and scale * D_g is the only
//     other rounding besides the fp32 sums, so the result is that of the
//     exact fp32 weights up to summation order.
//   * A = the activations as fp16, written by a staging kernel
//     (gemm_stage_kernel) into the workspace: each row times a power of two
//     2^-e chosen so that its largest finite magnitude lies in [2^14, 2^15),
//     and rowscale[m] = 2^e multiplies the row's outputs.  A bf16 value
//     (8 significant bits) is exact in fp16 after the scaling unless it lies
//     below 2^-32 times the row's largest magnitude, where fp16 subnormals
//     keep it to 2^-40 of that magnitude.  fp32 activations (and the SwiGLU
//     product silu(gate) * up of the down projection) become two fp16
//     planes, hi = RNE(t) and lo = RNE(t - hi), t = x 2^-e (22 significant
//     bits), laid out as one row [hi | lo] of 2K values; the GEMM runs over
//     K' = 2K with weight group g mod G, so both planes meet the same
//     weights.  fp16 activations are copied unscaled.
//   * The staging kernel also permutes each 8-value chunk into the slot
//     order [k0 k4 k1 k5 k2 k6 k3 k7], the order in which one packed dword's
//     nibble pairs fall out of a mask (bytes b and b + 2 share a 16-bit
//     lane), so the weights need no byte shuffle.
//
// Workgroup = 4 waves, output tile 128 x 256: wave w owns all 128 rows of the
// 64 output features [n0 + 64 w, n0 + 64 w + 64), as 8 x 4 blocks of 16 x 16.
// One K step = one 64-wide group.  Two workgroups share a CU (78 KB of LDS,
// at most 256 registers per lane each).
//   * Every load is a gfx950 direct global->LDS load into a ring of S = 3
//     stages, issued up to S steps ahead: the activation tile (16-byte
//     loads) and, per wave, its packed weight columns, scales and zero bytes.
//     Every 1 KB a wave instruction writes holds 8 tile rows; the 16 B
//     chunks of a row are XOR-swizzled by a_swizzle(row), which the fragment
//     reads undo, so fragment reads are conflict-free.
//   * Per step, a wave decodes its own 64 columns' (code - zero) for the
//     whole group (4 column blocks x 2 MFMAs), then walks its 8 row blocks:
//     for each, the four column blocks' 2-MFMA chains over the group (lane
//     group q of 4 takes K values [16 q, 16 q + 16) of the group, MFMA h
//     uses [16 q + 8 h, + 8)), then acc += scale * D, issued after the next
//     row block's MFMAs so the matrix cores and the FMAs overlap.
//   * Waits are explicit: every step issues the same number of vector memory
//     operations, so "step s has landed" is a vmcnt bound known at compile
//     time (steps past the end are not issued; the last waits tighten).
//     All loads are drained before the workgroup exits.
//   * Tiles are assigned so that the workgroups of one XCD (ids congruent
//     mod 8) cover consecutive tiles of one row band: they share the
//     activation band in their L2.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kStages = 3;
constexpr int kBN = 256;  // 4 waves x 64 output features
constexpr int kBM = 128;  // rows per tile
constexpr int kXcds = 8;

struct GemmArgs {
    const uint16_t* x;      // staged fp16 activations [M][K], slot order
    const float* rowscale;  // [tiles_m * kBM] power-of-two row factors; null: 1
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;
    void* y;
    int M;
    int N;
    int K;   // staged row length (2 in_features for two planes)
    int G;   // staged groups, K / 64
    int wg;  // weight groups (in_features / 64): step g reads weight group g mod wg
    int tiles_m;
    int tiles_n;
    int band_group;  // row bands per group of the tile order (tile_coords)
    int vec_out;    // y is 16-byte aligned and N % 8 == 0 (fp32: N % 4): 16-byte output stores
    int dp_tiles;   // tiles [0, dp_tiles): one workgroup each over the whole K range
    int splits;     // tiles [dp_tiles, tiles): `splits` workgroups each, one K range apiece
    int gps;        // groups per K range of a split tile
    float* partials;  // [(tile - dp_tiles) * splits + piece][kBM][kBN] fp32, already times rowscale
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;
// Word 3 of a raw gfx9 buffer resource (32-bit data format; no swizzle, no stride).
constexpr int kRsrcWord3 = 0x00020000;

// s_waitcnt with only the vector memory counter constrained (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4] and lgkmcnt [11:8] left at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4)); }
// Physical 16-byte chunk offset of tile row r (rows are 128 B = 8 chunks).
// Row r's chunks start at bank group 8 (r & 1) (mod 16 groups of 4 banks);
// the XOR term takes 8 distinct values over any 8 consecutive rows and over
// the 8 rows of either parity among 16 consecutive rows.
__device__ __forceinline__ int a_swizzle(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
// Workgroup execution barrier without a memory fence (a fence would drain the
// loads still in flight); the empty asm statements keep the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void block_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Bitwise select (x ^ C) & M | (C & ~M), one v_bitop3: inside the mask the
// nibble n XOR 8 = n' = code + 8, outside it the magic exponent bits of C.
template <uint32_t C, uint32_t M>
__device__ __forceinline__ uint32_t nib_select(uint32_t x) {
    return ((x ^ C) & M) | (C & ~M);
}
// fp16 pairs (1024 + n', 1024 + n'') from bits 0-3 / 16-19 and (64 + n', 64 +
// n'') from bits 4-7 / 20-23 (n' XOR-ed in by the 8s of C).
constexpr uint32_t kMaskLo = 0x000F000Fu, kSelLo = 0x64086408u;
constexpr uint32_t kMaskHi = 0x00F000F0u, kSelHi = 0x54805480u;

// (code - zero) of one packed dword (8 consecutive K values of a column), as
// 4 fp16 pairs in slot order [k0 k4 | k1 k5 | k2 k6 | k3 k7].  zlo = fp16
// pair (1032 + z, 1032 + z), zhi = (72 + z, 72 + z): (1024 + n') - (1032 + z)
// = (64 + n') - (72 + z) = code - z, exact.
__device__ __forceinline__ u32x4 decode_codes(uint32_t w, half2v zlo, half2v zhi) {
    const uint32_t w8 = w >> 8;
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, nib_select<kSelLo, kMaskLo>(w)) - zlo);
    r[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, nib_select<kSelHi, kMaskHi>(w)) - zhi);
    r[2] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, nib_select<kSelLo, kMaskLo>(w8)) - zlo);
    r[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, nib_select<kSelHi, kMaskHi>(w8)) - zhi);
    return r;
}

// Tile t -> (row band, column tile): bands in groups of bg, each group's
// tiles column by column (t = group-major, then column, then band), leftover
// bands row by row (bg = 1: row-major).  With data-parallel tiles (bg = 4),
// consecutive tiles -- what one XCD's workgroups take -- cover a few row
// bands by a run of column tiles, whose weights stay in that XCD's L2 while
// its bands are read (gate 8960x1536 at 2048 rows: GEMM fetch 107 -> 54 MB).
// Split-only GEMMs keep row-major tiles: their K-range-major deal already
// keeps a band's activation slice in one L2 (down 1536x8960: 63 MB against
// 75 with bg = 4).
__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int bg, int& tm, int& tn) {
    const int grouped = (tiles_m / bg) * bg * tiles_n;
    if (t < grouped) {
        const int g = t / (bg * tiles_n);
        const int w = t - g * (bg * tiles_n);
        tn = w / bg;
        tm = g * bg + (w - tn * bg);
    } else {
        const int r = t - grouped;
        tm = (tiles_m / bg) * bg + r / tiles_n;
        tn = r - (r / tiles_n) * tiles_n;
    }
}

// NWV waves per workgroup, each owning CW = 256 / NWV output features: 4
// waves (two workgroups per CU, gemm_kernel) or 8 (one workgroup per CU, two
// waves per SIMD on the same tile, gemm_kernel8, for launches with at most
// one workgroup per CU).  The body is a device function: kernels whose own
// template parameters decide the wave count were given no host-side launch
// handle by this compiler.
template <int OUTK, int NWV>
__device__ __forceinline__ void gemm_body(const GemmArgs& a) {
    static_assert(NWV == 4 || NWV == 8, "4 or 8 waves");
    constexpr int CW = kBN / NWV;               // output features per wave (64 or 32)
    constexpr int CB = CW / 16;                 // 16-column MFMA blocks per wave
    constexpr int WB = CW / 32;                 // 1 KB weight DMA instructions per wave (32 columns each)
    constexpr int RB = kBM / 16;                // 16-row MFMA blocks per wave
    constexpr int kABytes = kBM * 128;          // kBM rows x 64 fp16 values
    constexpr int kWBytes = NWV * WB * 1024;    // per wave WB x (32 columns x 32 B)
    // Sub-dword global->LDS loads write one zero-extended dword per lane.
    constexpr int kSBytes = NWV * 64 * 4;       // one fp16 scale per column (in a dword; lanes past CW unused)
    constexpr int kZBytes = NWV * 64 * 4;       // the byte holding each column's zero nibble (in a dword)
    constexpr int kStageBytes = kABytes + kWBytes + kSBytes + kZBytes;
    constexpr int kDma = kABytes / 1024 / NWV;  // 1 KB activation DMA instructions per wave
    constexpr int kOpsPerStep = kDma + WB + 1 + 1;  // + weight blocks, scales, zeros
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kStages][kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // uniform, so the LDS destinations (M0) and stage offsets derived from it stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- tile and K range of this workgroup ----
    // Data-parallel tiles: workgroup ids are dealt to the XCDs round robin
    // (id % 8); XCD x gets the contiguous tile range [start_x, start_x +
    // count_x) -- a bijection on [0, dp_tiles) -- so an XCD's workgroups share
    // activation row bands in their L2.  Split tiles follow: `splits`
    // workgroups per tile, each over its own K range, writing fp32 partial
    // sums that a second kernel adds up in range order.
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
        // split workgroups: the (K range, tile) list in K-range-major order is
        // dealt to the XCDs in contiguous runs, so an XCD's workgroups share
        // K ranges, and the activation slice of a row band (read by every
        // column tile) and the weight slice of a column tile (read by every
        // row band) stay in its L2
        const int split_tiles = a.tiles_m * a.tiles_n - a.dp_tiles;
        const int total = split_tiles * a.splits;
        const int sb = bid - a.dp_tiles;
        const int xcd = sb % kXcds;
        const int base = total / kXcds;
        const int extra = total % kXcds;
        const int e = xcd * base + (xcd < extra ? xcd : extra) + sb / kXcds;
        const int piece = e / split_tiles;
        const int ti = e - piece * split_tiles;
        t = a.dp_tiles + ti;
        slot = ti * a.splits + piece;  // partial-sum slot: tile-major, as the reduction reads them
        gbeg = piece * a.gps;
        gcnt = min(a.gps, a.G - gbeg);
    }
    int tile_m, tile_n;
    tile_coords(t, a.tiles_m, a.tiles_n, a.band_group, tile_m, tile_n);
    const int64_t m0 = (int64_t)tile_m * kBM;
    const int64_t nw = (int64_t)tile_n * kBN + CW * wave;  // this wave's first output feature

    // ---- per-lane DMA sources ----
    // Each load address is a uniform base advanced per step (scalar
    // registers) plus a fixed 32-bit per-lane byte offset, so a step's loads
    // cost no vector instructions.  The host keeps the staged rows and the
    // packed weights below 2^31 elements, so the byte offsets fit 32 bits.
    // activations: instruction d writes tile rows [8 (wave kDma + d), +8), 16 B per lane
    uint32_t a_off[kDma];
#pragma unroll
    for (int d = 0; d < kDma; ++d) {
        const int r = 8 * (wave * kDma + d) + (lane >> 3);
        const int chunk = (lane & 7) ^ a_swizzle(r);
        int m = (int)m0 + r;
        m = m < a.M ? m : a.M - 1;  // rows past M load a valid row; their outputs are not stored
        a_off[d] = 2u * ((uint32_t)m * (uint32_t)a.K + 8u * (uint32_t)chunk);
    }
    // weights: DMA instruction b, lane L -> column nw + 32 b + L % 32, bytes [16 (L / 32), +16)
    const int c = lane & 15;   // this lane's column within a 16-column block / row within a 16-row block
    const int kq = lane >> 4;  // this lane's K slot group
    uint32_t w_off[WB];
#pragma unroll
    for (int b = 0; b < WB; ++b) {
        int n = (int)nw + 32 * b + (lane & 31);
        n = n < a.N ? n : a.N - 1;
        w_off[b] = (uint32_t)n * (uint32_t)a.wg * 32u + 16u * (uint32_t)(lane >> 5);
    }
    // scale / zero of column nw + lane: element s_row + gw of weight group gw.
    // The zero nibble's byte is (s_row + gw) >> 1 = (s_row >> 1) + (s_row & gw & 1).
    int ncol = (int)nw + lane;
    ncol = ncol < a.N ? ncol : a.N - 1;
    const uint32_t s_row = (uint32_t)ncol * (uint32_t)a.wg;  // scale / zero element of weight group 0
    const uint32_t s_off = 2u * s_row;
    const uint32_t z_off_even = s_row >> 1, z_off_odd = (s_row >> 1) + (s_row & 1u);
    // weight group of this workgroup's K step gg (one wrap at most: K' <= 2 in_features)
    auto wgroup = [&](int gg) {
        const int gabs = gbeg + gg;
        return gabs >= a.wg ? gabs - a.wg : gabs;
    };

    // Buffer resources over the four operands (raw, stride 0, exact byte
    // sizes): a load's address is the per-lane offset plus a per-step scalar
    // offset, and a step's issue costs scalar instructions only.
    const __amdgpu_buffer_rsrc_t x_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, 0, (int)(2u * (uint32_t)a.M * (uint32_t)a.K), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t w_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.qweight, 0, (int)((uint32_t)a.N * (uint32_t)a.wg * 32u), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t s_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, 0, (int)((uint32_t)a.N * (uint32_t)a.wg * 2u), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t z_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.zeros, 0, (int)(((uint32_t)a.N * (uint32_t)a.wg + 1u) >> 1), kRsrcWord3);
    auto issue = [&](int gg) {  // callers pass gg < G only
        unsigned char* st = smem[gg % kStages];
        const int gw = wgroup(gg);
        const uint32_t z_off = (gw & 1) ? z_off_odd : z_off_even;
#pragma unroll
        for (int d = 0; d < kDma; ++d)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(x_rsrc, (lds_ptr_t)(st + 1024 * (wave * kDma + d)), 16, a_off[d],
                                                     128 * (gbeg + gg), 0, 0);
#pragma unroll
        for (int bj = 0; bj < WB; ++bj)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(w_rsrc, (lds_ptr_t)(st + kABytes + 1024 * (WB * wave + bj)), 16,
                                                     w_off[bj], 32 * gw, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rsrc, (lds_ptr_t)(st + kABytes + kWBytes + 256 * wave), 2, s_off,
                                                 2 * gw, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(z_rsrc, (lds_ptr_t)(st + kABytes + kWBytes + kSBytes + 256 * wave), 1,
                                                 z_off, gw >> 1, 0, 0);
    };

    float4v acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int bj = 0; bj < CB; ++bj) acc[i][bj] = float4v{0.f, 0.f, 0.f, 0.f};

    // Bit position of the zero nibble of this lane's columns nw + 16 bj + c in
    // its byte: the parity of the element index n wg + gw, i.e. of c wg + gw
    // (nw and 16 bj are even), for gw even / odd.  A column past N (clamped to
    // N - 1 in the loads) may take the other nibble: its outputs are not stored.
    const int cpar = c & a.wg & 1;
    const int zsh_even = 4 * cpar, zsh_odd = 4 * (cpar ^ 1);

    // Packed weights of step g for column block bj, read back from the stage:
    // the 8 bytes = K values [16 kq, 16 kq + 16) of column nw + 16 bj + c;
    // dword h holds the K slots of MFMA h (K values 16 kq + 8 h + [0, 8)).
    struct BRaw {
        u32x2 w;
        uint32_t sbits;
        uint32_t zb;
    };
    auto read_b = [&](int g, int bj) {
        const unsigned char* st = smem[g % kStages];
        const int col = 16 * bj + c;  // column within the wave
        BRaw r;
        r.w = *(const u32x2*)(st + kABytes + 1024 * (WB * wave + (col >> 5)) + 16 * ((col & 31) + 32 * (kq >> 1)) +
                              8 * (kq & 1));
        r.sbits = *(const uint16_t*)(st + kABytes + kWBytes + 256 * wave + 4 * col);
        r.zb = st[kABytes + kWBytes + kSBytes + 256 * wave + 4 * col];
        return r;
    };
    // Per-group constants of one column: the zero point's magic offsets and
    // the scale.  zsh = bit position of the column's zero nibble in its byte.
    struct BConst {
        half2v zlo;  // (1032 + z, 1032 + z)
        half2v zhi;  // (72 + z, 72 + z)
        float s;
    };
    auto group_const = [&](int zsh, const BRaw& r) {
        const int zn = __builtin_amdgcn_sbfe((int)r.zb, zsh, 4);  // signed zero point
        // fp16 bits of 1032 + z (mantissa unit 1) and of 72 + z (mantissa unit 1/16)
        const _Float16 zl = __builtin_bit_cast(_Float16, (uint16_t)(0x6408 + zn));
        const _Float16 zh = __builtin_bit_cast(_Float16, (uint16_t)(0x5480 + 16 * zn));
        BConst k;
        k.zlo = half2v{zl, zl};
        k.zhi = half2v{zh, zh};
        k.s = half_bits_to_float((uint16_t)r.sbits);
        return k;
    };
    // A fragment of row block bi for MFMA h: row 16 bi + c, K values 16 kq +
    // 8 h + [0, 8) = logical chunk 2 kq + h of the swizzled stage row.  The
    // swizzle of row 16 bi + c depends on c alone.
    const int a_lds0 = c * 128 + (((2 * kq) ^ a_swizzle(c)) * 16);
    const int a_lds1 = c * 128 + (((2 * kq + 1) ^ a_swizzle(c)) * 16);
    auto read_a = [&](const unsigned char* st, int bi, int h) {
        return *(const u32x4*)(st + 2048 * bi + (h ? a_lds1 : a_lds0));
    };
    auto mfma = [](const u32x4& av, const u32x4& bv, const float4v& acc_in) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av), __builtin_bit_cast(half8, bv),
                                                      acc_in, 0, 0, 0);
    };

    // ---- software pipeline ----
    // Step g: per row block the four column blocks' two-MFMA group chains and
    // the scaled accumulation of the previous row block, with the A fragments
    // of the row block two ahead read as soon as the current ones have been
    // issued; in row block 0 each column block's B (read at the end of step
    // g - 1) is decoded right before its first MFMA.  Before the last row
    // block: wait for this wave's loads of step g + 1, workgroup barrier
    // (every wave has finished reading stage g, and all of step g + 1 has
    // landed), refill of stage g with step g + 3; after it, the packed B of
    // step g + 1.
    // "Step s has landed" for this wave = its vector memory counter is at most
    // the number of operations issued after step s's (in-order completion).
    const int G = gcnt;  // steps of this workgroup's K range
    issue(0);
    if (G > 1) issue(1);
    if (G > 2) issue(2);
    if (G > 2) wait_vmcnt<2 * kOpsPerStep>();
    else if (G > 1) wait_vmcnt<kOpsPerStep>();
    else wait_vmcnt<0>();
    block_barrier();

    // Packed B of step 0 (every load of the first steps has landed and the
    // barrier above made them visible).  Stage g is refilled only after step
    // g's own barrier, so the B of step g + 1 can be read at the end of step
    // g, after that step's barrier.
    BRaw rb[CB];
#pragma unroll
    for (int bj = 0; bj < CB; ++bj) rb[bj] = read_b(0, bj);

    for (int g = 0; g < G; ++g) {
        const unsigned char* st = smem[g % kStages];
        u32x4 f[CB][2];  // (code - zero) of the column blocks, both MFMAs of the group
        float sc[CB];    // the column scales
        const int zsh = (wgroup(g) & 1) ? zsh_odd : zsh_even;
        // A fragments of row blocks bi (ab[bi & 1]), read two row blocks ahead
        u32x4 ab[2][2];
        ab[0][0] = read_a(st, 0, 0);
        ab[0][1] = read_a(st, 0, 1);
        ab[1][0] = read_a(st, 1, 0);
        ab[1][1] = read_a(st, 1, 1);
        // Row block bi's group products D go to dd[bi & 1]; its scaled
        // accumulation runs after row block bi + 1's MFMAs have been issued,
        // so the matrix cores and the FMAs of one wave overlap.
        float4v dd[2][CB];
        auto scale_add = [&](int bi) {
#pragma unroll
            for (int bj = 0; bj < CB; ++bj)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[bi][bj][i] = __builtin_fmaf(sc[bj], dd[bi & 1][bj][i], acc[bi][bj][i]);
            // the empty asm pins the accumulation here (sunk to the end of the
            // step, it would keep every block's products live)
#pragma unroll
            for (int bj = 0; bj < CB; ++bj) asm volatile("" : "+v"(acc[bi][bj]));
        };
        // Row block 0: each column block's B is decoded right before its first
        // MFMA, so the decode of the next column blocks overlaps the products.
#pragma unroll
        for (int bj = 0; bj < CB; ++bj) {
            const BConst k = group_const(zsh, rb[bj]);
#pragma unroll
            for (int h = 0; h < 2; ++h) f[bj][h] = decode_codes(rb[bj].w[h], k.zlo, k.zhi);
            sc[bj] = k.s;
            dd[0][bj] = mfma(ab[0][0], f[bj][0], float4v{0.f, 0.f, 0.f, 0.f});
            __builtin_amdgcn_sched_barrier(0);  // keeps the next decode behind this product
        }
        ab[0][0] = read_a(st, 2, 0);
#pragma unroll
        for (int bj = 0; bj < CB; ++bj) dd[0][bj] = mfma(ab[0][1], f[bj][1], dd[0][bj]);
        ab[0][1] = read_a(st, 2, 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int bi = 1; bi < RB; ++bi) {
            if (bi + 1 == RB) {
                // every A read of stage g has been issued; this wave's loads
                // of step g + 1 have landed once at most those of step g + 2
                // are outstanding
                if (g + 2 < G) wait_vmcnt<kOpsPerStep>();
                else wait_vmcnt<0>();
                if (g + 1 < G) {
                    wait_lgkmcnt0();
                    block_barrier();
                    if (g + 3 < G) issue(g + 3);
                }
            }
            float4v(&d)[CB] = dd[bi & 1];
#pragma unroll
            for (int bj = 0; bj < CB; ++bj) d[bj] = mfma(ab[bi & 1][0], f[bj][0], float4v{0.f, 0.f, 0.f, 0.f});
            if (bi + 2 < RB) ab[bi & 1][0] = read_a(st, bi + 2, 0);
#pragma unroll
            for (int bj = 0; bj < CB; ++bj) d[bj] = mfma(ab[bi & 1][1], f[bj][1], d[bj]);
            if (bi + 2 < RB) ab[bi & 1][1] = read_a(st, bi + 2, 1);
            scale_add(bi - 1);
            // the scheduling barrier stops later blocks' reads and products
            // from being hoisted (registers the accumulators need)
            __builtin_amdgcn_sched_barrier(0);
        }
        // packed B of step g + 1 (visible since this step's barrier); its LDS
        // reads are in flight during the last row block's accumulation
        if (g + 1 < G) {
#pragma unroll
            for (int bj = 0; bj < CB; ++bj) rb[bj] = read_b(g + 1, bj);
        }
        scale_add(RB - 1);
    }
    wait_vmcnt<0>();  // no DMA may still target this workgroup's LDS at exit

    // ---- row factors: acc *= rowscale[row] ----
    // 16x16 accumulator layout: column = lane % 16, row = 4 (lane / 16) + i
    // within the block, so rows 16 bi + 4 kq + [0, 4) are one float4.
    if (a.rowscale) {
#pragma unroll
        for (int bi = 0; bi < RB; ++bi) {
            const float4v rs = *(const float4v*)(a.rowscale + m0 + 16 * bi + 4 * kq);
#pragma unroll
            for (int bj = 0; bj < CB; ++bj)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[bi][bj][i] *= rs[i];
        }
    }

    // ---- split tile: fp32 partial sums, added up by gemm_reduce_kernel ----
    if (slot >= 0) {
        float* part = a.partials + (int64_t)slot * (kBM * kBN) + CW * wave + c;
#pragma unroll
        for (int bi = 0; bi < RB; ++bi)
#pragma unroll
            for (int bj = 0; bj < CB; ++bj)
#pragma unroll
                for (int i = 0; i < 4; ++i) part[(16 * bi + 4 * kq + i) * kBN + 16 * bj] = acc[bi][bj][i];
        return;
    }

    // ---- epilogue ----
    // Each wave stages its CW output columns through LDS, half of its rows
    // at a time, and writes 16 B per lane: full row segments of the wave's
    // columns.  Row stride 2 CW + 16 B (fp32: 4 CW + 16) keeps the 16-byte
    // reads aligned.
    block_barrier();  // every wave has finished reading the pipeline stages
    float bias_v[CB];
#pragma unroll
    for (int bj = 0; bj < CB; ++bj) {
        const int64_t n = nw + 16 * bj + c;
        bias_v[bj] = n < a.N ? load_bias(a.bias, a.bias_kind, n) : 0.0f;
    }
    constexpr int kHalfRows = kBM / 2;
    if constexpr (OUTK == kF32) {
        constexpr int kOutStride32 = 4 * CW + 16;
        constexpr int kLanesPerRow = CW / 4;  // 16 B per lane
        static_assert(NWV * kHalfRows * kOutStride32 <= kStages * kStageBytes, "output staging exceeds LDS");
        unsigned char* ost = &smem[0][0] + wave * kHalfRows * kOutStride32;
        float* y = (float*)a.y;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
            for (int bi = 0; bi < RB / 2; ++bi)
#pragma unroll
                for (int bj = 0; bj < CB; ++bj)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *(float*)(ost + (16 * bi + 4 * kq + i) * kOutStride32 + 4 * (16 * bj + c)) =
                            acc[hh * (RB / 2) + bi][bj][i] + bias_v[bj];
            asm volatile("" ::: "memory");
#pragma unroll
            for (int it = 0; it < kHalfRows * kLanesPerRow / 64; ++it) {
                const int row = (64 / kLanesPerRow) * it + lane / kLanesPerRow;
                const int c4 = lane % kLanesPerRow;
                const u32x4 v = *(const u32x4*)(ost + row * kOutStride32 + 16 * c4);
                const int64_t m = m0 + hh * kHalfRows + row;
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
    constexpr int kOutStride = 2 * CW + 16;
    constexpr int kLanesPerRow = CW / 8;  // 16 B per lane
    static_assert(NWV * kHalfRows * kOutStride <= kStages * kStageBytes, "output staging exceeds LDS");
    unsigned char* ost = &smem[0][0] + wave * kHalfRows * kOutStride;
    uint16_t* y = (uint16_t*)a.y;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
        for (int bi = 0; bi < RB / 2; ++bi)
#pragma unroll
            for (int bj = 0; bj < CB; ++bj)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float v = acc[hh * (RB / 2) + bi][bj][i] + bias_v[bj];
                    *(uint16_t*)(ost + (16 * bi + 4 * kq + i) * kOutStride + 2 * (16 * bj + c)) =
                        OUTK == kF16 ? float_to_half_bits(v) : float_to_bf16_bits(v);
                }
        // LDS accesses of one wave complete in order; the empty asm keeps the
        // compiler from reordering the staging writes and reads.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int it = 0; it < kHalfRows * kLanesPerRow / 64; ++it) {
            const int row = (64 / kLanesPerRow) * it + lane / kLanesPerRow;
            const int c8 = lane % kLanesPerRow;
            const u32x4 v = *(const u32x4*)(ost + row * kOutStride + 16 * c8);
            const int64_t m = m0 + hh * kHalfRows + row;
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

template <int OUTK>
__global__ __launch_bounds__(256, 2) void gemm_kernel(GemmArgs a) {
    gemm_body<OUTK, 4>(a);
}
template <int OUTK>
__global__ __launch_bounds__(512, 1) void gemm_kernel8(GemmArgs a) {
    gemm_body<OUTK, 8>(a);
}

// Sum of the K-range partials of every split tile, in range order
// (deterministic), plus bias, rounded to the output type.  One thread: 8
// consecutive outputs of one tile row.
template <int OUTK>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmArgs a) {
    constexpr int kPerTile = kBM * kBN / (256 * 8);  // workgroups per tile
    const int idx = blockIdx.x / kPerTile;           // split tile index
    const int e = ((blockIdx.x % kPerTile) * 256 + threadIdx.x) * 8;
    const int row = e / kBN;
    const int col = e % kBN;
    const int t = a.dp_tiles + idx;
    int tile_m, tile_n;
    tile_coords(t, a.tiles_m, a.tiles_n, a.band_group, tile_m, tile_n);
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

// ---- activation staging ----
// One workgroup per row.  The row's values t (fp16, bf16, fp32, or silu(gate)
// * up from a [gate | up] bf16 row, src/qwen_int4/model.py:133-136) are
// multiplied by 2^-e -- e chosen so that the largest finite |t| lands in
// [2^14, 2^15); fp16 input keeps e = 0 -- and stored as fp16 (two planes for
// the fp32-class kinds: hi = RNE(t) and lo = RNE(t - hi)), each 8-value chunk
// in slot order [k0 k4 k1 k5 k2 k6 k3 k7]; rowscale[m] = 2^e.
template <int XK>
__device__ __forceinline__ void stage_load8(const void* x, int64_t m, int K, int c, float (&v)[8]) {
    if constexpr (XK == kF16 || XK == kBF16) {
        const u32x4 d = *(const u32x4*)((const uint16_t*)x + m * K + 8 * c);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t bits = (d[i / 2] >> (16 * (i & 1))) & 0xFFFFu;
            v[i] = XK == kF16 ? half_bits_to_float((uint16_t)bits) : bf16_bits_to_float(bits);
        }
    } else if constexpr (XK == kF32) {
        const float4v f0 = *(const float4v*)((const float*)x + m * K + 8 * c);
        const float4v f1 = *(const float4v*)((const float*)x + m * K + 8 * c + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = f0[i];
            v[4 + i] = f1[i];
        }
    } else {
        const uint16_t* gu = (const uint16_t*)x + m * 2 * K + 8 * c;
        const u32x4 gv = *(const u32x4*)gu;
        const u32x4 uv = *(const u32x4*)(gu + K);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float gf = bf16_bits_to_float((gv[i / 2] >> (16 * (i & 1))) & 0xFFFFu);
            const float uf = bf16_bits_to_float((uv[i / 2] >> (16 * (i & 1))) & 0xFFFFu);
            v[i] = (gf / (1.0f + expf(-gf))) * uf;
        }
    }
}

// Scale 2^-e for a row whose largest finite magnitude is mx (e = 0 for 0).
__device__ __forceinline__ void row_factors(float mx, float& inv, float& rs) {
    inv = 1.0f;
    rs = 1.0f;
    if (mx > 0.0f) {
        int ex;
        (void)frexpf(mx, &ex);  // mx = f 2^ex, f in [0.5, 1)
        int sh = 15 - ex;       // mx 2^sh in [2^14, 2^15)
        sh = sh > 126 ? 126 : sh;
        inv = ldexpf(1.0f, sh);
        rs = ldexpf(1.0f, -sh);
    }
}

// Chunk c of the staged row: the 8 values times inv, as fp16 hi (and lo) in slot order.
template <bool kTwo>
__device__ __forceinline__ void stage_store8(uint16_t* row_out, int K, int c, const float (&v)[8], float inv) {
    constexpr int kSlot[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    u32x4 hi, lo;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        uint32_t hb[2], lb[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float t = v[kSlot[2 * p + h]] * inv;
            const _Float16 th = (_Float16)t;
            hb[h] = __builtin_bit_cast(uint16_t, th);
            // (an infinite hi keeps a zero lo: inf - inf would turn the row's results into NaN)
            lb[h] = __builtin_isfinite((float)th) ? __builtin_bit_cast(uint16_t, (_Float16)(t - (float)th)) : 0;
        }
        hi[p] = hb[0] | (hb[1] << 16);
        lo[p] = lb[0] | (lb[1] << 16);
    }
    *(u32x4*)(row_out + 8 * c) = hi;
    if constexpr (kTwo) *(u32x4*)(row_out + K + 8 * c) = lo;
}

// One pass when a thread holds at most kHeld chunks of the row (K <= 8 kHeld
// 256), else a second read of the row.
template <int XK>
__global__ __launch_bounds__(256) void gemm_stage_kernel(const void* x, uint16_t* out, float* rowscale, int K) {
    constexpr bool kTwo = XK == kF32 || XK == kSwiGLU;
    constexpr int kHeld = 8;
    __shared__ float wave_max[4];
    const int64_t m = blockIdx.x;
    const int chunks = K / 8;
    const bool held = chunks <= kHeld * 256;
    uint16_t* row_out = out + m * (kTwo ? 2 * (int64_t)K : K);
    float v[kHeld][8];
    float mx = 0.0f;
#pragma unroll
    for (int u = 0; u < kHeld; ++u) {
        const int cc = threadIdx.x + 256 * u;
        if (held && cc < chunks) {
            stage_load8<XK>(x, m, K, cc, v[u]);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (__builtin_isfinite(v[u][i])) mx = fmaxf(mx, fabsf(v[u][i]));
        }
    }
    if (!held) {
        for (int cc = threadIdx.x; cc < chunks; cc += 256) {
            float t[8];
            stage_load8<XK>(x, m, K, cc, t);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (__builtin_isfinite(t[i])) mx = fmaxf(mx, fabsf(t[i]));
        }
    }
    float inv = 1.0f, rsv = 1.0f;
    if constexpr (XK != kF16) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mx;
        __syncthreads();
        row_factors(fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3])), inv, rsv);
    }
    if (threadIdx.x == 0) rowscale[m] = rsv;
    if (held) {
#pragma unroll
        for (int u = 0; u < kHeld; ++u) {
            const int cc = threadIdx.x + 256 * u;
            if (cc < chunks) stage_store8<kTwo>(row_out, K, cc, v[u], inv);
        }
    } else {
        for (int cc = threadIdx.x; cc < chunks; cc += 256) {
            float t[8];
            stage_load8<XK>(x, m, K, cc, t);
            stage_store8<kTwo>(row_out, K, cc, t, inv);
        }
    }
}

struct GemmPlan {
    int tiles_m, tiles_n, dp_tiles, splits, gps, split_tiles;
    int64_t partial_bytes;
};

// Workgroup slots of the device (two per CU), queried once per device.
int gemm_slots() {
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
// fill, epilogue); the reduction kernel ~2 us plus the partial sums at ~2.5
// TB/s (written by the GEMM, read back by the reduction: at 5 TB/s the
// model split gate 8960x1536 at 128 rows into 6 K ranges, which measured
// 29.1 us against 27.2 us for 4).  Full rounds of tiles stay data-parallel; the tiles of a last,
// less than half full round -- or all tiles, when there are fewer than the
// workgroup slots -- are split into the K-range count with the lowest
// modelled time.
GemmPlan plan_gemm(int64_t rows, int64_t out_features, int64_t k_staged) {
    GemmPlan pl{};
    pl.tiles_m = (int)((rows + kBM - 1) / kBM);
    pl.tiles_n = (int)((out_features + kBN - 1) / kBN);
    const int tiles = pl.tiles_m * pl.tiles_n;
    const int G = (int)(k_staged / 64);
    const int slots = gemm_slots();
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
            const double t = 6.0 + gps * step_us(rem * used) + 2.0 + (double)rem * used * kBM * kBN * 4 / 2.5e6;
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

bool two_planes(int x_kind) { return x_kind == kF32 || x_kind == kSwiGLU; }

// 8-wave workgroups for launches of at most one workgroup per CU with no K
// split.  Measured (bf16 rows, same process, bit-identical outputs): gate
// 8960x1536 at 512 rows (140 tiles) 40.1 -> 38.2 us; split launches gain
// nothing or lose (gate at 128 rows, 35 tiles in 4 K ranges, 28.0 -> 26.5
// us, but down 1536x8960 at 512 rows, 24 tiles in 10 ranges, 40.3 -> 40.9,
// and the end-to-end prefill, whose small GEMMs all split, 6.16 -> 6.26 ms).
bool gemm_eight_waves(const GemmPlan& pl) {
    return pl.split_tiles == 0 && pl.dp_tiles <= gemm_slots() / 2;
}

// Workspace: [split-tile partials][staged fp16 rows][row factors], each part
// 256-byte aligned; the staged rows and row factors cover tiles_m * kBM rows.
struct GemmLayout {
    GemmPlan plan;
    int64_t staged_offset, rowscale_offset, bytes;
};
GemmLayout gemm_layout(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    GemmLayout l{};
    const int64_t k_staged = two_planes(x_kind) ? 2 * in_features : in_features;
    l.plan = plan_gemm(rows, out_features, k_staged);
    const int64_t padded_rows = (int64_t)l.plan.tiles_m * kBM;
    auto up256 = [](int64_t v) { return (v + 255) / 256 * 256; };
    l.staged_offset = up256(l.plan.partial_bytes);
    l.rowscale_offset = l.staged_offset + up256(rows * k_staged * 2);
    l.bytes = l.rowscale_offset + padded_rows * 4;
    return l;
}

}  // namespace

int64_t gemm_workspace_bytes(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    return gemm_layout(rows, out_features, in_features, x_kind).bytes;
}

bool gemm_supported(const LinearProblem& p) {
    if (p.x_kind != kF16 && p.x_kind != kBF16 && p.x_kind != kF32 && p.x_kind != kSwiGLU) return false;
    // the kernel addresses the staged rows and the packed weights with 32-bit offsets
    const int64_t k_staged = two_planes(p.x_kind) ? 2 * p.in_features : p.in_features;
    return p.rows * k_staged < (int64_t(1) << 31) && p.out_features * (p.in_features / 2) < (int64_t(1) << 31);
}

const char* gemm_kernel_name(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    const bool eight = gemm_eight_waves(gemm_layout(rows, out_features, in_features, x_kind).plan);
    if (x_kind == kF16)
        return eight ? "gemm_kernel<f16 a x int b,128x256,8 waves> (fp16 rows staged)"
                     : "gemm_kernel<f16 a x int b,128x256> (fp16 rows staged)";
    if (x_kind == kBF16)
        return eight ? "gemm_kernel<f16 a x int b,128x256,8 waves> (bf16 rows staged as scaled fp16)"
                     : "gemm_kernel<f16 a x int b,128x256> (bf16 rows staged as scaled fp16)";
    if (x_kind == kSwiGLU)
        return eight ? "gemm_kernel<f16 a x int b,128x256,8 waves> (silu(gate)*up staged as scaled fp16 hi|lo)"
                     : "gemm_kernel<f16 a x int b,128x256> (silu(gate)*up staged as scaled fp16 hi|lo)";
    return eight ? "gemm_kernel<f16 a x int b,128x256,8 waves> (f32 rows staged as scaled fp16 hi|lo)"
                 : "gemm_kernel<f16 a x int b,128x256> (f32 rows staged as scaled fp16 hi|lo)";
}

hipError_t launch_gemm(const LinearProblem& p, void* workspace, hipStream_t stream, hipEvent_t start,
                       hipEvent_t stop) {
    const GemmLayout l = gemm_layout(p.rows, p.out_features, p.in_features, p.x_kind);
    const GemmPlan& pl = l.plan;
    const bool two = two_planes(p.x_kind);
    uint16_t* staged = (uint16_t*)((char*)workspace + l.staged_offset);
    float* rowscale = (float*)((char*)workspace + l.rowscale_offset);
    GemmArgs args{};
    args.x = staged;
    args.rowscale = p.x_kind == kF16 ? nullptr : rowscale;
    args.qweight = p.qweight;
    args.scales = p.scales;
    args.zeros = p.zeros;
    args.bias = p.bias;
    args.bias_kind = p.bias_kind;
    args.y = p.y;
    args.M = (int)p.rows;
    args.N = (int)p.out_features;
    args.K = (int)(two ? 2 * p.in_features : p.in_features);
    args.G = args.K / 64;
    args.wg = (int)(p.in_features / 64);
    args.tiles_m = pl.tiles_m;
    args.tiles_n = pl.tiles_n;
    args.band_group = pl.dp_tiles > 0 ? 4 : 1;
    args.vec_out = (((uintptr_t)p.y & 15) == 0) && (p.out_features % (two ? 4 : 8) == 0);
    args.dp_tiles = pl.dp_tiles;
    args.splits = pl.splits;
    args.gps = pl.gps;
    args.partials = pl.split_tiles ? (float*)workspace : nullptr;
    const dim3 grid((unsigned)(pl.dp_tiles + pl.split_tiles * pl.splits));
    const bool reduce = pl.split_tiles > 0;
    constexpr int kPerTile = kBM * kBN / (256 * 8);
    const dim3 rgrid((unsigned)(pl.split_tiles * kPerTile));
    const dim3 sgrid((unsigned)p.rows);
    const int kin = (int)p.in_features;
    hipError_t err;
    switch (p.x_kind) {
        case kF16:
            err = launch_kernel(gemm_stage_kernel<kF16>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, staged,
                                rowscale, kin);
            break;
        case kBF16:
            err = launch_kernel(gemm_stage_kernel<kBF16>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, staged,
                                rowscale, kin);
            break;
        case kSwiGLU:
            err = launch_kernel(gemm_stage_kernel<kSwiGLU>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, staged,
                                rowscale, kin);
            break;
        default:
            err = launch_kernel(gemm_stage_kernel<kF32>, sgrid, dim3(256), 0, stream, start, nullptr, p.x, staged,
                                rowscale, kin);
            break;
    }
    if (err != hipSuccess) return err;
    // at most one workgroup per CU: 8 waves each (two per SIMD on one tile)
    const bool eight = gemm_eight_waves(pl);
    hipEvent_t gstop = reduce ? nullptr : stop;
    if (p.x_kind == kF16) {
        err = eight ? launch_kernel(gemm_kernel8<kF16>, grid, dim3(512), 0, stream, nullptr, gstop, args)
                    : launch_kernel(gemm_kernel<kF16>, grid, dim3(256), 0, stream, nullptr, gstop, args);
        if (err == hipSuccess && reduce)
            err = launch_kernel(gemm_reduce_kernel<kF16>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    } else if (p.x_kind == kBF16) {
        err = eight ? launch_kernel(gemm_kernel8<kBF16>, grid, dim3(512), 0, stream, nullptr, gstop, args)
                    : launch_kernel(gemm_kernel<kBF16>, grid, dim3(256), 0, stream, nullptr, gstop, args);
        if (err == hipSuccess && reduce)
            err = launch_kernel(gemm_reduce_kernel<kBF16>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    } else {
        err = eight ? launch_kernel(gemm_kernel8<kF32>, grid, dim3(512), 0, stream, nullptr, gstop, args)
                    : launch_kernel(gemm_kernel<kF32>, grid, dim3(256), 0, stream, nullptr, gstop, args);
        if (err == hipSuccess && reduce)
            err = launch_kernel(gemm_reduce_kernel<kF32>, rgrid, dim3(256), 0, stream, nullptr, stop, args);
    }
    return err;
}

}  // namespace w4g64
