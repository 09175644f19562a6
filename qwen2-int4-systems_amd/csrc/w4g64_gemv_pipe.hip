// Decode path, pipelined form: fused unpack + dequant + GEMV for 1..16
// fp16/bf16 activation rows, 16-byte weight loads kept in flight by a
// software pipeline for the whole life of every wave.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])  (+ bias[n])
// -- the reference's (x.float() @ W.t() + bias).to(x.dtype)
// (src/qwen_int4/backends.py:73-98) with each group's scale applied in fp32.
//
// Unit of work: a chunk, 16 B columns x one 16-byte load per lane = 1 KB of
// packed weights.  v_mfma_f32_16x16x32_{f16,bf16}:
//   * B column c = (row r, segment s), c = r SW + s, R = 16 / SW rows per
//     wave row block.  Lane (c, q) loads bytes [16 q, 16 q + 16) of group
//     pair jj = pb + s + SW t of its row at step t, so one load instruction
//     reads R rows x SW x 64 contiguous bytes.  Dword u of the lane feeds
//     MFMA u: K values 32 q + 8 u + 0..7 of the pair, so lanes q = 0, 1
//     carry the pair's first group and q = 2, 3 its second.
//   * A row i of tile mt = (virtual row v = 8 mt + i / 2, half p = i % 2),
//     v = m SW + s': x[m] over the pair of segment s' in the K slots of the
//     lanes q with q / 2 == p, zero elsewhere.  D[i, c] with s' == s is the
//     dot product of activation row m with weight row r over group 2 jj + p
//     alone; the other blocks are never read.  2 M SW <= 16 MT.
//   * fp16: B = code - zero exactly (1024 + n' and 64 + n' magic numbers,
//     one v_pk_add_f16 per pair of values subtracting 1032 + z / 72 + z);
//     bf16: B = 136 + code exactly, and the group result is corrected by
//     -(136 + zero) * sum_g x[m] (group sums formed once at staging).  The
//     group scale then multiplies in fp32.
//   * Grouped form (up to 16 rows, one segment): the four dwords of a
//     column's four lanes are transposed across the lanes (two
//     v_permlane32_swap and two v_permlane16_swap), so dword u of lane q
//     holds K values 32 u + 8 q + 0..7 and MFMAs 0, 1 see group 0 alone and
//     2, 3 group 1 alone: A row i is activation row i itself, one A tile
//     for all rows, and each group's D is scaled on its own.
//   * The activation range of the workgroup is staged once in LDS in MFMA
//     slot order.  Every wave first issues its share of the staging loads;
//     a barrier that waits for no memory keeps every weight load behind
//     every staging load (a CU returns vector memory data in issue order),
//     then each wave issues the loads of its first PF chunks (weights, the
//     row's two group scales, the zero byte), stages, and meets the others
//     at a barrier over LDS alone.
//   * Steps: each chunk waits for its own three loads alone, runs its
//     MFMAs and scaling, and issues the loads of the chunk PF chunks ahead,
//     so PF KB per wave stay in flight until the wave's last chunks.
//   * A wave owns RBW row blocks (interleaved with the other WR wave rows)
//     over its K part of SW T pairs; WK waves split the workgroup's K range
//     and meet in LDS at the end; K splits across workgroups (grid y) store
//     fp32 partial sums for the split-reduce kernel.
#include <stdio.h>

#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct PipeArgs {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    void* y;
    float* partials;  // [splits][Mo][N] (grid y > 1 or unreduced output)
    int bias_kind;
    int M;   // staged activation rows (bf16 planes: 3 Mo)
    int Mo;  // output rows
    int N;   // out_features (paired: 2 I)
    int I;   // paired: gate rows
    int K;   // in_features (a multiple of 128)
    int G;   // groups
    int P;   // group pairs
    int PS;  // pairs per K split
    // attention-merge form: x is the decode attention's partial results
    // (kAttnPartFloats per chunk, `att_chunks` chunks per key/value head,
    // att_bytes in all); query head h reads key/value head h / att_group
    // (att_ginv = 1 / att_group)
    int att_chunks;
    int att_group;
    int att_bytes;
    float att_ginv;
    // RMSNorm prologue (one row): x is the bf16 residual; the activation is
    // RMSNorm(x + delta) with `norm_w` and `eps`; workgroup (0, 0) stores
    // x + delta (bf16) to out_sum.  delta: bf16 [K] (FORM kNormBf16) or
    // `delta_parts` fp32 partial sums [parts][K] added in order (kNormParts).
    const void* delta;
    int delta_parts;
    const uint16_t* norm_w;
    float eps;
    uint16_t* out_sum;
    W4G64_TIMELINE_FIELDS
};

// LDS layout (bytes): xs [M][PS 128 + 8] slot-ordered activations | 64 zero
// bytes | sx [M][2 PS] fp32 group sums (bf16) | red (epilogue partial sums).
struct PipeLayout {
    int xw, zero, sx, red, total;
};
__host__ __device__ inline PipeLayout pipe_layout(int M, int PS, int red_floats) {
    PipeLayout L;
    L.xw = PS * 128 + 8;  // 16-bit elements per staged row (16 B of padding)
    L.zero = M * L.xw * 2;
    L.sx = L.zero + 64;
    L.red = L.sx + M * 2 * PS * 4;
    L.total = L.red + (red_floats > 16 ? red_floats : 16) * 4;  // >= 16 floats: the norm prologue's wave sums
    return L;
}

// Floats of the epilogue's reduction area: one K part per workgroup -- a
// private [RBW][M][R][SW] area per wave (no workgroup barrier), or none when
// every lane stores its own outputs (`direct`: one segment, plain rows, no
// pairing); several K parts -- [WK][M][rows][SW] shared by the workgroup.
__host__ __device__ constexpr int pipe_red_floats(int M, int SW, int WR, int WK, int RBW, bool direct) {
    return WK == 1 ? (direct ? 0 : WR * RBW * M * (16 / SW) * SW) : WK * M * (WR * RBW * (16 / SW)) * SW;
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float sum8_lanes(float s) {
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x4E, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x141, 0xF, 0xF, false));
    return s;
}

// ((w ^ 0x88888888) & MASK) | MAGIC: four nibbles with bit 3 flipped (a
// signed code c becomes c + 8) under a magic exponent.  Plain
// C on purpose: the compiler forms one v_bitop3_b32 from it and, unlike for
// inline asm, accounts for the wait states an MFMA needs after a VALU write
// of its operands (and before a VALU write of an MFMA's accumulator input).
template <uint32_t MASK, uint32_t MAGIC>
__device__ __forceinline__ uint32_t nibbles_magic(uint32_t w) {
    return ((w ^ 0x88888888u) & MASK) | MAGIC;
}
constexpr uint32_t kLoMask = 0x000F000Fu;
constexpr uint32_t kHiMask = 0x00F000F0u;
constexpr uint32_t kF16LoMagic = 0x64006400u;  // 1024 (fp16), nibble in bits 0-3
constexpr uint32_t kF16HiMagic = 0x54005400u;  // 64 (fp16), nibble in bits 4-7
constexpr uint32_t kBF16Magic = 0x43004300u;   // 128 (bf16)

// Exact (code - zero) of one packed dword as fp16 in slot order [k0 k4 k1 k5
// k2 k6 k3 k7]: 1024 + n' and 64 + n' (n' = code + 8) minus 1032 + z and
// 72 + z, whose fp16 bits are 0x6408 + z and 0x5480 + 16 z (ulps 1 and 1/16).
__device__ __forceinline__ half8 codes8_f16(uint32_t w, uint32_t clo, uint32_t chi) {
    const uint32_t w8 = w >> 8;
    const half2v c_lo = __builtin_bit_cast(half2v, clo), c_hi = __builtin_bit_cast(half2v, chi);
    const half2v h0 = __builtin_bit_cast(half2v, nibbles_magic<kLoMask, kF16LoMagic>(w)) - c_lo;
    const half2v h1 = __builtin_bit_cast(half2v, nibbles_magic<kHiMask, kF16HiMagic>(w)) - c_hi;
    const half2v h2 = __builtin_bit_cast(half2v, nibbles_magic<kLoMask, kF16LoMagic>(w8)) - c_lo;
    const half2v h3 = __builtin_bit_cast(half2v, nibbles_magic<kHiMask, kF16HiMagic>(w8)) - c_hi;
    half8 v = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
    return v;
}

// bf16 values 128 + n' = 136 + code (exact), slot order.
__device__ __forceinline__ bf16x8 codes8_bf16_biased(uint32_t w) {
    u32x4 v;
    v[0] = nibbles_magic<kLoMask, kBF16Magic>(w);
    v[1] = nibbles_magic<kLoMask, kBF16Magic>(w >> 4);
    v[2] = nibbles_magic<kLoMask, kBF16Magic>(w >> 8);
    v[3] = nibbles_magic<kLoMask, kBF16Magic>(w >> 12);
    return __builtin_bit_cast(bf16x8, v);
}

// A 16-bit load's bits, zero-extended where this statement stands.  The
// load is typed _Float16 and its register passes through an empty volatile
// asm here: the compiler cannot hoist the zero extension (which waits for
// the load) above this point, and -- as the asm emits nothing -- still sees
// every instruction it must keep hazard-free.
__device__ __forceinline__ uint32_t take_u16(_Float16 raw) {
    asm volatile("" : "+v"(raw));
    return (uint32_t)__builtin_bit_cast(uint16_t, raw);
}

template <int XK, int FORM, bool PAIRED, int SW, int MT, int WR, int WK, int RBW, int T, int DP, int STG>
__global__ __launch_bounds__(WR * WK * 64) void gemv_pipe_kernel(PipeArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int W = WR * WK;
    constexpr int kThreads = W * 64;
    constexpr int R = 16 / SW;          // rows per wave row block
    constexpr int RWG = WR * RBW * R;   // rows per workgroup
    constexpr int C = T * RBW;          // chunks per wave
    constexpr int PF = DP * RBW < C ? DP * RBW : C;  // chunks in flight
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wr = wave % WR;
    const int wk = wave / WR;
    const int M = a.M, N = a.N, K = a.K, G = a.G, P = a.P;
    constexpr int PL = FORM == kPlanes3 ? 3 : 1;  // staged rows per output row
    constexpr bool kNorm = FORM == kNormBf16 || FORM == kNormParts;
    constexpr bool kMerge = FORM == kAttnMerge;
    constexpr bool kGrp = FORM == kGrouped;
    static_assert(!kMerge || (!PAIRED && WK == 1), "attention merge: plain rows, the whole K range per workgroup");
    static_assert(!kGrp || (SW == 1 && MT == 1 && !PAIRED), "grouped: one segment, one A tile of up to 16 rows");
    static_assert(!PAIRED || (RBW == 2 && WK == 1), "paired: gate rows in row block 0, up rows in row block 1");
    static_assert(XK == kBF16 || FORM == kPlain || kGrp, "the fused forms are bf16");
    const int p0 = blockIdx.y * a.PS;        // first pair of the workgroup's K range
    const int pe = min(p0 + a.PS, P);        // end of its range
    const int ps = pe - p0;                  // pairs staged (>= 1)
    const int row0 = blockIdx.x * RWG;
    const PipeLayout L = pipe_layout(M, a.PS, pipe_red_floats(M, SW, WR, WK, RBW, SW == 1 && PL == 1 && !PAIRED));
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);

    // ---- lane roles ----
    const int c = lane & 15;
    const int q = lane >> 4;
    const int r = c / SW;
    const int s = c % SW;
    const int pb = p0 + wk * SW * T;  // this wave's first pair
    // Output row of row block b, row rl within the wave's block: blocks of
    // the workgroup's rows in turn, or -- paired -- gate row i (block 0) and
    // up row I + i (block 1) of the same i.
    auto rowof = [&](int b, int rl) -> int {
        if constexpr (PAIRED) return b * a.I + blockIdx.x * (WR * R) + wr * R + rl;
        else return row0 + (b * WR + wr) * R + rl;
    };
    // the rows a thread stores: with one K part per workgroup, lane l stores
    // row l % R of its row blocks b; otherwise thread t stores row t % RWG of
    // the workgroup (kThreads % RWG == 0)
    constexpr bool kWaveLocal = WK == 1;
    constexpr int NB = kWaveLocal ? RBW : 1;
    // one K part, one A tile, 2-8 segments: the segment sums stay in
    // registers (the epilogue below), and the storing lane of row r is lane
    // r SW of a lane row, so each lane's bias is that of row c / SW
    constexpr bool kRegSum = kWaveLocal && PL == 1 && MT == 1 && !kGrp && (SW == 2 || SW == 4 || SW == 8);
    static_assert(kWaveLocal || kThreads % RWG == 0, "a thread's outputs share its row");

    // ---- 0. bias of the stored outputs (raw bits, decoded at the stores) ----
    // one load whatever the kind (from the scales when there is no bias)
    // (fp32: the two halves of the element as two short loads)
    _Float16 bias_lo[NB], bias_hi[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        int brow = kWaveLocal ? rowof(b, kRegSum ? r : lane % R) : row0 + tid % RWG;
        brow = min(brow, N - 1);
        const _Float16* bp = (const _Float16*)(a.bias_kind == 0 ? (const void*)a.scales : a.bias);
        const int e = a.bias_kind == kF32 ? 2 * brow : (a.bias_kind == 0 ? 0 : brow);
        bias_lo[b] = bp[e];
        bias_hi[b] = bp[a.bias_kind == kF32 ? e + 1 : e];
    }
    auto bias_of = [&](int b) {
        const uint32_t lo = take_u16(bias_lo[b]);
        if (a.bias_kind == kF32) return __builtin_bit_cast(float, lo | (take_u16(bias_hi[b]) << 16));
        if (a.bias_kind == kF16) return half_bits_to_float((uint16_t)lo);
        if (a.bias_kind == kBF16) return bf16_bits_to_float(lo);
        return 0.0f;
    };

    // ---- 1. staging loads: item it = 8 activation values of row m ----
    // (norm forms: the residual's 8 values, the delta's and the norm
    // weight's; parts past delta_parts are not read)
    const int per_row = ps * 16;
    const int items = M * per_row;
    constexpr int kDeltaVecs = FORM == kNormParts ? 2 * kMaxDeltaParts : (FORM == kNormBf16 ? 1 : 0);
    u32x4 xv[STG];
    u32x4 dv[STG][kDeltaVecs > 0 ? kDeltaVecs : 1];
    u32x4 nwv[STG];
    int xit[STG];
#pragma unroll
    for (int u = 0; u < STG; ++u) {
        int it = kThreads * u + tid;
        it = it < items ? it : items - 1;
        xit[u] = it;
        const int m = it / per_row;
        const int k8 = it - m * per_row;
        if constexpr (!kMerge) xv[u] = *(const u32x4*)((const uint16_t*)a.x + (int64_t)m * K + (int64_t)p0 * 128 + 8 * k8);
        if constexpr (FORM == kNormBf16) {
            dv[u][0] = *(const u32x4*)((const uint16_t*)a.delta + 8 * k8);
        } else if constexpr (FORM == kNormParts) {
            // the delta_parts parts alone (a uniform branch each; the sums
            // below read only these)
#pragma unroll
            for (int pt = 0; pt < kMaxDeltaParts; ++pt)
                if (pt < a.delta_parts) {
                    const float* dsrc = (const float*)a.delta + (int64_t)pt * K + 8 * k8;
                    dv[u][2 * pt] = *(const u32x4*)dsrc;
                    dv[u][2 * pt + 1] = *(const u32x4*)(dsrc + 4);
                }
        }
        if constexpr (kNorm) nwv[u] = *(const u32x4*)(a.norm_w + 8 * k8);
    }
    // attention-merge form (one row): item it (values 8 it .. 8 it + 7 of
    // head h = 8 it / 128) reads the 8 exp-weighted value sums of every chunk
    // c < att_chunks (threads past the items load nothing), and for the
    // heads h = wave + W j each lane c < att_chunks loads chunk c's m and l
    static_assert(!kMerge || STG == 1, "attention merge: one staged item per thread");
    constexpr int kMC = kMerge ? kAttnMergeMaxChunks : 1;
    constexpr int kMJ = kMerge ? 4 : 1;
    // (held as float vectors: a bit cast of one element of an integer vector
    // compiles to element 0 of that vector with this compiler)
    float4v mv[kMC][2];
    float mstat[kMJ], lstat[kMJ];
    if constexpr (kMerge) {
        // buffer loads: the chunk's offset is a scalar operand, so a chunk's
        // loads need no per-lane address arithmetic (0x00020000: the gfx9
        // raw-buffer descriptor word; offsets past att_bytes read zeros)
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, 0, a.att_bytes, 0x00020000);
        const int heads = K / kAttnHeadDim;
        const int it = xit[0];  // one row, one K range: values 8 it .. 8 it + 7 of head it / 16
        const int h = it >> 4;
        const int kvh = (int)(((float)h + 0.5f) * a.att_ginv);  // exact for h < 2^20
        const int voff = 4 * (kvh * a.att_chunks * kAttnPartFloats + 2 * kAttnMaxGroup +
                              (h - kvh * a.att_group) * kAttnHeadDim + 8 * (it & 15));
        if (tid < items) {
#pragma unroll
            for (int c = 0; c < kMC; ++c)
                if (c < a.att_chunks) {
                    mv[c][0] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(prs, voff, c * 4 * kAttnPartFloats, 0));
                    mv[c][1] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(prs, voff + 16, c * 4 * kAttnPartFloats, 0));
                }
        }
        const int soff_lane = 4 * kAttnPartFloats * min(lane, a.att_chunks - 1);
#pragma unroll
        for (int j = 0; j < kMJ; ++j) {
            const int hj = min(wave + W * j, heads - 1);
            const int kj = (int)(((float)hj + 0.5f) * a.att_ginv);
            const int soff = 4 * (kj * a.att_chunks * kAttnPartFloats + hj - kj * a.att_group);
            mstat[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, soff_lane, soff, 0));
            lstat[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(prs, soff_lane + 4 * kAttnMaxGroup, soff, 0));
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's staging loads issue before any weight load
    asm volatile("" ::: "memory");

    // ---- 2. the first PF chunks' loads ----
    // chunk i = t RBW + b: row block b, step t; pairs past the range re-read
    // the range's first pair and get a zero scale
    const uint8_t* wbase[RBW];
    const uint16_t* sbase[RBW];
    const uint8_t* zbase[RBW];  // P is even, so a zero byte's parity is its pair's
#pragma unroll
    for (int b = 0; b < RBW; ++b) {
        const int row = min(rowof(b, r), N - 1);
        wbase[b] = a.qweight + (int64_t)row * (K / 2) + 16 * q;
        sbase[b] = a.scales + (int64_t)row * G;
        zbase[b] = a.zeros + (int64_t)row * P;
    }
    u32x4 wbuf[PF];
    uint32_t sbuf[PF];
    _Float16 zbuf[PF];  // the aligned 16 bits holding the zero byte (raw)
    auto issue = [&](int i) {
        const int t = i / RBW, b = i % RBW;
        const int jj = pb + s + SW * t;
        const int jl = jj < pe ? jj : p0;
        wbuf[i % PF] = __builtin_nontemporal_load((const u32x4*)(wbase[b] + 64 * (int64_t)jl));
        sbuf[i % PF] = *(const uint32_t*)(sbase[b] + 2 * jl);
        zbuf[i % PF] = *(const _Float16*)(zbase[b] + (jl & ~1));
        asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int i = 0; i < PF; ++i) issue(i);
#pragma unroll
    for (int u = 0; u < STG; ++u) {
        if constexpr (kMerge) {
#pragma unroll
            for (int c = 0; c < kMC; ++c) asm volatile("" : "+v"(mv[c][0]), "+v"(mv[c][1]));
        } else {
            asm volatile("" : "+v"(xv[u]));
        }
        if constexpr (kNorm) asm volatile("" : "+v"(nwv[u]));
#pragma unroll
        for (int k = 0; k < kDeltaVecs; ++k) asm volatile("" : "+v"(dv[u][k]));
    }
#pragma unroll
    for (int j = 0; j < kMJ; ++j) asm volatile("" : "+v"(mstat[j]), "+v"(lstat[j]));
    W4G64_STAMP(1);

    // ---- 2a. attention merge (model.py:101-104: softmax over all positions, then P V) ----
    // The decode attention's own merge, operation for operation: per (row,
    // head) m = max_c m_c, l = sum_c l_c exp(m_c - m) (lane c, then a wave
    // sum), scale_c = exp(m_c - m) / l; then per value the sum over chunks in
    // order of fmaf(sum_c, scale_c, .), rounded to bf16.  Chunks past the
    // position hold m = -inf, l = 0 and zero sums, so they add exactly
    // nothing, as the chunks past the position do in that merge.
    if constexpr (kMerge) {
        const int heads = K / kAttnHeadDim;
        float* scl = (float*)(smem + L.total);  // [M heads][kMC]
        // the kMJ pairs of a wave side by side (independent chains; pairs
        // past the heads repeat the last one and are not stored)
        const bool live = lane < a.att_chunks;
        float mx[kMJ], ex[kMJ], lsum[kMJ];
#pragma unroll
        for (int j = 0; j < kMJ; ++j) mx[j] = wave_max64(live ? fmaxf(-INFINITY, mstat[j]) : -INFINITY);
#pragma unroll
        for (int j = 0; j < kMJ; ++j) ex[j] = live ? expf(mstat[j] - mx[j]) : 0.0f;
#pragma unroll
        for (int j = 0; j < kMJ; ++j) lsum[j] = wave_sum64(live ? fmaf(lstat[j], ex[j], 0.0f) : 0.0f);
#pragma unroll
        for (int j = 0; j < kMJ; ++j) {
            const int hm = wave + W * j;
            if (hm < M * heads && lane < kMC) scl[hm * kMC + lane] = live ? ex[j] / lsum[j] : 0.0f;
        }
        lds_barrier();
        W4G64_STAMP(5);
        {
            const int hm = 8 * xit[0] / kAttnHeadDim;
            float scv[kMC];
#pragma unroll
            for (int c = 0; c < kMC; ++c) scv[c] = scl[hm * kMC + c];  // all read before the sums
            // the chunks that were loaded (a uniform branch each; threads
            // past the items hold no value and store none)
            float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < kMC; ++c)
                if (c < a.att_chunks) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        o[e] = fmaf(mv[c][0][e], scv[c], o[e]);
                        o[4 + e] = fmaf(mv[c][1][e], scv[c], o[4 + e]);
                    }
                }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                xv[0][e] = float_to_bf16_bits(o[2 * e]) | ((uint32_t)float_to_bf16_bits(o[2 * e + 1]) << 16);
        }
        W4G64_STAMP(6);
    }

    // ---- 2b. RMSNorm prologue (model.py:40-44, residual adds :149-154) ----
    // s = bf16(x + bf16(delta)) (the partial sums added in order from 0, then
    // + 0, as the split-K reduction does); the activation is
    // bf16(bf16(s * r) * w), r = rsqrt(mean(s^2) + eps) over the whole row
    // (squares rounded before the fp32 sum, as x.pow(2) is): each thread's
    // items, a wave sum, the waves' sums added in order after one barrier.
    // Workgroup (0, 0) stores s.
    if constexpr (kNorm) {
        float pt = 0.0f;
#pragma unroll
        for (int u = 0; u < STG; ++u) {
            const int it = kThreads * u + tid;
            float ps_ = 0.0f;
            u32x4 sb;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                // (each pair rounded to bf16 by one conversion instruction)
                const uint32_t xw = xv[u][e / 2];
                float df[2];
                if constexpr (FORM == kNormBf16) {
                    const uint32_t dw = dv[u][0][e / 2];
                    df[0] = bf16_lo(dw);
                    df[1] = bf16_hi(dw);
                } else {
                    float t[2] = {0.0f, 0.0f};
#pragma unroll
                    for (int pt2 = 0; pt2 < kMaxDeltaParts; ++pt2)
                        if (pt2 < a.delta_parts) {
#pragma unroll
                            for (int h = 0; h < 2; ++h) {
                                const uint32_t bits = dv[u][2 * pt2 + (e + h) / 4][(e + h) % 4];
                                t[h] = t[h] + __builtin_bit_cast(float, bits);
                            }
                        }
                    const uint32_t dp = pack_bf16x2(t[0] + 0.0f, t[1] + 0.0f);
                    df[0] = bf16_lo(dp);
                    df[1] = bf16_hi(dp);
                }
                const uint32_t sp = pack_bf16x2(bf16_lo(xw) + df[0], bf16_hi(xw) + df[1]);
                const float sv0 = bf16_lo(sp), sv1 = bf16_hi(sp);
                ps_ += __fmul_rn(sv0, sv0);
                ps_ += __fmul_rn(sv1, sv1);
                sb[e / 2] = sp;
            }
            xv[u] = sb;
            pt += it < items ? ps_ : 0.0f;  // clamped items repeat a real one
            if (blockIdx.x == 0 && blockIdx.y == 0 && it < items) *(u32x4*)(a.out_sum + 8 * xit[u]) = sb;
        }
        float* wsum = (float*)(smem + L.red);  // the epilogue's area, unused until then
        const float ws = wave_sum64(pt);
        if (lane == 0) wsum[wave] = ws;
        lds_barrier();
        float sq = wsum[0];
#pragma unroll
        for (int w = 1; w < W; ++w) sq += wsum[w];
        const float rinv = rsqrtf(sq / (float)K + a.eps);
#pragma unroll
        for (int u = 0; u < STG; ++u) {
            u32x4 xb;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t r = pack_bf16x2(bf16_lo(xv[u][e]) * rinv, bf16_hi(xv[u][e]) * rinv);
                xb[e] = pack_bf16x2(bf16_lo(r) * bf16_lo(nwv[u][e]), bf16_hi(r) * bf16_hi(nwv[u][e]));
            }
            xv[u] = xb;
        }
        // (the staging barrier below keeps the epilogue's later use of the
        // area behind every wave's read of the sums)
    }

    // ---- 3. staging into LDS (slot order) with the bf16 group sums ----
    {
        float* sx = (float*)(smem + L.sx);
#pragma unroll
        for (int u = 0; u < STG; ++u) {
            const int it = xit[u];
            const int m = it / per_row;
            const int k8 = it - m * per_row;
            // (threads past the items repeat the last one; in the merge form
            // they hold no value and leave its slot to the thread that has it)
            if (!kMerge || kThreads * u + tid < items) *(u32x4*)(smem + 2 * (m * L.xw + 8 * k8)) = permute_slots(xv[u]);
            if constexpr (XK == kBF16) {
                float sum = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    sum += __builtin_bit_cast(float, xv[u][e] << 16) + __builtin_bit_cast(float, xv[u][e] & 0xFFFF0000u);
                sum = sum8_lanes(sum);  // the 8 items of one (row, group) sit in 8 aligned lanes
                if ((it & 7) == 0) sx[m * 2 * a.PS + (k8 >> 3)] = sum;
            }
        }
        if (tid < 16) ((uint32_t*)(smem + L.zero))[tid] = 0u;
    }
    lds_barrier();
    W4G64_STAMP(2);

    // ---- 4. steps ----
    // A row of this lane in tile mt: i = lane % 16 -> v = 8 mt + i / 2, half
    // p = i % 2; it reads x only for m < M and q / 2 == p.  Grouped: A row i
    // is activation row i (rows past M repeat row M - 1; their D rows are
    // not stored).
    const int ai = lane & 15;
    const int ap = ai & 1;
    int am[MT], as_[MT];
    bool alive0[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int v = 8 * mt + (ai >> 1);
        am[mt] = v / SW;
        as_[mt] = v % SW;
        alive0[mt] = am[mt] < M && (q >> 1) == ap;
    }
    // D rows of this lane: i = 4 q + r' -> v = 8 mt + 2 q + r' / 2, p = r' % 2
    const float* sxl = (const float*)(smem + L.sx);
    const unsigned char* xs = smem;
    // (grouped: acc[g] sums group g of every pair, D row i = 4 q + r')
    constexpr int NA = kGrp ? 2 : MT;
    float4v acc[NA][RBW];
#pragma unroll
    for (int mt = 0; mt < NA; ++mt)
#pragma unroll
        for (int b = 0; b < RBW; ++b) acc[mt][b] = float4v{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int t = 0; t < T; ++t) {
        // this step's A fragments (shared by the RBW row blocks)
        u16x8 av[MT][4];
        if constexpr (kGrp) {
            // MFMA u: K values 32 u + 8 q + 0..7 of the pair (a pair past
            // the range reads the zero bytes, the same 16 for every u)
            const int ja = pb + t;
            const bool in = ja < pe;
            const unsigned char* asrc = in ? xs + 2 * (min(ai, M - 1) * L.xw + (ja - p0) * 128 + 8 * q) : smem + L.zero;
            const int ust = in ? 64 : 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) av[0][u] = *(const u16x8*)(asrc + ust * u);
        } else {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int ja = pb + as_[mt] + SW * t;
                const bool alive = alive0[mt] && ja < pe;
                // (dead lanes read the 64 zero bytes)
                const unsigned char* asrc =
                    alive ? xs + 2 * (am[mt] * L.xw + (ja - p0) * 128 + 32 * q) : smem + L.zero;
#pragma unroll
                for (int u = 0; u < 4; ++u) av[mt][u] = *(const u16x8*)(asrc + 16 * u);
            }
        }
        // bf16 group sums of the D rows' (m, pair) (clamped into the staged range)
        float2v gsum[MT][kGrp ? 4 : 2];
        if constexpr (XK == kBF16 && kGrp) {
            // D rows 4 q + r' (clamped), the step's pair
            const int jp = min(pb + t - p0, ps - 1);
#pragma unroll
            for (int h = 0; h < 4; ++h) gsum[0][h] = *(const float2v*)(sxl + min(4 * q + h, M - 1) * 2 * a.PS + 2 * jp);
        } else if constexpr (XK == kBF16) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int v = 8 * mt + 2 * q + h;
                    const int m = min(v / SW, M - 1);
                    const int jp = min(pb + (v % SW) + SW * t - p0, ps - 1);
                    gsum[mt][h] = *(const float2v*)(sxl + m * 2 * a.PS + 2 * jp);
                }
        }
        const int jj = pb + s + SW * t;  // this lane's pair (column side)
#pragma unroll
        for (int b = 0; b < RBW; ++b) {
            const int i = t * RBW + b;
            u32x4 w = wbuf[i % PF];
            uint32_t sw2 = sbuf[i % PF];
            asm volatile("" : "+v"(w), "+v"(sw2));  // this chunk's loads land here
            if constexpr (kGrp) {
                // 4 x 4 transpose of (lane row q, dword u) over the column's
                // lanes c, c + 16, c + 32, c + 48
                const auto t02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
                const auto t13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
                const auto t01 = __builtin_amdgcn_permlane16_swap(t02[0], t13[0], false, false);
                const auto t23 = __builtin_amdgcn_permlane16_swap(t02[1], t13[1], false, false);
                w = u32x4{t01[0], t01[1], t23[0], t23[1]};
            }
            const uint32_t zb = take_u16(zbuf[i % PF]);
            const int zoff = 8 * ((jj < pe ? jj : p0) & 1);  // the zero byte's half
            // a pair past the range re-reads an in-range pair and has zero A
            // fragments, so it adds 0; bf16 also zeroes its scale, as its
            // group correction (an in-range group's sum) is not zero
            const bool live = XK == kF16 || jj < pe;
            const float s0 = live ? half_bits_to_float((uint16_t)(sw2 & 0xFFFFu)) : 0.0f;
            const float s1 = live ? half_bits_to_float((uint16_t)(sw2 >> 16)) : 0.0f;
            float4v d[NA];
            if constexpr (kGrp) {
                // MFMAs 0, 1: group 0 of the pair; 2, 3: group 1
                const int z0 = (int)__builtin_amdgcn_sbfe((int)zb, zoff, 4);
                const int z1 = (int)__builtin_amdgcn_sbfe((int)zb, zoff + 4, 4);
                if constexpr (XK == kF16) {
                    half8 bv[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int zl = u < 2 ? z0 : z1;
                        bv[u] = codes8_f16(w[u], (uint32_t)(0x6408 + zl) * 0x00010001u,
                                           (uint32_t)(0x5480 + 16 * zl) * 0x00010001u);
                    }
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        d[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av[0][2 * g]), bv[2 * g],
                                                                      float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        d[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av[0][2 * g + 1]),
                                                                      bv[2 * g + 1], d[g], 0, 0, 0);
                    }
                } else {
                    bf16x8 bv[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) bv[u] = codes8_bf16_biased(w[u]);
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[0][2 * g]), bv[2 * g],
                                                                       float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        d[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[0][2 * g + 1]),
                                                                       bv[2 * g + 1], d[g], 0, 0, 0);
                    }
                    const float c0 = 136.0f + (float)z0, c1 = 136.0f + (float)z1;
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        d[0][h] = fmaf(-c0, gsum[0][h][0], d[0][h]);
                        d[1][h] = fmaf(-c1, gsum[0][h][1], d[1][h]);
                    }
                }
            } else if constexpr (XK == kF16) {
                // the zero point of this lane's own group (q / 2)
                const int zl = (int)__builtin_amdgcn_sbfe((int)zb, zoff + 4 * (q >> 1), 4);
                const uint32_t clo = (uint32_t)(0x6408 + zl) * 0x00010001u;
                const uint32_t chi = (uint32_t)(0x5480 + 16 * zl) * 0x00010001u;
                half8 bv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) bv[u] = codes8_f16(w[u], clo, chi);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    d[mt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        d[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av[mt][u]), bv[u],
                                                                       d[mt], 0, 0, 0);
                }
            } else {
                bf16x8 bv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) bv[u] = codes8_bf16_biased(w[u]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    d[mt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        d[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[mt][u]), bv[u],
                                                                        d[mt], 0, 0, 0);
                }
                const float c0 = 136.0f + (float)(int)__builtin_amdgcn_sbfe((int)zb, zoff, 4);  // (the builtin is unsigned)
                const float c1 = 136.0f + (float)(int)__builtin_amdgcn_sbfe((int)zb, zoff + 4, 4);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        d[mt][2 * h] = fmaf(-c0, gsum[mt][h][0], d[mt][2 * h]);
                        d[mt][2 * h + 1] = fmaf(-c1, gsum[mt][h][1], d[mt][2 * h + 1]);
                    }
            }
            if constexpr (kGrp) {
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    acc[0][b][h] = fmaf(s0, d[0][h], acc[0][b][h]);
                    acc[1][b][h] = fmaf(s1, d[1][h], acc[1][b][h]);
                }
            } else {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        acc[mt][b][2 * h] = fmaf(s0, d[mt][2 * h], acc[mt][b][2 * h]);
                        acc[mt][b][2 * h + 1] = fmaf(s1, d[mt][2 * h + 1], acc[mt][b][2 * h + 1]);
                    }
            }
            asm volatile("" ::: "memory");
            if (i + PF < C) issue(i + PF);
        }
    }
    W4G64_STAMP(3);

    // ---- 5. outputs ----
    // value of staged row mv for row block b and row rl, summed over segments
    // (and K parts) -- then, planes: the three staged rows of an output row
    // added; paired: silu(gate) * up stored as bf16 planes
    const bool split_out = a.partials != nullptr;
    const int Mo = a.Mo;
    auto emit = [&](int m, int n, float v, int b) {
        if (split_out) a.partials[((int64_t)blockIdx.y * Mo + m) * N + n] = v;
        else store_out<FORM == kPlanes3 ? kF32 : XK>(a.y, (int64_t)m * N + n, v + bias_of(b));
    };
    if constexpr (kGrp && kWaveLocal) {
        // lane (q, c): D rows 4 q + h are activation rows, column c is row r
#pragma unroll
        for (int b = 0; b < RBW; ++b)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int m = 4 * q + h;
                const int n = rowof(b, r);
                if (m < M && n < N) emit(m, n, acc[0][b][h] + acc[1][b][h], b);
            }
    } else if constexpr (kGrp) {
        float* red = (float*)(smem + L.red);  // [WK][M][RWG]
#pragma unroll
        for (int b = 0; b < RBW; ++b)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const int m = 4 * q + h;
                if (m < M) red[(wk * M + m) * RWG + (b * WR + wr) * R + r] = acc[0][b][h] + acc[1][b][h];
            }
        lds_barrier();
        for (int o = tid; o < Mo * RWG; o += kThreads) {
            const int m = o / RWG, wrow = o % RWG;
            const int n = row0 + wrow;
            if (n < N) {
                float v = 0.0f;
#pragma unroll
                for (int k2 = 0; k2 < WK; ++k2) v += red[(k2 * M + m) * RWG + wrow];
                emit(m, n, v, 0);
            }
        }
    } else if constexpr (kWaveLocal && SW == 1 && PL == 1 && !PAIRED) {
        // lane (q, c): rows v = 8 mt + 2 q + h of D are activation rows m = v
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int b = 0; b < RBW; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int m = 8 * mt + 2 * q + h;
                    const int n = rowof(b, r);
                    if (m < M && n < N) emit(m, n, acc[mt][b][2 * h] + acc[mt][b][2 * h + 1], b);
                }
    } else if constexpr (kRegSum) {
        // Row m, row r, segment s: D row v = m SW + s of lane (r SW + s, q =
        // v / 2) (one A tile: v < 8), both halves of the pair added.  The lane
        // rows holding one activation row's segments are added by row swaps
        // (v_permlane16_swap: rows 2m, 2m + 1 at SW 4; v_permlane32_swap as
        // well at SW 8, one row), then the SW lanes of the segment group by
        // DPP (quad swaps, half-row mirror), so every lane of the group holds
        // the row's sum; lane r SW of the row's first lane row stores it.
        // (the swapped pair is bit cast as a whole: a bit cast of one element
        // of an integer vector compiles to element 0 with this compiler)
        auto swap_sum = [](float v, auto swap) {
            const uint32_t a = __builtin_bit_cast(uint32_t, v);
            const float2v r = __builtin_bit_cast(float2v, swap(a, a));
            return r[0] + r[1];
        };
        const int h = s & 1;
        const int vr = 2 * q + h;  // this lane's D row pair: virtual row vr
        const bool own = vr % SW == s && vr / SW < Mo;
        auto rowsum = [&](int b) {
            float v = own ? acc[0][b][2 * h] + acc[0][b][2 * h + 1] : 0.0f;
            if constexpr (SW >= 4)
                v = swap_sum(v, [](uint32_t x, uint32_t y) { return __builtin_amdgcn_permlane16_swap(x, y, false, false); });
            if constexpr (SW == 8)
                v = swap_sum(v, [](uint32_t x, uint32_t y) { return __builtin_amdgcn_permlane32_swap(x, y, false, false); });
            v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
            if constexpr (SW >= 4)
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
            if constexpr (SW == 8)
                v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
            return v;
        };
        const int m = SW == 2 ? q : (SW == 4 ? q >> 1 : 0);
        const bool storer = s == 0 && (SW == 2 || (SW == 4 ? (q & 1) == 0 : q == 0)) && m < Mo;
        if constexpr (PAIRED) {
            const float g = rowsum(0), u = rowsum(1);
            const int i = blockIdx.x * (WR * R) + wr * R + r;
            if (storer && i < a.I) store_silu_planes(a.y, m, i, Mo, a.I, g + bias_of(0), u + bias_of(1));
        } else {
#pragma unroll
            for (int b = 0; b < RBW; ++b) {
                const float v = rowsum(b);
                const int n = rowof(b, r);
                if (storer && n < N) emit(m, n, v, b);
            }
        }
    } else if constexpr (kWaveLocal) {
        // the segments of a row meet in a private area of the wave: no
        // workgroup barrier, only the wave's own LDS order
        float* red = (float*)(smem + L.red) + wave * (RBW * M * R * SW);  // [RBW][M][R][SW]
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int b = 0; b < RBW; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int v = 8 * mt + 2 * q + h;
                    const int m = v / SW;
                    if ((v % SW) == s && m < M)
                        red[((b * M + m) * R + r) * SW + s] = acc[mt][b][2 * h] + acc[mt][b][2 * h + 1];
                }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        auto total = [&](int b, int m, int rr) {  // planes in order, segments in order
            float v = 0.0f;
#pragma unroll
            for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                for (int s2 = 0; s2 < SW; ++s2) v += red[((b * M + pl * Mo + m) * R + rr) * SW + s2];
            return v;
        };
        if constexpr (PAIRED) {
            for (int o = lane; o < Mo * R; o += 64) {  // 64 % R == 0: row r = lane % R
                const int m = o / R, rr = o % R;
                const int i = blockIdx.x * (WR * R) + wr * R + rr;
                if (i < a.I) store_silu_planes(a.y, m, i, Mo, a.I, total(0, m, rr) + bias_of(0), total(1, m, rr) + bias_of(1));
            }
        } else {
#pragma unroll
            for (int b = 0; b < RBW; ++b)
                for (int o = lane; o < Mo * R; o += 64) {
                    const int m = o / R, rr = o % R;
                    const int n = rowof(b, rr);
                    if (n < N) emit(m, n, total(b, m, rr), b);
                }
        }
    } else {
        float* red = (float*)(smem + L.red);  // [WK][M][RWG][SW]
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int b = 0; b < RBW; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int v = 8 * mt + 2 * q + h;
                    const int m = v / SW;
                    if ((v % SW) == s && m < M) {
                        const int wrow = (b * WR + wr) * R + r;
                        red[((wk * M + m) * RWG + wrow) * SW + s] = acc[mt][b][2 * h] + acc[mt][b][2 * h + 1];
                    }
                }
        lds_barrier();
        for (int o = tid; o < Mo * RWG; o += kThreads) {
            const int m = o / RWG, wrow = o % RWG;
            const int n = row0 + wrow;
            if (n < N) {
                float v = 0.0f;
#pragma unroll
                for (int k2 = 0; k2 < WK; ++k2)
#pragma unroll
                    for (int pl = 0; pl < PL; ++pl)
#pragma unroll
                        for (int s2 = 0; s2 < SW; ++s2) v += red[((k2 * M + pl * Mo + m) * RWG + wrow) * SW + s2];
                emit(m, n, v, 0);
            }
        }
    }
    W4G64_STAMP(4);
    W4G64_TIMELINE_STORE(a);
}

// ---- instantiations ----
// (SW, MT, WR, WK, RBW, T, DP, STG): the shapes the planner produces.
#define W4G64_PIPE_SHAPES(X)   \
    X(8, 1, 4, 1, 2, 9, 2, 5)  \
    X(8, 1, 4, 1, 1, 9, 5, 5)  \
    X(4, 1, 4, 1, 2, 3, 3, 1)  \
    X(4, 1, 1, 3, 1, 1, 1, 1)  \
    X(4, 1, 4, 1, 1, 3, 3, 1)  \
    X(8, 1, 4, 1, 1, 2, 2, 1)  \
    X(4, 1, 2, 4, 1, 5, 3, 5)  \
    X(2, 1, 1, 12, 1, 3, 2, 6) \
    X(2, 1, 4, 1, 2, 6, 3, 3)  \
    X(2, 1, 2, 2, 1, 3, 3, 3)  \
    X(1, 1, 1, 7, 1, 2, 2, 4)  \
    X(1, 1, 1, 4, 1, 3, 3, 6)  \
    X(1, 2, 2, 7, 1, 2, 2, 4)  \
    X(1, 2, 4, 2, 1, 6, 3, 6)  \
    X(1, 2, 1, 12, 1, 1, 1, 4)

// The fused forms of the decode step (bf16): (FORM, PAIRED, SW, MT, WR, WK,
// RBW, T, DP, STG).
#define W4G64_PIPE_FUSED_SHAPES(X)                   \
    X(kNormBf16, true, 4, 1, 4, 1, 2, 3, 2, 1)       \
    X(kPlain, true, 4, 1, 4, 1, 2, 3, 3, 1)          \
    X(kNormParts, false, 8, 1, 4, 1, 1, 2, 2, 1)     \
    X(kPlanes3, false, 2, 1, 4, 1, 1, 7, 4, 3)       \
    X(kAttnMerge, false, 8, 1, 4, 1, 1, 2, 2, 1)

// The grouped form (9..16 rows): (SW, MT, WR, WK, RBW, T, DP, STG).
#define W4G64_PIPE_GROUPED_SHAPES(X) \
    X(1, 1, 2, 7, 1, 2, 1, 4)        \
    X(1, 1, 4, 2, 1, 6, 2, 6)        \
    X(1, 1, 1, 12, 1, 1, 1, 4)

typedef void (*PipeKernel)(PipeArgs);
struct PipeEntry {
    int form, paired, sw, mt, wr, wk, rbw, t, dp, stg;
    PipeKernel f16, bf16;
};

#define W4G64_PIPE_ENTRY(SW, MT, WR, WK, RBW, T, DP, STG)                                              \
    {kPlain, 0, SW, MT, WR, WK, RBW, T, DP, STG,                                                       \
     gemv_pipe_kernel<kF16, kPlain, false, SW, MT, WR, WK, RBW, T, DP, STG>,                           \
     gemv_pipe_kernel<kBF16, kPlain, false, SW, MT, WR, WK, RBW, T, DP, STG>},
#define W4G64_PIPE_GROUPED_ENTRY(SW, MT, WR, WK, RBW, T, DP, STG)                                      \
    {kGrouped, 0, SW, MT, WR, WK, RBW, T, DP, STG,                                                     \
     gemv_pipe_kernel<kF16, kGrouped, false, SW, MT, WR, WK, RBW, T, DP, STG>,                         \
     gemv_pipe_kernel<kBF16, kGrouped, false, SW, MT, WR, WK, RBW, T, DP, STG>},
#define W4G64_PIPE_FUSED_ENTRY(FORM, PAIRED, SW, MT, WR, WK, RBW, T, DP, STG)                          \
    {FORM, PAIRED ? 1 : 0, SW, MT, WR, WK, RBW, T, DP, STG, nullptr,                                   \
     gemv_pipe_kernel<kBF16, FORM, PAIRED, SW, MT, WR, WK, RBW, T, DP, STG>},

const PipeEntry kPipeTable[] = {
    W4G64_PIPE_SHAPES(W4G64_PIPE_ENTRY)
    W4G64_PIPE_FUSED_SHAPES(W4G64_PIPE_FUSED_ENTRY)
    W4G64_PIPE_GROUPED_SHAPES(W4G64_PIPE_GROUPED_ENTRY)
#ifdef W4G64_PIPE_EXTRA_SHAPES  // tuning builds: more shapes, fp16 only
#define W4G64_PIPE_ENTRY_F16(SW, MT, WR, WK, RBW, T, DP, STG) \
    {kPlain, 0, SW, MT, WR, WK, RBW, T, DP, STG, gemv_pipe_kernel<kF16, kPlain, false, SW, MT, WR, WK, RBW, T, DP, STG>, nullptr},
    W4G64_PIPE_EXTRA_SHAPES(W4G64_PIPE_ENTRY_F16)
#endif
#ifdef W4G64_PIPE_EXTRA_FUSED_SHAPES  // tuning builds: more fused shapes
    W4G64_PIPE_EXTRA_FUSED_SHAPES(W4G64_PIPE_FUSED_ENTRY)
#endif
#ifdef W4G64_PIPE_EXTRA_GROUPED_SHAPES  // tuning builds: more grouped shapes, fp16 only
#define W4G64_PIPE_GROUPED_ENTRY_F16(SW, MT, WR, WK, RBW, T, DP, STG) \
    {kGrouped, 0, SW, MT, WR, WK, RBW, T, DP, STG, gemv_pipe_kernel<kF16, kGrouped, false, SW, MT, WR, WK, RBW, T, DP, STG>, nullptr},
    W4G64_PIPE_EXTRA_GROUPED_SHAPES(W4G64_PIPE_GROUPED_ENTRY_F16)
#endif
};

const PipeEntry* find_pipe(const GemvPlan& plan) {
    for (const PipeEntry& e : kPipeTable)
        if (e.form == plan.form && e.paired == plan.pair && e.sw == plan.segments && e.mt == plan.tiles &&
            e.wr == plan.fblocks && e.wk == plan.kparts && e.rbw == plan.rbw && e.t == plan.steps &&
            e.dp == plan.depth && e.stg == plan.stage)
            return &e;
    return nullptr;
}

}  // namespace

constexpr int64_t kPipeMaxLds = 160 * 1024;  // gfx950: the whole LDS of a CU per workgroup

// Fills the derived fields of a pipelined plan (tiles, blocks, splits, LDS,
// workspace, staging loads) from its shape and form; false if it does not
// fit.
bool finish_pipe_plan(int64_t rows, int64_t out_features, int64_t in_features, GemvPlan& plan) {
    const int64_t P = in_features / 128;
    const int sw = plan.segments, wr = plan.fblocks, wk = plan.kparts, rbw = plan.rbw, t = plan.steps;
    if (rows < 1 || rows > kGemvMaxRows || in_features % 128 || sw < 1 || 16 % sw) return false;
    const int64_t staged = rows * (plan.form == kPlanes3 ? 3 : 1);
    if (plan.form == kGrouped ? (sw != 1 || plan.tiles != 1 || plan.pair || staged > 16)
                              : 2 * staged * sw > 16 * plan.tiles)
        return false;
    const bool norm = plan.form == kNormBf16 || plan.form == kNormParts;
    const bool merge = plan.form == kAttnMerge;
    if ((norm || merge) && rows != 1) return false;
    if (plan.pair && (rbw != 2 || wk != 1 || out_features % 2)) return false;
    const int64_t span = (int64_t)wk * sw * t;  // pairs per workgroup K range
    const int64_t splits = (P + span - 1) / span;
    if ((norm || merge || plan.pair) && splits != 1) return false;  // the whole row, the whole (gate, up) pair
    plan.splits = (int)splits;
    plan.groups_per_split = (int)span;  // pairs per split (PS)
    const int64_t rows_per_block = (int64_t)wr * (16 / sw);
    plan.n_blocks = plan.pair ? (int)((out_features / 2 + rows_per_block - 1) / rows_per_block)
                              : (int)((out_features + rows_per_block * rbw - 1) / (rows_per_block * rbw));
    const int64_t items = staged * (span < P ? span : P) * 16;
    const int64_t threads = (int64_t)wr * wk * 64;
    if (items > (int64_t)plan.stage * threads) return false;
    const int red = pipe_red_floats((int)staged, sw, wr, wk, rbw, sw == 1 && plan.form != kPlanes3 && !plan.pair);
    plan.lds_bytes = pipe_layout((int)staged, (int)span, red).total;
    if (merge) {  // the chunk scales [rows heads][kAttnMergeMaxChunks] after the layout
        if (in_features % kAttnHeadDim) return false;
        plan.lds_bytes += (int)(rows * (in_features / kAttnHeadDim) * kAttnMergeMaxChunks * 4);
    }
    if (plan.lds_bytes > kPipeMaxLds) return false;
    plan.workspace_bytes = splits > 1 ? splits * rows * out_features * 4 : 0;
    plan.kind = 4;
    return true;
}

// Launch shapes by rows, pairs (K / 128) and out_features, first match
// first: (SW, MT, WR, WK, RBW, T, DP); the staging loads per lane are the
// smallest instantiated count that fits.  Chosen from forced-shape sweeps
// over cold weights, graph-replayed (decode calls) and one launch over a
// 28-layer stack (steady state): one row, gate 8960x1536 4.3 us, down
// 1536x8960 4.6 us, the stacked gate|up 5.7 TB/s and down 4.5 TB/s; 16
// rows, gate 6.4 us, down 8.5 us (five K splits and the reduction; shapes
// with 64-128 rows and 4-10 pairs per workgroup, 10-18 K splits, measured
// 9.2-10.9 us).  A K range longer than a shape's span is split across
// workgroups.
struct PipeShape {
    int min_rows, max_rows;
    int64_t min_pairs, max_pairs;
    int64_t min_n, max_n;
    int sw, mt, wr, wk, rbw, t, dp;
    int form = kPlain;
};
constexpr int64_t kAnyN = int64_t(1) << 40;
const PipeShape kPipeShapes[] = {
    // one row: long K (span 72); past 32768 outputs two row blocks per wave
    // (a 43008x8960 stack 47.1 -> 43.6 us)
    {1, 1, 48, 1 << 20, 32768, kAnyN, 8, 1, 4, 1, 2, 9, 2},
    {1, 1, 48, 1 << 20, 1, kAnyN, 8, 1, 4, 1, 1, 9, 5},
    // one row: span 12
    {1, 1, 1, 47, 32768, kAnyN, 4, 1, 4, 1, 2, 3, 3},
    {1, 1, 1, 47, 1, 512, 4, 1, 1, 3, 1, 1, 1},
    {1, 1, 1, 47, 1, 2048, 8, 1, 4, 1, 1, 2, 2},  // q/o 1536x1536 3.11 -> 2.99 us
    {1, 1, 1, 47, 1, kAnyN, 4, 1, 4, 1, 1, 3, 3},
    // 2..4 rows: long K in one workgroup (72 or 80 pairs), no split-K
    // reduction launch (down 1536x8960: 2 rows 7.3 -> 5.0 us, 4 rows 7.3 ->
    // 6.2; two segments, one A tile and two chunks in flight: 4 rows 6.4 ->
    // 5.6 us)
    {2, 2, 48, 1 << 20, 1, kAnyN, 4, 1, 2, 4, 1, 5, 3},
    {3, 4, 48, 1 << 20, 1, kAnyN, 2, 1, 1, 12, 1, 3, 2},
    {2, 4, 1, 47, 32768, kAnyN, 2, 1, 4, 1, 2, 6, 3},
    {2, 4, 1, 47, 1, kAnyN, 2, 1, 2, 2, 1, 3, 3},
    // 5..8 rows
    {5, 8, 48, 1 << 20, 1, kAnyN, 1, 1, 1, 7, 1, 2, 2},
    {5, 8, 1, 47, 1, kAnyN, 1, 1, 1, 4, 1, 3, 3},
    // 9..16 rows: one group per MFMA (fewer chunks in flight: down 8.5 ->
    // 8.15 us, gate 6.54 -> 6.43)
    {9, 16, 48, 1 << 20, 1, kAnyN, 1, 1, 2, 7, 1, 2, 1, kGrouped},
    {9, 16, 1, 47, 4096, kAnyN, 1, 1, 4, 2, 1, 6, 2, kGrouped},
    {9, 16, 1, 47, 1, kAnyN, 1, 1, 1, 12, 1, 1, 1, kGrouped},
};

bool plan_pipe(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, GemvPlan& plan) {
    if ((x_kind != kF16 && x_kind != kBF16) || in_features % 128 || rows < 1 || rows > kGemvMaxRows) return false;
    const int64_t P = in_features / 128;
    for (const PipeShape& sh : kPipeShapes) {
        if (rows < sh.min_rows || rows > sh.max_rows || P < sh.min_pairs || P > sh.max_pairs ||
            out_features < sh.min_n || out_features > sh.max_n)
            continue;
        const PipeEntry* best = nullptr;
        for (const PipeEntry& e : kPipeTable) {
            if (e.form != sh.form || e.paired || e.sw != sh.sw || e.mt != sh.mt || e.wr != sh.wr || e.wk != sh.wk ||
                e.rbw != sh.rbw || e.t != sh.t || e.dp != sh.dp || !e.bf16 || !e.f16)
                continue;
            GemvPlan cand{};
            cand.form = e.form;
            cand.segments = e.sw;
            cand.tiles = e.mt;
            cand.fblocks = e.wr;
            cand.kparts = e.wk;
            cand.rbw = e.rbw;
            cand.steps = e.t;
            cand.depth = e.dp;
            cand.stage = e.stg;
            if (finish_pipe_plan(rows, out_features, in_features, cand) && (!best || e.stg < best->stg)) {
                best = &e;
                plan = cand;
            }
        }
        if (best) return true;
    }
    return false;
}

// The decode step's fused forms (bf16, out_features rows; paired: gate rows
// then up rows): one shape each, from forced-shape sweeps of the Qwen2-1.5B
// decode step at one row over cold weights, graph-replayed: RMSNorm + gate|up
// 17920x1536 6.8 us (7.3 with three chunks in flight per row block; two,
// since the segment sums moved into registers: decode 0.840 -> 0.833 ms per
// token), the
// planes down projection 1536x8960 into five partial sums 4.4 us (5.3 with
// seven K parts per workgroup), RMSNorm over five partial sums + q|k|v
// 2048x1536 4.1 us (4.6 with three K parts).  RMSNorm + q|k|v and the
// attention-merge o_proj take 8 segments and two steps per wave, whose
// segment sums stay in registers (decode 0.849 -> 0.841 ms per token; the
// paired forms at 8 segments: 0.855-0.861).  The RMSNorm and paired forms
// need the whole K range in one workgroup.
struct PipeFusedShape {
    int form;
    bool paired;
    int min_rows, max_rows;
    int64_t max_pairs;
    int sw, mt, wr, wk, rbw, t, dp;
};
const PipeFusedShape kPipeFusedShapes[] = {
    {kNormBf16, true, 1, 1, 12, 4, 1, 4, 1, 2, 3, 2},
    {kPlain, true, 1, 1, 12, 4, 1, 4, 1, 2, 3, 3},
    {kNormParts, false, 1, 1, 12, 8, 1, 4, 1, 1, 2, 2},
    {kPlanes3, false, 1, 1, 1 << 20, 2, 1, 4, 1, 1, 7, 4},
    {kAttnMerge, false, 1, 1, 12, 8, 1, 4, 1, 1, 2, 2},
};

bool plan_pipe_fused(int form, bool paired, int64_t rows, int64_t out_features, int64_t in_features,
                     GemvPlan& plan) {
    if (in_features % 256) return false;
    const int64_t P = in_features / 128;
    for (const PipeFusedShape& sh : kPipeFusedShapes) {
        if (sh.form != form || sh.paired != paired || rows < sh.min_rows || rows > sh.max_rows || P > sh.max_pairs)
            continue;
        const PipeEntry* best = nullptr;
        for (const PipeEntry& e : kPipeTable) {
            if (e.form != form || e.paired != (paired ? 1 : 0) || e.sw != sh.sw || e.mt != sh.mt || e.wr != sh.wr ||
                e.wk != sh.wk || e.rbw != sh.rbw || e.t != sh.t || e.dp != sh.dp || !e.bf16)
                continue;
            GemvPlan cand{};
            cand.form = form;
            cand.pair = paired ? 1 : 0;
            cand.segments = e.sw;
            cand.tiles = e.mt;
            cand.fblocks = e.wr;
            cand.kparts = e.wk;
            cand.rbw = e.rbw;
            cand.steps = e.t;
            cand.depth = e.dp;
            cand.stage = e.stg;
            if (finish_pipe_plan(rows, out_features, in_features, cand) && (!best || e.stg < best->stg)) {
                best = &e;
                plan = cand;
            }
        }
        if (best) return true;
    }
    return false;
}

bool pipe_supported(const LinearProblem& p) {
    // zero bytes are read as the aligned 16-bit words holding them: with an
    // even pair count per row (in_features a multiple of 256) every row's
    // bytes start at an even index, and no word reaches past its row
    const bool norm = p.x_kind == kNormB || p.x_kind == kNormP || p.x_kind == kNormF;
    if (!(p.x_kind == kF16 || p.x_kind == kBF16 || p.x_kind == kPlanes || p.x_kind == kAttnM || norm)) return false;
    if (p.x_kind == kAttnM && (p.att_chunks < 1 || p.att_chunks > kAttnMergeMaxChunks || p.att_group < 1 ||
                               p.att_group > kAttnMaxGroup || p.att_kv_heads < 1 ||
                               p.in_features != (int64_t)p.att_group * p.att_kv_heads * kAttnHeadDim))
        return false;
    if (p.paired && p.x_kind == kF16) return false;  // the fused forms are bf16
    if (norm &&
        (((uintptr_t)p.norm_delta % 16) || ((uintptr_t)p.norm_weight % 16) || ((uintptr_t)p.norm_out_sum % 16)))
        return false;
    return p.in_features % 256 == 0 && ((uintptr_t)p.qweight % 16) == 0 && ((uintptr_t)p.x % 16) == 0 &&
           ((uintptr_t)p.scales % 4) == 0 && ((uintptr_t)p.zeros % 2) == 0;
}

bool pipe_plan_launchable(const GemvPlan& plan) { return find_pipe(plan) != nullptr; }

hipError_t launch_gemv_pipe(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                            hipEvent_t start, hipEvent_t stop) {
    const PipeEntry* e = find_pipe(plan);
    if (!e || plan.kind != 4) return hipErrorInvalidValue;
    PipeArgs a{};
    a.x = p.x;
    a.qweight = p.qweight;
    a.scales = p.scales;
    a.zeros = p.zeros;
    a.bias = p.bias;
    a.bias_kind = p.bias_kind;
    a.y = p.y;
    a.Mo = (int)p.rows;
    a.M = (int)p.rows * (plan.form == kPlanes3 ? 3 : 1);
    a.N = (int)p.out_features;
    a.I = (int)(p.out_features / 2);
    a.delta = p.norm_delta;
    a.delta_parts = p.norm_delta_parts;
    a.norm_w = p.norm_weight;
    a.eps = p.norm_eps;
    a.out_sum = (uint16_t*)p.norm_out_sum;
    a.att_chunks = p.att_chunks;
    a.att_group = p.att_group;
    a.att_bytes = (int)((int64_t)p.att_kv_heads * p.att_chunks * kAttnPartFloats * 4);
    a.att_ginv = p.att_group > 0 ? 1.0f / (float)p.att_group : 0.0f;
    a.K = (int)p.in_features;
    a.G = a.K / 64;
    a.P = a.G / 2;
    a.PS = plan.groups_per_split;
    W4G64_TIMELINE_SET(a);
    const bool unreduced = p.partials_out != nullptr;
    const bool split = plan.splits > 1 && !unreduced;
    a.partials = unreduced ? p.partials_out : (plan.splits > 1 ? (float*)workspace : nullptr);
    if (plan.splits > 1 && !a.partials) return hipErrorInvalidValue;
    PipeKernel k = p.x_kind == kF16 ? e->f16 : e->bf16;
    if (!k || (plan.pair != 0) != (p.paired != 0)) return hipErrorInvalidValue;
    // an fp32 delta is the one-part case of the partial-sums form
    const int want_form = p.x_kind == kPlanes                       ? kPlanes3
                          : p.x_kind == kAttnM                      ? kAttnMerge
                          : p.x_kind == kNormB                      ? kNormBf16
                          : (p.x_kind == kNormP || p.x_kind == kNormF) ? kNormParts
                                                                      : kPlain;
    const bool form_ok = want_form == plan.form || (want_form == kPlain && plan.form == kGrouped);
    if (!form_ok || (plan.pair && (split || unreduced))) return hipErrorInvalidValue;
    const dim3 grid(plan.n_blocks, plan.splits), block(plan.fblocks * plan.kparts * 64);
    hipError_t err = launch_kernel(k, grid, block, (size_t)plan.lds_bytes, stream, start, split ? nullptr : stop, a);
    if (err != hipSuccess || !split) return err;
    return launch_split_reduce(a.partials, p.bias, p.bias_kind, p.y, a.Mo, a.N, plan.splits, false,
                               plan.form == kPlanes3 ? kF32 : p.x_kind, stream, stop);
}

}  // namespace w4g64
