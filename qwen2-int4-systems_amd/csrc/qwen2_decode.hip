// Fused decode-step kernels between the W4G64 linears of a Qwen2 decoder
// layer (C ABI in include/qwen2_decode.h).  One token per sequence, bf16
// hidden states; each kernel restates a block of src/qwen_int4/model.py with
// the reference's roundings:
//
//   add_rmsnorm_kernel  one workgroup per row: residual add, fp32 sum of
//                       squares, bf16(bf16(s * rsqrt(mean + eps)) * w)
//                       (model.py:40-44, :149-154).
//   attention_kernel    one workgroup per (sequence, key/value head, chunk of
//                       64 positions).  It rotates the group's query heads
//                       (and, in the chunk that holds the new position, the
//                       new key, which it also writes to the cache with the
//                       new value), stages the chunk's keys and values in LDS
//                       (16-byte loads, rows padded to 272 B), computes fp32
//                       scores, the chunk's softmax maximum and sum and its
//                       probability-weighted value sums.  The last workgroup
//                       of a (sequence, head) to arrive merges the chunks
//                       (rescaled by exp(m_chunk - m)) and writes bf16
//                       (model.py:61-122).
//   prefill_rope_kernel, prefill_attention_kernel
//                       a prompt: rotary of every position (queries to a
//                       workspace, keys and values into the caches), then
//                       causal GQA attention, one workgroup per (sequence,
//                       head, 64 query rows) over 64-key blocks staged in LDS,
//                       online softmax (model.py:17-31, :61-122).
//   silu_mul_kernel     silu(gate) * up in fp32 (model.py:133-136).
//
// The new key at position p is read by the chunk that holds p from LDS, never
// from the cache, so no workgroup reads a cache row another one is writing.
#include <math.h>
#include <stdarg.h>

#include "../../include/qwen2_decode.h"
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kNormThreads = 256;
constexpr int kNormIters = 4;  // hidden <= 256 threads x 8 elements x 4 = 8192

constexpr int kHeadDim = 128;
constexpr int kChunk = 64;        // positions per attention workgroup (one per lane of a wave)
constexpr int kMaxGroup = 8;      // query heads per key/value head
constexpr int kAttnThreads = 256;
constexpr int kRowStride = kHeadDim + 8;  // bf16 elements per staged row (272 B)
constexpr int kPartFloats = 2 * kMaxGroup + kMaxGroup * kHeadDim;  // m[8], l[8], acc[8][128]
static_assert(kPartFloats == kAttnPartFloats && kChunk == kAttnChunk && kMaxGroup == kAttnMaxGroup &&
                  kHeadDim == kAttnHeadDim,
              "the partial-result layout the attention-merge GEMV reads");
constexpr int kMergeBatch = 16;   // chunks whose partial sums one merge pass loads together
// The merge keeps per-chunk statistics in the staging rows' LDS.
constexpr int kMaxChunks = (kChunk * kRowStride * 2) / (2 * kMaxGroup * 4);
constexpr int kMaxLength = kMaxChunks * kChunk;


// Thread t owns the 8-element pieces 8 t + 2048 i (i < kNormIters).  Every
// load is unconditional at a clamped address and issued before any use (a
// guarded load would be waited for on its own); pieces past the row end are
// masked out of the sum and not stored.
// delta_kind kNormP: delta holds delta_parts fp32 partial sums [parts][rows][hidden]
// of a split-K projection, added in order from 0 and then + 0 (no bias): the
// value the split-K reduction would have stored as an fp32 delta.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const uint16_t* x, const void* delta,
                                                                   int delta_kind, int delta_parts,
                                                                   const uint16_t* weight, float eps,
                                                                   uint16_t* out_sum, uint16_t* out_norm,
                                                                   int hidden) {
    constexpr int kStride = kNormThreads * 8;
    const int64_t base = (int64_t)blockIdx.x * hidden;
    int col[kNormIters];
    u32x4 xr[kNormIters], wr[kNormIters], dr[kNormIters][2];
#pragma unroll
    for (int i = 0; i < kNormIters; ++i) {
        col[i] = 8 * (int)threadIdx.x + kStride * i;
        const int c = min(col[i], hidden - 8);
        xr[i] = *(const u32x4*)(x + base + c);
        wr[i] = *(const u32x4*)(weight + c);
        if (delta_kind == kBF16) {
            dr[i][0] = *(const u32x4*)((const uint16_t*)delta + base + c);
        } else if (delta_kind == kF32) {
            dr[i][0] = *(const u32x4*)((const float*)delta + base + c);
            dr[i][1] = *(const u32x4*)((const float*)delta + base + c + 4);
        }
    }
    if (delta_kind == kNormP) {
        const int64_t part_stride = (int64_t)gridDim.x * hidden;
#pragma unroll
        for (int i = 0; i < kNormIters; ++i) {
            const int c = min(col[i], hidden - 8);
            float t[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int pt = 0; pt < delta_parts; ++pt) {
                const float* src = (const float*)delta + pt * part_stride + base + c;
                const float4v lo = *(const float4v*)src, hi = *(const float4v*)(src + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    t[e] += lo[e];
                    t[4 + e] += hi[e];
                }
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dr[i][0][e] = __builtin_bit_cast(uint32_t, t[e] + 0.0f);
                dr[i][1][e] = __builtin_bit_cast(uint32_t, t[4 + e] + 0.0f);
            }
        }
    }
    float v[kNormIters][8];
    float sq = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormIters; ++i) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t xw = xr[i][e / 2];
            float s = bf16_bits_to_float(e & 1 ? xw >> 16 : xw & 0xFFFFu);
            if (delta_kind == kBF16) {
                const uint32_t dw = dr[i][0][e / 2];
                s = bf16_round(s + bf16_bits_to_float(e & 1 ? dw >> 16 : dw & 0xFFFFu));
            } else if (delta_kind == kF32 || delta_kind == kNormP) {
                // (a scalar copy first: bit_cast of a vector element lvalue reads element 0)
                const uint32_t bits = dr[i][e / 4][e % 4];
                s = bf16_round(s + bf16_round(__builtin_bit_cast(float, bits)));
            }
            v[i][e] = s;
            // the square is rounded before it is summed, as x.pow(2) is
            if (col[i] < hidden) sq += __fmul_rn(s, s);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    __shared__ float red[kNormThreads / 64];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sq;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kNormThreads / 64; ++w) total += red[w];
    const float r = rsqrtf(total / (float)hidden + eps);
#pragma unroll
    for (int i = 0; i < kNormIters; ++i) {
        if (col[i] >= hidden) continue;
        u32x4 so, no;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t ww = wr[i][e / 2];
            const float n0 = bf16_round(v[i][e] * r) * bf16_bits_to_float(ww & 0xFFFFu);
            const float n1 = bf16_round(v[i][e + 1] * r) * bf16_bits_to_float(ww >> 16);
            so[e / 2] = float_to_bf16_bits(v[i][e]) | ((uint32_t)float_to_bf16_bits(v[i][e + 1]) << 16);
            no[e / 2] = float_to_bf16_bits(n0) | ((uint32_t)float_to_bf16_bits(n1) << 16);
        }
        if (out_sum) *(u32x4*)(out_sum + base + col[i]) = so;
        *(u32x4*)(out_norm + base + col[i]) = no;
    }
}

struct AttnArgs {
    const uint16_t* qkv;
    const uint16_t* cos;
    const uint16_t* sin;
    uint16_t* k_cache;
    uint16_t* v_cache;
    const int64_t* position;
    uint16_t* out;
    int heads;
    int kv_heads;
    int max_len;
    int chunks;
    float scale;
    unsigned* counters;  // [batch * kv_heads]
    float* partials;     // [batch * kv_heads][chunks][kPartFloats]
    // nonzero: no merge -- every chunk's workgroup stores its partial result
    // (a chunk past the position an empty one: m = -inf, l = 0, sums 0) and
    // the next launch merges them (w4g64_linear_attention_merge)
    int unmerged;
    W4G64_TIMELINE_FIELDS
};

// Element d of the rotated head vector: x * cos + rotate_half(x) * sin, with
// rotate_half(x)[d] = -x[d + D/2] (d < D/2) or x[d - D/2], each product and
// the sum rounded to bf16 (bf16 tensor arithmetic, model.py:17-19, :76-77).
// x = vec[d], other = vec[d ^ D/2], c = cos[d], n = sin[d] (bf16 bits).
__device__ __forceinline__ float rope_elem(uint16_t x, uint16_t other, uint16_t c, uint16_t n, int d) {
    const float partner = d < kHeadDim / 2 ? -bf16_bits_to_float(other) : bf16_bits_to_float(other);
    const float a = bf16_round(bf16_bits_to_float(x) * bf16_bits_to_float(c));
    const float b = bf16_round(partner * bf16_bits_to_float(n));
    return bf16_round(a + b);
}

// Wave-wide max / sum by DPP (quad swaps, half-row and row mirrors, row
// broadcasts 15 and 31: lane 63 ends with the result), then a read of lane 63.
__device__ __forceinline__ float dpp_step(float v, int ctrl_kind) {
    const int x = __builtin_bit_cast(int, v);
    int y;
    switch (ctrl_kind) {
        case 0: y = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
        case 1: y = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
        case 2: y = __builtin_amdgcn_update_dpp(x, x, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
        case 3: y = __builtin_amdgcn_update_dpp(x, x, 0x140, 0xF, 0xF, false); break;  // row_mirror
        case 4: y = __builtin_amdgcn_update_dpp(x, x, 0x142, 0xA, 0xF, false); break;  // row_bcast15 -> rows 1, 3
        default: y = __builtin_amdgcn_update_dpp(x, x, 0x143, 0xC, 0xF, false); break; // row_bcast31 -> rows 2, 3
    }
    return __builtin_bit_cast(float, y);
}
__device__ __forceinline__ float wave_max(float v) {
    // lanes outside a row mask receive `old` = their own value: max is unchanged
#pragma unroll
    for (int k = 0; k < 6; ++k) v = fmaxf(v, dpp_step(v, k));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int k = 0; k < 4; ++k) v += dpp_step(v, k);  // every lane: its row's sum
    // rows 1 and 3 add the sums of rows 0 and 2, then rows 2 and 3 add row 1's
    // (lanes outside the row mask receive the `old` operand, 0)
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// MFMA layout (v_mfma_f32_16x16x32_bf16): lane l = 16 q + j supplies A row j
// and B column j with the 8 values of K slots [8 q, 8 q + 8); it receives
// D[4 q + r][j], r < 4.
//   scores: A = rotated queries (row = head, K = dimension), B = staged keys
//           (column = position): wave w scores positions 16 w .. 16 w + 15,
//           four MFMAs over the 128 dimensions;
//   sums:   A = probabilities (row = head, K = position), split exactly enough
//           into bf16 hi + lo, B = staged values transposed (column =
//           dimension): wave w owns dimensions 32 w .. 32 w + 31, eight MFMAs.
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t qsb[16][kRowStride];     // rotated queries, bf16
    __shared__ __attribute__((aligned(16))) uint16_t ks[kChunk][kRowStride];  // keys [position][dim]
    __shared__ __attribute__((aligned(16))) uint16_t vt[kHeadDim][kChunk + 8];  // values [dim][position]
    __shared__ __attribute__((aligned(16))) float pr[kMaxGroup][kChunk + 4];    // scores, then exp(s - m)
    __shared__ float stat_m[kMaxGroup];
    __shared__ float stat_l[kMaxGroup];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int chunk = blockIdx.x % a.chunks;
    const int kvh = (blockIdx.x / a.chunks) % a.kv_heads;
    const int b = blockIdx.x / (a.chunks * a.kv_heads);
    const int group = a.heads / a.kv_heads;
    const uint16_t* qkv = a.qkv + (int64_t)b * (a.heads + 2 * a.kv_heads) * kHeadDim;
    const uint16_t* cs = a.cos + (int64_t)b * kHeadDim;
    const uint16_t* sn = a.sin + (int64_t)b * kHeadDim;
    const int slot = b * a.kv_heads + kvh;
    const int64_t cache_base = (int64_t)slot * a.max_len * kHeadDim;
    float* part = a.partials + ((int64_t)slot * a.chunks + chunk) * kPartFloats;
    const int mj = lane & 15;  // MFMA row / column of this lane
    const int mq = lane >> 4;  // MFMA K-slot quarter of this lane
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);

    // ---- loads that do not depend on the position: queries, rotary factors, new key/value ----
    // Thread t: dimensions qd = 8 (t % 16) .. qd + 7 (and their rotate_half
    // partners qd ^ 64 ..) of query head t / 16 of the group (threads past the
    // group re-read its last head), the rotary factors of those dimensions,
    // and -- used by threads t < 16 -- the same dimensions of the new key and
    // value: 16-byte loads.
    const int qg = tid / 16;
    const int qd = 8 * (tid % 16);
    const u32x4 qcv = *(const u32x4*)(cs + qd);
    const u32x4 qnv = *(const u32x4*)(sn + qd);
    const uint16_t* qvec = qkv + (kvh * group + min(qg, group - 1)) * kHeadDim;
    const u32x4 qxv = *(const u32x4*)(qvec + qd);
    const u32x4 qpv = *(const u32x4*)(qvec + (qd ^ (kHeadDim / 2)));
    const uint16_t* kvec = qkv + (a.heads + kvh) * kHeadDim;
    const u32x4 kxv = *(const u32x4*)(kvec + qd);
    const u32x4 kpv = *(const u32x4*)(kvec + (qd ^ (kHeadDim / 2)));
    const u32x4 vxv = *(const u32x4*)(qkv + (a.heads + a.kv_heads + kvh) * kHeadDim + qd);
    // 8 rotated dimensions qd .. qd + 7 of a head vector: rope_elem's
    // operations, two dimensions per bf16 conversion instruction (the 8
    // dimensions lie in one half of the head, so rotate_half's sign is one)
    const float rsign = qd < kHeadDim / 2 ? -1.0f : 1.0f;
    auto rope8 = [&](const u32x4& x, const u32x4& partner) {
        u32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t pa = pack_bf16x2(bf16_lo(x[e]) * bf16_lo(qcv[e]), bf16_hi(x[e]) * bf16_hi(qcv[e]));
            const uint32_t pb = pack_bf16x2((rsign * bf16_lo(partner[e])) * bf16_lo(qnv[e]),
                                            (rsign * bf16_hi(partner[e])) * bf16_hi(qnv[e]));
            r[e] = pack_bf16x2(bf16_lo(pa) + bf16_lo(pb), bf16_hi(pa) + bf16_hi(pb));
        }
        return r;
    };
    // The position is read first (its load returns before the chunk's), then
    // the chunk's 64 cache rows are loaded without waiting for it: rows past
    // the cache end re-read its last row, and rows at or past the position
    // are replaced (the new key and value, zero values) or masked below, so
    // no load address depends on the position.
    int64_t p64 = *a.position;
    asm volatile("" ::: "memory");
    const int t0 = chunk * kChunk;
    const int last_row = a.max_len - 1 - t0;  // >= 0: the launch covers max_len with chunks
    constexpr int kPieces = kChunk * (kHeadDim / 8) / kAttnThreads;
    static_assert(kPieces == 4 && kAttnThreads == 16 * (kHeadDim / 8), "value staging: 16 columns x 4 rows");
    // keys: piece e = tid + 256 i -> row e / 16, 16-byte column e % 16
    // (row-major LDS stores); values: thread t takes column vc = t / 16 of
    // the four rows 4 (t % 16) + i, so that it holds four consecutive
    // positions of 8 dimensions for the transposed stores
    const int vcol = tid / (kHeadDim / 8);
    const int vrow0 = kPieces * (tid % (kHeadDim / 8));
    u32x4 kr[kPieces], vr[kPieces];
#pragma unroll
    for (int i = 0; i < kPieces; ++i) {
        const int e = tid + kAttnThreads * i;
        const int r = min(e / (kHeadDim / 8), last_row);
        kr[i] = *(const u32x4*)(a.k_cache + cache_base + (int64_t)(t0 + r) * kHeadDim + 8 * (e % (kHeadDim / 8)));
        const int rv = min(vrow0 + i, last_row);
        vr[i] = *(const u32x4*)(a.v_cache + cache_base + (int64_t)(t0 + rv) * kHeadDim + 8 * vcol);
    }
    // the new value's 8 dimensions of column vcol (used when pos is in this chunk)
    const u32x4 vnew8 = *(const u32x4*)(qkv + (a.heads + a.kv_heads + kvh) * kHeadDim + 8 * vcol);
    p64 = p64 < 0 ? 0 : (p64 >= a.max_len ? a.max_len - 1 : p64);
    const int pos = (int)p64;
    const int nk = min(kChunk, pos + 1 - t0);  // positions of this chunk that are attended (<= 0: none)

    if (nk > 0) {
        // cached rows t0 .. t0 + cached - 1 are used as loaded
        const int cached = min(nk, pos - t0);
        if (qg < group) *(u32x4*)&qsb[qg][qd] = rope8(qxv, qpv);
        if (pos - t0 < kChunk && tid < kHeadDim / 8) {  // this chunk holds the new position
            const u32x4 kb = rope8(kxv, kpv);
            *(u32x4*)(a.k_cache + cache_base + (int64_t)pos * kHeadDim + qd) = kb;
            *(u32x4*)(a.v_cache + cache_base + (int64_t)pos * kHeadDim + qd) = vxv;
            *(u32x4*)&ks[pos - t0][qd] = kb;
        }
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int e = tid + kAttnThreads * i;
            const int r = e / (kHeadDim / 8);
            const int c = e % (kHeadDim / 8);
            if (r < cached) *(u32x4*)&ks[r][8 * c] = kr[i];
        }
        // values transposed, four positions per 8-byte store: cached rows,
        // the new value at pos, zeros past pos (their probability is 0)
        {
            u32x4 v4[kPieces];
#pragma unroll
            for (int i = 0; i < kPieces; ++i) {
                const int r = vrow0 + i;
                const u32x4 zero = {0u, 0u, 0u, 0u};
                v4[i] = r < cached ? vr[i] : (t0 + r == pos ? vnew8 : zero);
            }
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                const uint32_t sel = (h & 1) ? 0x07060302u : 0x05040100u;  // high or low halves
                const uint32_t p01 = __builtin_amdgcn_perm(v4[1][h / 2], v4[0][h / 2], sel);
                const uint32_t p23 = __builtin_amdgcn_perm(v4[3][h / 2], v4[2][h / 2], sel);
                *(u32x2*)&vt[8 * vcol + h][vrow0] = u32x2{p01, p23};
            }
        }
        __syncthreads();
        W4G64_STAMP(1);

        // ---- scores (MFMA): wave w, positions 16 w + mj ----
        {
            float4v sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int sl = 0; sl < kHeadDim / 32; ++sl) {
                const u32x4 av = *(const u32x4*)&qsb[mj][32 * sl + 8 * mq];
                const u32x4 bv = *(const u32x4*)&ks[16 * wave + mj][32 * sl + 8 * mq];
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av),
                                                               __builtin_bit_cast(bf16x8, bv), sacc, 0, 0, 0);
            }
            const int j = 16 * wave + mj;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int g = 4 * mq + r;
                if (g < group) pr[g][j] = j < nk ? sacc[r] * a.scale : -INFINITY;
            }
        }
        __syncthreads();
        W4G64_STAMP(2);

        // ---- chunk softmax statistics: wave w takes heads w and w + 4 side by
        // side (two independent chains); lane = position ----
        {
            static_assert(kMaxGroup <= 2 * (kAttnThreads / 64), "two heads per wave");
            const int g0 = wave, g1 = wave + kAttnThreads / 64;
            const bool has0 = g0 < group, has1 = g1 < group;  // uniform
            const float sv0 = pr[min(g0, group - 1)][lane];
            const float sv1 = pr[min(g1, group - 1)][lane];
            const float m0 = wave_max(sv0), m1 = wave_max(sv1);
            const float e0 = lane < nk ? expf(sv0 - m0) : 0.0f;
            const float e1 = lane < nk ? expf(sv1 - m1) : 0.0f;
            const float l0 = wave_sum(e0), l1 = wave_sum(e1);
            if (has0) pr[g0][lane] = e0;
            if (has1) pr[g1][lane] = e1;
            if (lane == 0) {
                if (has0) {
                    stat_m[g0] = m0;
                    stat_l[g0] = l0;
                }
                if (has1) {
                    stat_m[g1] = m1;
                    stat_l[g1] = l1;
                }
            }
        }
        __syncthreads();
        W4G64_STAMP(3);

        // ---- probability-weighted value sums (MFMA): wave w, dimensions 32 w .. 32 w + 31 ----
        float4v oacc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
        for (int sl = 0; sl < kChunk / 32; ++sl) {
            u32x4 phi = {0u, 0u, 0u, 0u}, plo = {0u, 0u, 0u, 0u};
            if (mj < group) {
                const float4v p0 = *(const float4v*)&pr[mj][32 * sl + 8 * mq];
                const float4v p1 = *(const float4v*)&pr[mj][32 * sl + 8 * mq + 4];
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float x0 = h < 2 ? p0[2 * h] : p1[2 * h - 4];
                    const float x1 = h < 2 ? p0[2 * h + 1] : p1[2 * h - 3];
                    const uint16_t h0 = float_to_bf16_bits(x0), h1 = float_to_bf16_bits(x1);
                    const uint16_t l0 = float_to_bf16_bits(x0 - bf16_bits_to_float(h0));
                    const uint16_t l1 = float_to_bf16_bits(x1 - bf16_bits_to_float(h1));
                    phi[h] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                    plo[h] = (uint32_t)l0 | ((uint32_t)l1 << 16);
                }
            }
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) {
                const u32x4 bv = *(const u32x4*)&vt[32 * wave + 16 * cb + mj][32 * sl + 8 * mq];
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, phi),
                                                                   __builtin_bit_cast(bf16x8, bv), oacc[cb], 0, 0, 0);
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, plo),
                                                                   __builtin_bit_cast(bf16x8, bv), oacc[cb], 0, 0, 0);
            }
        }
        // plain stores: the arrival below publishes them at agent scope (the
        // merging workgroup may run on another XCD)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int g = 4 * mq + r;
                if (g < group) part[2 * kMaxGroup + g * kHeadDim + 32 * wave + 16 * cb + mj] = oacc[cb][r];
            }
        if (tid < group) {
            part[tid] = stat_m[tid];
            part[kMaxGroup + tid] = stat_l[tid];
        }
    }

    W4G64_STAMP(4);
    if (a.unmerged) {
        // An empty chunk's partial adds exactly nothing to the merge:
        // exp(-inf - m) = 0 scales its zero sums and its zero l.
        if (nk <= 0)
            for (int e = tid; e < 2 * kMaxGroup + group * kHeadDim; e += kAttnThreads)
                part[e] = e < kMaxGroup ? -INFINITY : 0.0f;
        W4G64_STAMP(5);
        W4G64_TIMELINE_STORE(a);
        return;
    }
    // ---- arrival: the last workgroup of this (sequence, head) merges ----
    // The partial stores are published by the arrival's agent-scope release
    // and acquired by the last arriver (arrive_last).
    if (!arrive_last(a.counters + slot, (unsigned)a.chunks, &s_last)) {
        W4G64_STAMP(5);
        W4G64_TIMELINE_STORE(a);
        return;
    }
    W4G64_STAMP(5);
    // After the acquire, plain loads see every other workgroup's partials.
    // The merge issues them all at once: the statistics first (their loads
    // return first), then per thread t < group * 32 the weighted sums of head
    // t / 32, dimensions 4 (t % 32) .. + 3, of up to kMergeBatch chunks as
    // 16-byte loads.  Loads of chunks past `used` (or threads past the
    // group's heads) re-read a valid partial; their scale is zero (or their
    // result is not stored), so the accumulation needs no branches.
    const int used = pos / kChunk + 1;  // chunks that hold positions 0..pos (all wrote partials)
    const float* base = a.partials + (int64_t)slot * a.chunks * kPartFloats;
    float* stats = (float*)&ks[0][0];    // [used][2 * kMaxGroup]: m, l per head
    float* scale_c = (float*)&vt[0][0];  // [kMaxChunks][kMaxGroup]: exp(m_c - m) / l, zero past `used`
    for (int e = tid; e < used * 2 * kMaxGroup; e += kAttnThreads)
        stats[e] = base[(e / (2 * kMaxGroup)) * kPartFloats + e % (2 * kMaxGroup)];
    const int f = min(tid, group * (kHeadDim / 4) - 1);
    const int gh = f / (kHeadDim / 4);     // head within the group
    const int d4 = 4 * (f % (kHeadDim / 4));  // first of its four dimensions
    float4v v[kMergeBatch];
    auto load_batch = [&](int c0) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u)
            v[u] = *(const float4v*)(base + min(c0 + u, used - 1) * kPartFloats + 2 * kMaxGroup + gh * kHeadDim + d4);
    };
    load_batch(0);
    __syncthreads();
    // per head g (wave w takes heads w, w + 4): lanes walk the chunks; the
    // head's maximum and rescaled sum are wave reductions.  Heads past
    // `group` get zero scales.
    for (int g = wave; g < kMaxGroup; g += kAttnThreads / 64) {
        if (g >= group) {
            for (int c = lane; c < kMaxChunks; c += 64) scale_c[c * kMaxGroup + g] = 0.0f;
            continue;
        }
        float m = -INFINITY;
        for (int c = lane; c < used; c += 64) m = fmaxf(m, stats[c * 2 * kMaxGroup + g]);
        m = wave_max(m);
        float l = 0.0f;
        for (int c = lane; c < used; c += 64)
            l = fmaf(stats[c * 2 * kMaxGroup + kMaxGroup + g], expf(stats[c * 2 * kMaxGroup + g] - m), l);
        l = wave_sum(l);
        for (int c = lane; c < kMaxChunks; c += 64)
            scale_c[c * kMaxGroup + g] = c < used ? expf(stats[c * 2 * kMaxGroup + g] - m) / l : 0.0f;
    }
    __syncthreads();
    W4G64_STAMP(6);
    float4v o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < used; c0 += kMergeBatch) {
        if (c0 > 0) load_batch(c0);
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
            float sc = scale_c[min(c0 + u, kMaxChunks - 1) * kMaxGroup + gh];
            sc = c0 + u < used ? sc : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = fmaf(v[u][i], sc, o[i]);
        }
    }
    if (tid < group * (kHeadDim / 4)) {
        const uint32_t lo = float_to_bf16_bits(o[0]) | ((uint32_t)float_to_bf16_bits(o[1]) << 16);
        const uint32_t hi = float_to_bf16_bits(o[2]) | ((uint32_t)float_to_bf16_bits(o[3]) << 16);
        *(u32x2*)(a.out + (int64_t)b * a.heads * kHeadDim + (kvh * group + gh) * kHeadDim + d4) = u32x2{lo, hi};
    }
    if (tid == 0) __hip_atomic_store(a.counters + slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    W4G64_TIMELINE_STORE(a);
}

// Reduction over the 16 lanes of a row (quad swaps, half-row and row
// mirrors): every lane of the row ends with the row's result.
__device__ __forceinline__ float row16_max(float v) {
#pragma unroll
    for (int k = 0; k < 4; ++k) v = fmaxf(v, dpp_step(v, k));
    return v;
}
__device__ __forceinline__ float row16_sum(float v) {
#pragma unroll
    for (int k = 0; k < 4; ++k) v += dpp_step(v, k);
    return v;
}
// ---- prefill: rotary + cache write, then causal GQA attention over the prompt ----

struct PrefillArgs {
    const uint16_t* qkv;  // [batch * length][(heads + 2 kv_heads) * 128]
    const uint16_t* cos;  // [batch * length][128]
    const uint16_t* sin;
    uint16_t* k_cache;    // [batch][kv_heads][max_len][128]
    uint16_t* v_cache;
    uint16_t* qrot;       // [batch][heads][length][128] rotated queries (workspace)
    uint16_t* out;        // [batch * length][heads * 128]
    int length;
    int heads;
    int kv_heads;
    int max_len;
    float scale2;         // scale * log2(e): the softmax runs in base 2
};

constexpr int kPrefillBlock = 64;  // query rows per workgroup and keys per staged block

// One workgroup per (sequence, position): rotated query heads into qrot, the
// rotated key heads and the values into the caches (model.py:17-31, :76-77).
__global__ __launch_bounds__(256) void prefill_rope_kernel(PrefillArgs a) {
    const int row = blockIdx.x;  // b * length + i
    const int b = row / a.length;
    const int i = row - b * a.length;
    const int width = (a.heads + 2 * a.kv_heads) * kHeadDim;
    const uint16_t* src = a.qkv + (int64_t)row * width;
    const uint16_t* cs = a.cos + (int64_t)row * kHeadDim;
    const uint16_t* sn = a.sin + (int64_t)row * kHeadDim;
    for (int e = threadIdx.x; e < width; e += blockDim.x) {
        const int head = e / kHeadDim;  // query heads, then key heads, then value heads
        const int d = e % kHeadDim;
        if (head < a.heads) {
            const uint16_t* vec = src + head * kHeadDim;
            a.qrot[(((int64_t)b * a.heads + head) * a.length + i) * kHeadDim + d] =
                float_to_bf16_bits(rope_elem(vec[d], vec[d ^ (kHeadDim / 2)], cs[d], sn[d], d));
        } else if (head < a.heads + a.kv_heads) {
            const uint16_t* vec = src + head * kHeadDim;
            const int kvh = head - a.heads;
            a.k_cache[(((int64_t)b * a.kv_heads + kvh) * a.max_len + i) * kHeadDim + d] =
                float_to_bf16_bits(rope_elem(vec[d], vec[d ^ (kHeadDim / 2)], cs[d], sn[d], d));
        } else {
            const int kvh = head - a.heads - a.kv_heads;
            a.v_cache[(((int64_t)b * a.kv_heads + kvh) * a.max_len + i) * kHeadDim + d] = src[e];
        }
    }
}

// One workgroup of 4 waves per (sequence, query head, block of 64 query
// rows); wave w owns rows 16 w .. 16 w + 15 of the block.  For each key block
// kb <= the query block (causal):
//   staging: the 64 keys as rows [key][dim] and the values transposed
//            [dim][key] in LDS (shared by the 4 waves);
//   scores:  MFMA, A = the wave's rotated query rows (registers), B = keys;
//            D[row 4 q + r][key 16 cb + j], times scale * log2(e), masked
//            past the row's position;
//   softmax: online per row in base 2 (running max m and sum l, earlier
//            sums rescaled by 2^(m_old - m_new));
//   values:  MFMA, A = probabilities (bf16 hi + lo, through LDS), B = the
//            transposed values; D[row 4 q + r][dimension 16 cb + j].
// Every row sees key 0 in the first block, so its running max is finite.
__global__ __launch_bounds__(256) void prefill_attention_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[kPrefillBlock][kRowStride];          // keys
    __shared__ __attribute__((aligned(16))) uint16_t vt[kHeadDim][kPrefillBlock + 8];       // values^T
    __shared__ __attribute__((aligned(16))) float pw[4][16][kPrefillBlock + 4];             // probabilities
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int mj = lane & 15;
    const int mq = lane >> 4;
    const int qblocks = (a.length + kPrefillBlock - 1) / kPrefillBlock;
    const int qb = blockIdx.x % qblocks;
    const int head = (blockIdx.x / qblocks) % a.heads;
    const int b = blockIdx.x / (qblocks * a.heads);
    const int kvh = head / (a.heads / a.kv_heads);
    const int q0 = qb * kPrefillBlock + 16 * wave;  // this wave's first query row
    const uint16_t* kc = a.k_cache + ((int64_t)b * a.kv_heads + kvh) * a.max_len * kHeadDim;
    const uint16_t* vc = a.v_cache + ((int64_t)b * a.kv_heads + kvh) * a.max_len * kHeadDim;

    // A operands: query row q0 + mj (clamped), dimensions 32 sl + 8 mq .. + 7
    u32x4 qa[kHeadDim / 32];
    {
        const int qi = min(q0 + mj, a.length - 1);
        const uint16_t* qrow = a.qrot + (((int64_t)b * a.heads + head) * a.length + qi) * kHeadDim;
#pragma unroll
        for (int sl = 0; sl < kHeadDim / 32; ++sl) qa[sl] = *(const u32x4*)(qrow + 32 * sl + 8 * mq);
    }
    float m_run[4], l_run[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m_run[r] = -INFINITY;
        l_run[r] = 0.0f;
    }
    float4v oacc[kHeadDim / 16];
#pragma unroll
    for (int cb = 0; cb < kHeadDim / 16; ++cb) oacc[cb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // Keys: piece e = tid + 256 u -> key e / 16, dimensions 8 (e % 16) .. + 7
    // (row-major LDS stores).  Values: thread t takes dimensions 8 vcol .. + 7,
    // vcol = t / 16, of the four consecutive keys vrow0 + u, vrow0 = 4 (t % 16),
    // so that one 8-byte store writes four keys of a transposed dimension row.
    // Keys past the prompt re-read its last row (their scores are masked).
    // A block's loads are issued while the previous block is computed.
    const int vcol = tid / 16;
    const int vrow0 = 4 * (tid % 16);
    u32x4 kr[4], vr[4];
    auto load_kv = [&](int kb) {
        const int t0 = kb * kPrefillBlock;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + 256 * u;
            const int key = min(t0 + e / 16, a.length - 1);
            kr[u] = *(const u32x4*)(kc + (int64_t)key * kHeadDim + 8 * (e % 16));
            const int vkey = min(t0 + vrow0 + u, a.length - 1);
            vr[u] = *(const u32x4*)(vc + (int64_t)vkey * kHeadDim + 8 * vcol);
        }
    };
    load_kv(0);
    for (int kb = 0; kb <= qb; ++kb) {
        const int t0 = kb * kPrefillBlock;
        // ---- stage the block's keys and transposed values ----
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = tid + 256 * u;
            *(u32x4*)&ks[e / 16][8 * (e % 16)] = kr[u];
        }
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const uint32_t sel = (h & 1) ? 0x07060302u : 0x05040100u;  // high or low halves
            const uint32_t p01 = __builtin_amdgcn_perm(vr[1][h / 2], vr[0][h / 2], sel);
            const uint32_t p23 = __builtin_amdgcn_perm(vr[3][h / 2], vr[2][h / 2], sel);
            *(u32x2*)&vt[8 * vcol + h][vrow0] = u32x2{p01, p23};
        }
        __syncthreads();
        if (kb < qb) load_kv(kb + 1);  // in flight during this block's products
        // ---- scores ----
        float s[4][4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            float4v sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int sl = 0; sl < kHeadDim / 32; ++sl) {
                const u32x4 bv = *(const u32x4*)&ks[16 * cb + mj][32 * sl + 8 * mq];
                sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, qa[sl]),
                                                               __builtin_bit_cast(bf16x8, bv), sacc, 0, 0, 0);
            }
            const int t = t0 + 16 * cb + mj;
#pragma unroll
            for (int r = 0; r < 4; ++r) s[cb][r] = t <= q0 + 4 * mq + r ? sacc[r] * a.scale2 : -INFINITY;
        }
        // ---- online softmax per row 4 mq + r ----
        float alpha[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float bm = row16_max(fmaxf(fmaxf(s[0][r], s[1][r]), fmaxf(s[2][r], s[3][r])));
            const float mn = fmaxf(m_run[r], bm);
            alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - mn);  // 2^-inf = 0 on the first block
            float ps = 0.0f;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const float p = __builtin_amdgcn_exp2f(s[cb][r] - mn);  // masked: 2^-inf = 0
                pw[wave][4 * mq + r][16 * cb + mj] = p;
                ps += p;
            }
            l_run[r] = fmaf(l_run[r], alpha[r], row16_sum(ps));
            m_run[r] = mn;
        }
        // LDS operations of one wave complete in order; the fences keep the
        // compiler from moving the reads above the writes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
        for (int cb = 0; cb < kHeadDim / 16; ++cb)
#pragma unroll
            for (int r = 0; r < 4; ++r) oacc[cb][r] *= alpha[r];
#pragma unroll
        for (int kh = 0; kh < kPrefillBlock / 32; ++kh) {
            // A = probabilities of row mj, keys 32 kh + 8 mq .. + 7, as bf16 hi + lo
            const float4v p0 = *(const float4v*)&pw[wave][mj][32 * kh + 8 * mq];
            const float4v p1 = *(const float4v*)&pw[wave][mj][32 * kh + 8 * mq + 4];
            u32x4 phi, plo;
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float x0 = h < 2 ? p0[2 * h] : p1[2 * h - 4];
                const float x1 = h < 2 ? p0[2 * h + 1] : p1[2 * h - 3];
                const uint16_t h0 = float_to_bf16_bits(x0), h1 = float_to_bf16_bits(x1);
                const uint16_t l0 = float_to_bf16_bits(x0 - bf16_bits_to_float(h0));
                const uint16_t l1 = float_to_bf16_bits(x1 - bf16_bits_to_float(h1));
                phi[h] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                plo[h] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            }
#pragma unroll
            for (int cb = 0; cb < kHeadDim / 16; ++cb) {
                const u32x4 bv = *(const u32x4*)&vt[16 * cb + mj][32 * kh + 8 * mq];
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, phi),
                                                                   __builtin_bit_cast(bf16x8, bv), oacc[cb], 0, 0, 0);
                oacc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, plo),
                                                                   __builtin_bit_cast(bf16x8, bv), oacc[cb], 0, 0, 0);
            }
        }
        __syncthreads();  // the next block's staging overwrites ks and vt
    }
    // ---- out[b * length + i][head * 128 + d] = bf16(o / l) ----
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int i = q0 + 4 * mq + r;
        if (i >= a.length) continue;
        uint16_t* orow = a.out + ((int64_t)b * a.length + i) * a.heads * kHeadDim + head * kHeadDim;
        const float inv = 1.0f / l_run[r];
#pragma unroll
        for (int cb = 0; cb < kHeadDim / 16; ++cb) orow[16 * cb + mj] = float_to_bf16_bits(oacc[cb][r] * inv);
    }
}

// Decode-step prologue, one workgroup per sequence: the token's embedding
// row into x, and the rotary factors of the common position p: angle =
// float(p) * inv_freq[d % (D/2)] (one fp32 product), cos/sin in fp32, then
// bf16 (model.py: the embedding lookup and RotaryEmbedding.forward for one
// position).  A token id outside [0, vocab) gives a row of NaN.  With a norm
// weight, also the first layer's input RMSNorm of x into `normed`
// (bf16(bf16(x r) w), r = rsqrt(mean(x^2) + eps), as add_rmsnorm_kernel).
__global__ __launch_bounds__(256) void decode_prologue_kernel(const int64_t* token_ids, const uint16_t* embed,
                                                              const int64_t* position, const float* inv_freq,
                                                              uint16_t* x, uint16_t* cos_out, uint16_t* sin_out,
                                                              const uint16_t* norm_w, float eps, uint16_t* normed,
                                                              int hidden, int64_t vocab) {
    __shared__ float wsum[4];
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t tok = token_ids[b];
    const bool valid = tok >= 0 && tok < vocab;
    const uint16_t* src = embed + (valid ? tok : 0) * (int64_t)hidden;
    uint16_t* dst = x + (int64_t)b * hidden;
    const u32x4 nan4 = {0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u, 0x7FC07FC0u};
    float sq = 0.0f;
    for (int c = tid; c < hidden / 8; c += 256) {
        const u32x4 v = valid ? *(const u32x4*)(src + 8 * c) : nan4;
        *(u32x4*)(dst + 8 * c) = v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = bf16_bits_to_float((uint16_t)(v[e / 2] >> (16 * (e & 1))));
            sq += __fmul_rn(f, f);
        }
    }
    if (normed) {
        const float ws = wave_sum64(sq);
        if ((tid & 63) == 0) wsum[tid >> 6] = ws;
        __syncthreads();
        const float r = rsqrtf((((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) / (float)hidden + eps);
        uint16_t* ndst = normed + (int64_t)b * hidden;
        for (int c = tid; c < hidden / 8; c += 256) {
            const u32x4 v = valid ? *(const u32x4*)(src + 8 * c) : nan4;
            const u32x4 w = *(const u32x4*)(norm_w + 8 * c);
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float n0 = bf16_round(bf16_bits_to_float(v[e] & 0xFFFFu) * r) * bf16_bits_to_float(w[e] & 0xFFFFu);
                const float n1 = bf16_round(bf16_bits_to_float(v[e] >> 16) * r) * bf16_bits_to_float(w[e] >> 16);
                o[e] = float_to_bf16_bits(n0) | ((uint32_t)float_to_bf16_bits(n1) << 16);
            }
            *(u32x4*)(ndst + 8 * c) = o;
        }
    }
    if (tid < kHeadDim) {
        const float angle = (float)*position * inv_freq[tid % (kHeadDim / 2)];
        cos_out[(int64_t)b * kHeadDim + tid] = float_to_bf16_bits(cosf(angle));
        sin_out[(int64_t)b * kHeadDim + tid] = float_to_bf16_bits(sinf(angle));
    }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gate_up, float* out, int64_t total,
                                                       int inter) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t r = i / inter;
    const int64_t c = i - r * inter;
    const float g = bf16_bits_to_float(gate_up[r * 2 * inter + c]);
    const float u = bf16_bits_to_float(gate_up[r * 2 * inter + inter + c]);
    out[i] = (g / (1.0f + expf(-g))) * u;
}

bool aligned16(const void* p) { return (((uintptr_t)p) & 15) == 0; }

int launch_status(hipError_t err, const char* what) {
    if (err != hipSuccess)
        return set_error(W4G64_STATUS_HIP_ERROR, "%s launch failed: %s", what, hipGetErrorString(err));
    return clear_error();
}

}  // namespace
}  // namespace w4g64

using namespace w4g64;

extern "C" {

int qwen2_add_rmsnorm(const void* x, const void* delta, int delta_dtype, const void* weight, float eps,
                      void* out_sum, void* out_norm, int64_t rows, int64_t hidden, void* stream) {
    if (rows < 0) return set_error(W4G64_STATUS_INVALID_VALUE, "rows must be non-negative, got %lld", (long long)rows);
    if (hidden <= 0 || hidden % 8 || hidden > kNormThreads * 8 * kNormIters)
        return set_error(W4G64_STATUS_INVALID_VALUE, "hidden must be a multiple of 8 in [8, %d], got %lld",
                         kNormThreads * 8 * kNormIters, (long long)hidden);
    const int parts = W4G64_DTYPE_F32_PARTS_OF(delta_dtype);
    if (delta && delta_dtype != W4G64_DTYPE_BF16 && delta_dtype != W4G64_DTYPE_F32 && parts == 0)
        return set_error(W4G64_STATUS_INVALID_DTYPE, "residual delta must be bf16, fp32 or fp32 partial sums");
    if (rows == 0) return clear_error();
    if (!x || !weight || !out_norm)
        return set_error(W4G64_STATUS_INVALID_VALUE, "x, weight and out_norm must be non-null device pointers");
    if (!aligned16(x) || !aligned16(weight) || !aligned16(out_norm) || (out_sum && !aligned16(out_sum)) ||
        (delta && !aligned16(delta)))
        return set_error(W4G64_STATUS_INVALID_VALUE, "add_rmsnorm tensors must be 16-byte aligned");
    if (rows > 0x7FFFFFFF) return set_error(W4G64_STATUS_INVALID_VALUE, "too many rows");
    const int kind = !delta ? 0 : (parts ? (int)kNormP : delta_dtype);
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, (hipStream_t)stream,
                       (const uint16_t*)x, delta, kind, parts, (const uint16_t*)weight, eps, (uint16_t*)out_sum,
                       (uint16_t*)out_norm, (int)hidden);
    return launch_status(hipGetLastError(), "add_rmsnorm");
}

int64_t qwen2_decode_attention_workspace_bytes(int64_t batch, int64_t num_kv_heads, int64_t max_length) {
    if (batch <= 0 || num_kv_heads <= 0 || max_length <= 0) return 0;
    const int64_t chunks = (max_length + kChunk - 1) / kChunk;
    return attention_counter_bytes(batch, num_kv_heads) +
           batch * num_kv_heads * chunks * kPartFloats * (int64_t)sizeof(float);
}

static int decode_attention(const void* qkv, const void* cos, const void* sin, void* k_cache, void* v_cache,
                            const int64_t* position, void* out, bool unmerged, int64_t batch, int64_t num_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t max_length, float scale,
                            void* workspace, int64_t workspace_bytes, void* stream) {
    if (batch < 0) return set_error(W4G64_STATUS_INVALID_VALUE, "batch must be non-negative");
    if (head_dim != kHeadDim)
        return set_error(W4G64_STATUS_UNSUPPORTED, "head_dim must be %d, got %lld", kHeadDim, (long long)head_dim);
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 ||
        num_heads / num_kv_heads > kMaxGroup)
        return set_error(W4G64_STATUS_INVALID_VALUE,
                         "num_heads (%lld) must be a positive multiple of num_kv_heads (%lld), at most %d times",
                         (long long)num_heads, (long long)num_kv_heads, kMaxGroup);
    if (max_length <= 0 || max_length > kMaxLength)
        return set_error(W4G64_STATUS_INVALID_VALUE, "max_length must be in [1, %d], got %lld", kMaxLength,
                         (long long)max_length);
    if (batch == 0) return clear_error();
    if (!qkv || !cos || !sin || !k_cache || !v_cache || !position || (!out && !unmerged))
        return set_error(W4G64_STATUS_INVALID_VALUE, "all tensors must be non-null device pointers");
    if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache))
        return set_error(W4G64_STATUS_INVALID_VALUE, "qkv, k_cache and v_cache must be 16-byte aligned");
    if (((uintptr_t)out) & 7) return set_error(W4G64_STATUS_INVALID_VALUE, "out must be 8-byte aligned");
    if (workspace && !aligned16(workspace))
        return set_error(W4G64_STATUS_WORKSPACE, "attention workspace must be 16-byte aligned");
    const int64_t need = qwen2_decode_attention_workspace_bytes(batch, num_kv_heads, max_length);
    if (!workspace || workspace_bytes < need)
        return set_error(W4G64_STATUS_WORKSPACE, "attention workspace of %lld bytes required, got %lld",
                         (long long)need, (long long)(workspace ? workspace_bytes : 0));
    const int64_t chunks = (max_length + kChunk - 1) / kChunk;
    const int64_t blocks = batch * num_kv_heads * chunks;
    if (blocks > 0x7FFFFFFF) return set_error(W4G64_STATUS_INVALID_VALUE, "problem too large");
    AttnArgs args;
    args.qkv = (const uint16_t*)qkv;
    args.cos = (const uint16_t*)cos;
    args.sin = (const uint16_t*)sin;
    args.k_cache = (uint16_t*)k_cache;
    args.v_cache = (uint16_t*)v_cache;
    args.position = position;
    args.out = (uint16_t*)out;
    args.heads = (int)num_heads;
    args.kv_heads = (int)num_kv_heads;
    args.max_len = (int)max_length;
    args.chunks = (int)chunks;
    args.scale = scale;
    args.counters = (unsigned*)workspace;
    args.partials = (float*)((char*)workspace + attention_counter_bytes(batch, num_kv_heads));
    args.unmerged = unmerged ? 1 : 0;
    W4G64_TIMELINE_SET(args);
    hipLaunchKernelGGL(attention_kernel, dim3((unsigned)blocks), dim3(kAttnThreads), 0, (hipStream_t)stream, args);
    return launch_status(hipGetLastError(), "decode_attention");
}

int qwen2_decode_attention(const void* qkv, const void* cos, const void* sin, void* k_cache, void* v_cache,
                           const int64_t* position, void* out, int64_t batch, int64_t num_heads,
                           int64_t num_kv_heads, int64_t head_dim, int64_t max_length, float scale,
                           void* workspace, int64_t workspace_bytes, void* stream) {
    return decode_attention(qkv, cos, sin, k_cache, v_cache, position, out, false, batch, num_heads, num_kv_heads,
                            head_dim, max_length, scale, workspace, workspace_bytes, stream);
}

int qwen2_decode_attention_partials(const void* qkv, const void* cos, const void* sin, void* k_cache,
                                    void* v_cache, const int64_t* position, int64_t batch, int64_t num_heads,
                                    int64_t num_kv_heads, int64_t head_dim, int64_t max_length, float scale,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
    return decode_attention(qkv, cos, sin, k_cache, v_cache, position, nullptr, true, batch, num_heads,
                            num_kv_heads, head_dim, max_length, scale, workspace, workspace_bytes, stream);
}

int64_t qwen2_prefill_attention_workspace_bytes(int64_t batch, int64_t num_heads, int64_t length) {
    if (batch <= 0 || num_heads <= 0 || length <= 0) return 0;
    return batch * num_heads * length * kHeadDim * (int64_t)sizeof(uint16_t);
}

int qwen2_prefill_attention(const void* qkv, const void* cos, const void* sin, void* k_cache, void* v_cache,
                            void* out, int64_t batch, int64_t length, int64_t num_heads, int64_t num_kv_heads,
                            int64_t head_dim, int64_t max_length, float scale, void* workspace,
                            int64_t workspace_bytes, void* stream) {
    if (batch < 0 || length < 0) return set_error(W4G64_STATUS_INVALID_VALUE, "batch and length must be non-negative");
    if (head_dim != kHeadDim)
        return set_error(W4G64_STATUS_UNSUPPORTED, "head_dim must be %d, got %lld", kHeadDim, (long long)head_dim);
    if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0 ||
        num_heads / num_kv_heads > kMaxGroup)
        return set_error(W4G64_STATUS_INVALID_VALUE,
                         "num_heads (%lld) must be a positive multiple of num_kv_heads (%lld), at most %d times",
                         (long long)num_heads, (long long)num_kv_heads, kMaxGroup);
    if (length > max_length || max_length > 0x7FFFFFFF)
        return set_error(W4G64_STATUS_INVALID_VALUE, "length (%lld) must be at most max_length (%lld)",
                         (long long)length, (long long)max_length);
    if (batch == 0 || length == 0) return clear_error();
    if (!qkv || !cos || !sin || !k_cache || !v_cache || !out)
        return set_error(W4G64_STATUS_INVALID_VALUE, "all tensors must be non-null device pointers");
    if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache))
        return set_error(W4G64_STATUS_INVALID_VALUE, "qkv, k_cache and v_cache must be 16-byte aligned");
    const int64_t need = qwen2_prefill_attention_workspace_bytes(batch, num_heads, length);
    if (!workspace || workspace_bytes < need || !aligned16(workspace))
        return set_error(W4G64_STATUS_WORKSPACE, "prefill attention workspace of %lld bytes (16-byte aligned) required, got %lld",
                         (long long)need, (long long)(workspace ? workspace_bytes : 0));
    const int64_t qblocks = (length + kPrefillBlock - 1) / kPrefillBlock;
    if (batch * length > 0x7FFFFFFF || batch * num_heads * qblocks > 0x7FFFFFFF)
        return set_error(W4G64_STATUS_INVALID_VALUE, "problem too large");
    PrefillArgs args;
    args.qkv = (const uint16_t*)qkv;
    args.cos = (const uint16_t*)cos;
    args.sin = (const uint16_t*)sin;
    args.k_cache = (uint16_t*)k_cache;
    args.v_cache = (uint16_t*)v_cache;
    args.qrot = (uint16_t*)workspace;
    args.out = (uint16_t*)out;
    args.length = (int)length;
    args.heads = (int)num_heads;
    args.kv_heads = (int)num_kv_heads;
    args.max_len = (int)max_length;
    args.scale2 = scale * 1.4426950408889634f;
    hipLaunchKernelGGL(prefill_rope_kernel, dim3((unsigned)(batch * length)), dim3(256), 0, (hipStream_t)stream, args);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return launch_status(err, "prefill_rope");
    hipLaunchKernelGGL(prefill_attention_kernel, dim3((unsigned)(batch * num_heads * qblocks)), dim3(256), 0,
                       (hipStream_t)stream, args);
    return launch_status(hipGetLastError(), "prefill_attention");
}

int qwen2_decode_prologue(const int64_t* token_ids, const void* embed, const int64_t* position, const float* inv_freq,
                          void* x, void* cos, void* sin, const void* norm_weight, float eps, void* normed,
                          int64_t batch, int64_t hidden, int64_t vocab, int64_t head_dim, void* stream) {
    if (batch < 0) return set_error(W4G64_STATUS_INVALID_VALUE, "batch must be non-negative");
    if (head_dim != kHeadDim)
        return set_error(W4G64_STATUS_UNSUPPORTED, "head_dim must be %d, got %lld", kHeadDim, (long long)head_dim);
    if (hidden <= 0 || hidden % 8 || hidden > (1 << 20))
        return set_error(W4G64_STATUS_INVALID_VALUE, "hidden must be a positive multiple of 8, got %lld",
                         (long long)hidden);
    if (vocab <= 0) return set_error(W4G64_STATUS_INVALID_VALUE, "vocab must be positive");
    if (batch == 0) return clear_error();
    if (batch > 0x7FFFFFFF) return set_error(W4G64_STATUS_INVALID_VALUE, "problem too large");
    if (!token_ids || !embed || !position || !inv_freq || !x || !cos || !sin)
        return set_error(W4G64_STATUS_INVALID_VALUE, "all tensors must be non-null device pointers");
    if (!aligned16(embed) || !aligned16(x) || ((uintptr_t)cos & 1) || ((uintptr_t)sin & 1) ||
        ((uintptr_t)token_ids & 7) || ((uintptr_t)position & 7) || ((uintptr_t)inv_freq & 3))
        return set_error(W4G64_STATUS_INVALID_VALUE, "embed and x must be 16-byte aligned, the others element aligned");
    if ((norm_weight == nullptr) != (normed == nullptr))
        return set_error(W4G64_STATUS_INVALID_VALUE, "norm_weight and normed must both be given or both be null");
    if (normed && (!aligned16(norm_weight) || !aligned16(normed)))
        return set_error(W4G64_STATUS_INVALID_VALUE, "norm_weight and normed must be 16-byte aligned");
    hipLaunchKernelGGL(decode_prologue_kernel, dim3((unsigned)batch), dim3(256), 0, (hipStream_t)stream, token_ids,
                       (const uint16_t*)embed, position, inv_freq, (uint16_t*)x, (uint16_t*)cos, (uint16_t*)sin,
                       (const uint16_t*)norm_weight, eps, (uint16_t*)normed, (int)hidden, vocab);
    return launch_status(hipGetLastError(), "decode_prologue");
}

int qwen2_silu_mul(const void* gate_up, float* out, int64_t rows, int64_t intermediate, void* stream) {
    if (rows < 0 || intermediate <= 0 || intermediate > 0x3FFFFFFF)
        return set_error(W4G64_STATUS_INVALID_VALUE, "rows must be non-negative and intermediate positive");
    if (rows == 0) return clear_error();
    if (!gate_up || !out) return set_error(W4G64_STATUS_INVALID_VALUE, "gate_up and out must be non-null");
    const int64_t total = rows * intermediate;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7FFFFFFF) return set_error(W4G64_STATUS_INVALID_VALUE, "problem too large");
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)gate_up, out, total, (int)intermediate);
    return launch_status(hipGetLastError(), "silu_mul");
}

}  // extern "C"
