// Device-side helpers shared by the W4G64 kernels (gfx950 only).
//
// Nibble decode.  A packed dword holds 8 consecutive K values; byte b holds
// k = 2b (low nibble) and k = 2b+1 (high nibble).  XOR with 0x8 maps every
// signed nibble s in [-8, 7] to n' = s + 8 in [0, 15].  OR-ing n' into the
// mantissa of a power of two builds an exact small float:
//   fp16 0x6400 | n'         = 1024 + n'   (n' in mantissa bits 0-3)
//   fp16 0x5400 | (n' << 4)  =   64 + n'   (n' in mantissa bits 4-7)
//   bf16 0x4300 | n'         =  128 + n'
// Masks 0x000F000F / 0x00F000F0 on the dword and on the dword >> 8 give the
// pairs (k0,k4), (k1,k5), (k2,k6), (k3,k7), so an 8-value MFMA operand is
// ordered [k0 k4 k1 k5 k2 k6 k3 k7]; activations are staged in the same
// order, which leaves every dot product unchanged.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4g64 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Activation kinds.  kSwiGLU forms the activation in the decode GEMV's
// staging: silu(gate) * up in fp32 from a [gate | up] bf16 row (fp32 result).
enum XKind : int {
    kF16 = 1, kBF16 = 2, kF32 = 3, kSwiGLU = 5, kPlanes = 6,
    // bf16 activations formed in the decode GEMV's staging as RMSNorm(residual
    // + delta), delta bf16 (kNormB), fp32 (kNormF) or the sum of up to
    // kMaxDeltaParts fp32 split-K partial sums of the previous projection
    // (kNormP); internal kinds
    kNormB = 7, kNormF = 8, kNormP = 9,
    // bf16 activations merged in the decode GEMV's staging from the decode
    // attention's per-chunk partial results (internal kind)
    kAttnM = 10
};
constexpr int kMaxDeltaParts = 8;

// Slot order of the 8 values in an MFMA operand: slot p holds k = kSlotK[p].
// (Used by host-side documentation/tests; kernels permute with v_perm.)

__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t mask, uint32_t magic) {
    return ((w ^ 0x88888888u) & mask) | magic;
}

// Exact signed (code - zero) as fp16, slot order [k0 k4 k1 k5 k2 k6 k3 k7].
// c_lo = 1032 + zero, c_hi = 72 + zero (both exact in fp16).
__device__ __forceinline__ half8 dequant8_f16_int(uint32_t w, half2v c_lo, half2v c_hi) {
    half2v h0 = __builtin_bit_cast(half2v, nib_pair(w, 0x000F000Fu, 0x64006400u)) - c_lo;
    half2v h1 = __builtin_bit_cast(half2v, nib_pair(w, 0x00F000F0u, 0x54005400u)) - c_hi;
    half2v h2 = __builtin_bit_cast(half2v, nib_pair(w >> 8, 0x000F000Fu, 0x64006400u)) - c_lo;
    half2v h3 = __builtin_bit_cast(half2v, nib_pair(w >> 8, 0x00F000F0u, 0x54005400u)) - c_hi;
    half8 r = {h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
    return r;
}

// bf16 values 128 + n' (exact), slot order [k0 k4 k1 k5 k2 k6 k3 k7].
// The caller subtracts (136 + zero) * sum(x) from the fp32 dot product.
__device__ __forceinline__ bf16x8 dequant8_bf16_biased(uint32_t w) {
    u32x4 v;
    v[0] = nib_pair(w, 0x000F000Fu, 0x43004300u);
    v[1] = nib_pair(w >> 4, 0x000F000Fu, 0x43004300u);
    v[2] = nib_pair(w >> 8, 0x000F000Fu, 0x43004300u);
    v[3] = nib_pair(w >> 12, 0x000F000Fu, 0x43004300u);
    return __builtin_bit_cast(bf16x8, v);
}

// Signed INT4 nibble e of a packed byte array (canonical order).
__device__ __forceinline__ int nibble_at(const uint8_t* p, int64_t e) {
    int b = p[e >> 1];
    int n = (e & 1) ? (b >> 4) : (b & 0xF);
    return n - ((n & 8) << 1);
}

// Permute 8 consecutive 16-bit values (as 4 dwords) into slot order.
__device__ __forceinline__ u32x4 permute_slots(u32x4 d) {
    u32x4 o;
    o[0] = __builtin_amdgcn_perm(d[2], d[0], 0x05040100u);  // (x0, x4)
    o[1] = __builtin_amdgcn_perm(d[2], d[0], 0x07060302u);  // (x1, x5)
    o[2] = __builtin_amdgcn_perm(d[3], d[1], 0x05040100u);  // (x2, x6)
    o[3] = __builtin_amdgcn_perm(d[3], d[1], 0x07060302u);  // (x3, x7)
    return o;
}

__device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
    return __builtin_bit_cast(float, b << 16);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Round-to-nearest-even conversions used for outputs.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Exact three-way split of an fp32 value into bf16 parts (hi + mid + lo == x
// for every normal x whose parts stay normal), by truncation.  No FP
// contraction here: fused into a caller's product (fma(a, b, -hi)), the first
// remainder would belong to the unrounded a * b rather than to x.
__device__ __forceinline__ void split3_bf16(float x, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
#pragma clang fp contract(off)
    uint32_t xb = __builtin_bit_cast(uint32_t, x);
    uint32_t hb = xb & 0xFFFF0000u;
    float r1 = x - __builtin_bit_cast(float, hb);
    uint32_t r1b = __builtin_bit_cast(uint32_t, r1);
    uint32_t mb = r1b & 0xFFFF0000u;
    float r2 = r1 - __builtin_bit_cast(float, mb);
    hi = (uint16_t)(hb >> 16);
    mid = (uint16_t)(mb >> 16);
    lo = (uint16_t)(__builtin_bit_cast(uint32_t, r2) >> 16);
}

// Two-way split for the GEMM (16 significant bits; the bf16 weight tile
// carries 8): hi by truncation, lo rounded.
__device__ __forceinline__ void split2_bf16(float x, uint16_t& hi, uint16_t& lo) {
#pragma clang fp contract(off)
    uint32_t xb = __builtin_bit_cast(uint32_t, x);
    uint32_t hb = xb & 0xFFFF0000u;
    float r1 = x - __builtin_bit_cast(float, hb);
    hi = (uint16_t)(hb >> 16);
    lo = float_to_bf16_bits(r1);
}

__device__ __forceinline__ float load_bias(const void* bias, int kind, int64_t n) {
    if (kind == kF16) return half_bits_to_float(((const uint16_t*)bias)[n]);
    if (kind == kBF16) return bf16_bits_to_float(((const uint16_t*)bias)[n]);
    if (kind == kF32) return ((const float*)bias)[n];
    return 0.0f;
}

template <int XK>
__device__ __forceinline__ void store_out(void* y, int64_t idx, float v) {
    if constexpr (XK == kF16) {
        ((uint16_t*)y)[idx] = float_to_half_bits(v);
    } else if constexpr (XK == kBF16) {
        ((uint16_t*)y)[idx] = float_to_bf16_bits(v);
    } else {
        ((float*)y)[idx] = v;
    }
}

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_float(float_to_bf16_bits(v)); }

// Two values rounded to bf16 (round to nearest even, as float_to_bf16_bits)
// by one conversion instruction: a in the low half, b in the high half.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{a, b}, bf16x2v));
}
// The low and high bf16 halves of a word as fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }

// Sum over the 64 lanes of a wave (quad swaps, half-row and row mirrors give
// every lane its row's sum; row broadcasts 15 and 31 add the rows up in
// lane 63), read from lane 63: one fixed order of additions.
__device__ __forceinline__ float wave_sum64(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    // lanes outside a broadcast's row mask receive the `old` operand, 0
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Wave-wide maximum over the wave sum's steps (quad swaps, half-row and row
// mirrors, row broadcasts 15 and 31; lanes outside a broadcast's row mask
// keep their own value); the result is lane 63's.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_keep(float x) {
    const int b = __builtin_bit_cast(int, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_keep<0xB1, 0xF>(v));
    v = fmaxf(v, dpp_keep<0x4E, 0xF>(v));
    v = fmaxf(v, dpp_keep<0x141, 0xF>(v));
    v = fmaxf(v, dpp_keep<0x140, 0xF>(v));
    v = fmaxf(v, dpp_keep<0x142, 0xA>(v));
    v = fmaxf(v, dpp_keep<0x143, 0xC>(v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// h = silu(bf16(g)) * bf16(up) in fp32 (the projections' outputs are bf16,
// model.py:133-135; silu(x) = x / (1 + exp(-x))), stored as its exact
// three-way bf16 split: planes [3][M][I], hi + mid + lo == h.
__device__ __forceinline__ void store_silu_planes(void* y, int m, int i, int M, int I, float g, float up) {
    const float gb = bf16_round(g), ub = bf16_round(up);
    const float h = (gb / (1.0f + expf(-gb))) * ub;
    uint16_t hi, mid, lo;
    split3_bf16(h, hi, mid, lo);
    uint16_t* planes = (uint16_t*)y;
    const int64_t at = (int64_t)m * I + i, plane = (int64_t)M * I;
    planes[at] = hi;
    planes[plane + at] = mid;
    planes[2 * plane + at] = lo;
}

// Arrival of a workgroup at a cross-workgroup merge: true in the last of
// `expected` workgroups to arrive on `counter`.  The workgroup barrier orders
// every thread's partial-sum stores before thread 0's agent-scope release
// (the fetch_add), and the last arriver's agent-scope acquire fence before
// the barrier that releases its threads to read the partial sums, so the
// merge sees every other workgroup's stores under the HIP memory model
// (happens-before is transitive across the workgroup and agent scopes).
// `flag` is a __shared__ int of the caller.  Every thread must call this.
// 16 bytes at byte offset `off` of a buffer resource over `size` bytes;
// bytes past the end read as 0.  A raw buffer load that reaches past the
// resource's end returns zero as a whole, so the chunk that straddles the
// end is read byte by byte (each byte load is in range or reads 0).
__device__ __forceinline__ u32x4 load16_bounded(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t size) {
    if (off + 16u <= size) return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
    u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t b = __builtin_amdgcn_raw_buffer_load_b8(r, (int)(off + (uint32_t)i), 0, 0);
        v[i >> 2] |= (b & 0xFFu) << (8 * (i & 3));
    }
    return v;
}

// ---- workgroup timelines (profiling builds only) ----
// Built with -DW4G64_TIMELINE (a separate library, libw4g64_hip_timeline.so),
// an instrumented kernel records up to 8 chip-wide timestamps (s_memrealtime,
// 100 MHz) of its phases in registers, and thread 0 of each workgroup (linear
// id x + X y) below the registered count stores them to stamps[workgroup][8]
// at exit, after its own stores have completed.  Without the define every macro is empty.
#ifdef W4G64_TIMELINE
#define W4G64_TIMELINE_FIELDS unsigned long long* tl_stamps; int tl_workgroups;
#define W4G64_TIMELINE_DECL unsigned long long tl_[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define W4G64_STAMP(k) (tl_[(k)] = __builtin_amdgcn_s_memrealtime())
#define W4G64_TIMELINE_STORE(args)                                                                   \
    do {                                                                                             \
        __builtin_amdgcn_s_waitcnt(0);                                                               \
        W4G64_STAMP(7);                                                                              \
        const int wg_ = (int)(blockIdx.x + gridDim.x * blockIdx.y);                                  \
        if ((args).tl_stamps && threadIdx.x == 0 && wg_ < (args).tl_workgroups)                      \
            for (int k_ = 0; k_ < 8; ++k_) (args).tl_stamps[(int64_t)wg_ * 8 + k_] = tl_[k_];        \
    } while (0)
#define W4G64_TIMELINE_SET(args) ((args).tl_stamps = ::w4g64::g_timeline_stamps, (args).tl_workgroups = ::w4g64::g_timeline_workgroups)
#else
#define W4G64_TIMELINE_FIELDS
#define W4G64_TIMELINE_DECL ((void)0)
#define W4G64_STAMP(k) ((void)0)
#define W4G64_TIMELINE_STORE(args) ((void)0)
#define W4G64_TIMELINE_SET(args) ((void)0)
#endif

__device__ __forceinline__ bool arrive_last(unsigned* counter, unsigned expected, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = prev == expected - 1u;
        if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        *flag = last;
    }
    __syncthreads();
    return *flag != 0;
}

}  // namespace w4g64
