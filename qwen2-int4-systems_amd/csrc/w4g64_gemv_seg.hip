// Decode path, lean form: fused unpack + dequant + GEMV for 1..8 fp16/bf16
// activation rows, 16-byte weight loads, no workspace.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])  (+ bias[n])
// -- the reference's (x.float() @ W.t() + bias).to(x.dtype)
// (src/qwen_int4/backends.py:73-98) with each group's scale applied in fp32.
//
// Work per lane is what bounds a decode GEMV once its loads are wide: a
// launch streams 0.2-7.4 MB, so instruction issue per SIMD, not bytes, sets
// the time above the bare-stream floor.  This kernel keeps every lane on a
// few 16-byte weight loads and the arithmetic of its own columns.
//
// MFMA mapping (v_mfma_f32_16x16x32_{f16,bf16}), with a group pair (two
// 64-wide groups, 64 packed bytes of a row) as the unit of work:
//   * B = weights: column c = (row r, segment s), c = r SW + s, R = 16 / SW
//     rows per wave.  Lane (c, q) loads 16 bytes of row r: bytes [16 q, 16 q
//     + 16) of pair jj = base + s + SW t at step t, so one load instruction
//     reads R rows x SW x 64 contiguous bytes.  Dword u of the lane feeds
//     MFMA u (K values 32 q + 8 u + 0..7 of the pair): lanes q = 0, 1 carry
//     the pair's first group, q = 2, 3 its second.
//   * A = activations: row i = (m, segment s', half p), i = 2 (m SW + s') +
//     p, holding x[m, pair of s'] in the K slots of lanes q with q / 2 == p
//     and zero elsewhere.  D[i, c] with s' == s is the dot product of row m
//     with row r over group 2 jj + p alone; the other blocks are unused
//     (2 M SW <= 16 rows of A).
//   * fp16: B = code exactly (1024 + n' magic minus 1032, one v_pk_add_f16
//     per pair); the zero point enters after the MFMA as -zero * sum_g x.
//     bf16: B = 136 + code exactly (128 + n' magic); the correction is
//     -(136 + zero) * sum_g x.  Then the group scale multiplies in fp32.
//   * Every load is issued before any is used: the workgroup's activations,
//     scales and zero bytes (16-byte chunks into LDS), then every weight
//     load of the lane (immediate offsets off one address).  Staging lands
//     first (in-order return), goes to LDS, one LDS-only barrier, and each
//     step waits for its own weight load alone.
//   * A workgroup owns NR R whole rows; its NR NK waves split them into NR
//     row blocks and K into NK parts, and meet in LDS at the end: no partial
//     sum leaves the workgroup.  Steps past a part's last pair re-load a
//     pair of the same row and get a zero scale, so every lane issues the
//     same loads and waits.
#include <stdio.h>

#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

struct SegArgs {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    void* y;
    int bias_kind;
    int M;   // activation rows (2 M SW <= 16)
    int N;   // out_features (N G 2 and N P multiples of 16)
    int K;   // in_features
    int G;   // groups (even)
    int P;   // group pairs
    int PK;  // pairs per K part
    W4G64_TIMELINE_FIELDS
};

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float dpp_sum8(float s) {
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x4E, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x141, 0xF, 0xF, false));
    return s;
}

// Signed codes of one packed dword as fp16, slot order [k0 k4 k1 k5 k2 k6 k3 k7].
__device__ __forceinline__ half8 codes8_f16(uint32_t w) {
    const half2v c_lo = {(_Float16)1032.0f, (_Float16)1032.0f}, c_hi = {(_Float16)72.0f, (_Float16)72.0f};
    return dequant8_f16_int(w, c_lo, c_hi);
}

// LDS layout (bytes): xs [M][K] slot-ordered activations | 64 zero bytes |
// xsum [M][G] fp32 | scales of the workgroup's rows (16-byte aligned span) |
// zero bytes of its rows (16-byte aligned span) | red [waves][M][R][SW] fp32.
struct SegLayout {
    int zero, xsum, sc, zb, red, total;
};
__host__ __device__ inline SegLayout seg_layout(int M, int K, int rows, int waves, int R, int SW) {
    const int G = K / 64, P = G / 2;
    SegLayout L;
    L.zero = M * K * 2;
    L.xsum = L.zero + 64;
    L.sc = (L.xsum + M * G * 4 + 15) & ~15;
    L.zb = L.sc + ((rows * G * 2 + 32 + 15) & ~15);
    L.red = L.zb + ((rows * P + 32 + 15) & ~15);
    L.total = L.red + waves * M * R * SW * 4;
    return L;
}

template <int XK, int SW, int NR, int NK, int STEPS, int STAGE>
__global__ __launch_bounds__(NR * NK * 64) void gemv_seg_kernel(SegArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int R = 16 / SW;        // rows per wave
    constexpr int RW = NR * R;        // rows per workgroup
    constexpr int W = NR * NK;        // waves
    constexpr int kThreads = W * 64;
    static_assert(kThreads % RW == 0, "a thread's outputs share its row");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int M = a.M, K = a.K, G = a.G, P = a.P, N = a.N;
    const SegLayout L = seg_layout(M, K, RW, W, R, SW);
    const int row0 = blockIdx.x * RW;
    const int row_end = min(row0 + RW, N);
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);

    // ---- 1. staging loads: activations, scales, zero bytes (16-byte chunks) ----
    const int64_t s_lo = ((int64_t)row0 * G * 2) & ~15ll;
    const int64_t s_hi = min((((int64_t)row_end * G * 2) + 15) & ~15ll, (int64_t)N * G * 2);
    const int64_t z_lo = ((int64_t)row0 * P) & ~15ll;
    const int64_t z_hi = min((((int64_t)row_end * P) + 15) & ~15ll, (int64_t)N * P);
    const int XI = M * K / 8;
    const int SI = (int)((s_hi - s_lo) >> 4);
    const int ZI = (int)((z_hi - z_lo) >> 4);
    const int items = XI + SI + ZI;
    u32x4 sv[STAGE];
#pragma unroll
    for (int u = 0; u < STAGE; ++u) {
        int it = kThreads * u + tid;
        it = it < items ? it : items - 1;
        const uint8_t* src = it < XI ? (const uint8_t*)a.x + (int64_t)it * 16
                                     : (it < XI + SI ? (const uint8_t*)a.scales + s_lo + (int64_t)(it - XI) * 16
                                                     : a.zeros + z_lo + (int64_t)(it - XI - SI) * 16);
        sv[u] = *(const u32x4*)src;
    }
    asm volatile("" ::: "memory");

    // ---- 2. weight loads: lane (c, q) -> row r, segment s ----
    const int c = lane & 15;
    const int q = lane >> 4;
    const int r = c / SW;
    const int s = c % SW;
    const int rb = wave % NR;  // row block
    const int kp = wave / NR;  // K part
    const int wrow = rb * R + r;                   // row within the workgroup
    const int row = min(row0 + wrow, N - 1);       // rows past N re-read row N - 1 (outputs dropped)
    const int pbase = kp * a.PK;                   // first pair of this wave's K part
    const int pend = min(pbase + a.PK, P);         // end of its pairs
    const uint8_t* wsrc = a.qweight + (int64_t)row * (K / 2) + 16 * q;
    u32x4 wv[STEPS];
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int jj = pbase + s + SW * t;
        const int jl = jj < pend ? jj : (pbase < P ? pbase : 0);  // past the part: a pair of the same row
        wv[t] = __builtin_nontemporal_load((const u32x4*)(wsrc + 64 * jl));
    }
    asm volatile("" ::: "memory");  // the bias load below issues after the weights
    // the bias of the output this thread stores: one dword load whatever the
    // bias kind (a 16-bit bias element lies in the aligned dword holding it;
    // N is even), from the scales when there is no bias.  Its half is taken
    // out in the epilogue, so nothing here waits for it.
    int bias_row = row0 + tid % RW;
    bias_row = bias_row < N ? bias_row : N - 1;
    uint32_t bias_word;
    {
        const uint8_t* bsrc = a.bias_kind == 0 ? (const uint8_t*)a.scales
                              : a.bias_kind == kF32 ? (const uint8_t*)a.bias + 4 * (int64_t)bias_row
                                                    : (const uint8_t*)a.bias + 4 * (int64_t)(bias_row >> 1);
        bias_word = *(const uint32_t*)bsrc;
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < STAGE; ++u) asm volatile("" : "+v"(sv[u]));

    W4G64_STAMP(1);
    // ---- 3. staging data into LDS ----
    wait_vm<STEPS + 1>();  // everything issued before the weights has landed
    W4G64_STAMP(2);
    {
        float* xsum = (float*)(smem + L.xsum);
#pragma unroll
        for (int u = 0; u < STAGE; ++u) {
            int it = kThreads * u + tid;
            const bool real = it < items;
            it = real ? it : items - 1;
            if (it < XI) {
                *(u32x4*)(smem + (int64_t)it * 16) = permute_slots(sv[u]);
                float sum = 0.0f;
                if constexpr (XK == kF16) {
                    // 16-bit halves taken out with shifts (a bit_cast of a
                    // vector element to half2 was folded to element 0 here)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t bits = sv[u][e];
                        sum += half_bits_to_float((uint16_t)(bits & 0xFFFFu)) + half_bits_to_float((uint16_t)(bits >> 16));
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sum += __builtin_bit_cast(float, sv[u][e] << 16) + __builtin_bit_cast(float, sv[u][e] & 0xFFFF0000u);
                }
                sum = dpp_sum8(sum);  // the 8 items of one (row, group) sit in 8 aligned lanes
                if ((it & 7) == 0) xsum[it >> 3] = sum;
            } else if (real) {
                *(u32x4*)(smem + (it < XI + SI ? L.sc + (it - XI) * 16 : L.zb + (it - XI - SI) * 16)) = sv[u];
            }
        }
        if (tid < 16) ((uint32_t*)(smem + L.zero))[tid] = 0u;
    }
    lds_barrier();
    W4G64_STAMP(3);

    // ---- 4. MFMA steps ----
    // A row of this lane: i = lane % 16 = 2 (m SW + s') + p; it reads x only
    // for m < M and q / 2 == p.
    const int ai = lane & 15;
    const int am = ai / (2 * SW), as = (ai >> 1) % SW, ap = ai & 1;
    const bool a_live = am < M && (q >> 1) == ap;
    // D rows of this lane: 4 q .. 4 q + 3 = (m, s', p) for halves h = 0, 1
    // (rows 4 q + 2 h + p); the half whose segment is s belongs to column c.
    int hm[2];
    bool hu[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int ms = 2 * q + h;  // m SW + s'
        hu[h] = (ms % SW) == s && ms / SW < M;
        hm[h] = min(ms / SW, M - 1);
    }
    const uint16_t* sc = (const uint16_t*)(smem + L.sc);
    const uint8_t* zb = smem + L.zb;
    const float* xsum = (const float*)(smem + L.xsum);
    const int sc_row = (int)(((int64_t)row * G * 2 - s_lo) >> 1);  // scale element of (row, group 0)
    const int zb_row = (int)((int64_t)row * P - z_lo);            // zero byte of (row, pair 0)
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int jj = pbase + s + SW * t;    // this lane's pair (column side)
        const int ja = pbase + as + SW * t;   // the A row's pair
        const bool live = jj < pend;
        const bool alive = a_live && ja < pend;
        const unsigned char* asrc = alive ? smem + ((int64_t)am * K + 128 * ja + 32 * q) * 2 : smem + L.zero;
        u16x8 av[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) av[u] = *(const u16x8*)(asrc + (alive ? 16 * u : 0));
        // this step's weights: at most STEPS - 1 - t later weight loads and
        // the bias load outstanding
        if (t == 0) wait_vm<STEPS>();
        else if (t == 1) wait_vm<(STEPS > 1 ? STEPS - 1 : 0)>();
        else if (t == 2) wait_vm<(STEPS > 2 ? STEPS - 2 : 0)>();
        else if (t == 3) wait_vm<(STEPS > 3 ? STEPS - 3 : 0)>();
        else wait_vm<0>();
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if constexpr (XK == kF16) {
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av[u]), codes8_f16(wv[t][u]), d, 0,
                                                           0, 0);
            } else {
                d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[u]),
                                                            dequant8_bf16_biased(wv[t][u]), d, 0, 0, 0);
            }
        }
        // scales and zero points of (row, groups 2 jj, 2 jj + 1); a step past
        // the part reads an in-range pair (a K part may hold no pair at all:
        // pbase >= P) and adds s = 0 times those finite values
        const int jc = live ? jj : min(pbase, P - 1);
        const uint32_t s2 = *(const uint32_t*)(sc + sc_row + 2 * jc);
        const uint32_t z2 = zb[zb_row + jc];
        const float s0 = live ? half_bits_to_float((uint16_t)s2) : 0.0f;
        const float s1 = live ? half_bits_to_float((uint16_t)(s2 >> 16)) : 0.0f;
        int z0 = (int)(z2 & 0xF), z1 = (int)(z2 >> 4);
        z0 -= (z0 & 8) << 1;
        z1 -= (z1 & 8) << 1;
        const float c0 = XK == kF16 ? (float)z0 : 136.0f + (float)z0;
        const float c1 = XK == kF16 ? (float)z1 : 136.0f + (float)z1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // halves of other segments accumulate what is never read
            const float x0 = xsum[hm[h] * G + 2 * jc], x1 = xsum[hm[h] * G + 2 * jc + 1];
            acc[h] = fmaf(s0, fmaf(-c0, x0, d[2 * h]), acc[h]);
            acc[h] = fmaf(s1, fmaf(-c1, x1, d[2 * h + 1]), acc[h]);
        }
    }

    W4G64_STAMP(4);
    // ---- 5. reduction over segments and K parts, then the outputs ----
    float* red = (float*)(smem + L.red);  // [wave][m][r][SW]
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (hu[h]) red[((wave * M + hm[h]) * R + r) * SW + s] = acc[h];
    lds_barrier();
    W4G64_STAMP(5);
    // outputs o = m RW + wr; the thread count is a multiple of RW, so every
    // output of this thread has the row (and bias) of tid % RW
    for (int o = tid; o < M * RW; o += kThreads) {
        const int m = o / RW, wr = o % RW;
        const int n = row0 + wr;
        if (n < N) {
            const int b = wr / R, rr = wr % R;
            float v = 0.0f;
#pragma unroll
            for (int k2 = 0; k2 < NK; ++k2)
#pragma unroll
                for (int s2 = 0; s2 < SW; ++s2) v += red[(((k2 * NR + b) * M + m) * R + rr) * SW + s2];
            const uint32_t half_bits = bias_row & 1 ? bias_word >> 16 : bias_word & 0xFFFFu;
            if (a.bias_kind == kF32) v += __builtin_bit_cast(float, bias_word);
            else if (a.bias_kind == kF16) v += half_bits_to_float((uint16_t)half_bits);
            else if (a.bias_kind == kBF16) v += bf16_bits_to_float(half_bits);
            store_out<XK>(a.y, (int64_t)m * N + n, v);
        }
    }
    W4G64_STAMP(6);
    W4G64_TIMELINE_STORE(a);
}

// ---- one bf16 row of the decode step's MLP entry: residual add + RMSNorm,
// then the paired gate|up projection with the SiLU product as bf16 planes ----
//
// The same layout as gemv_seg_kernel with 4 segments and 4 row blocks of 4
// rows (16 rows per workgroup), its rows the 8 gate rows i0 .. i0 + 7 (row
// blocks 0, 1) and the matching up rows I + i0 .. (row blocks 2, 3), i0 = 8
// (workgroup).  Staging: every thread below K / 8 loads 8 values of the
// residual, the delta and the norm weight; the others load 16-byte chunks
// of the two rows' scale spans and zero-byte spans.  s = bf16(x + delta)
// (workgroup 0 stores it), the squares' fp32 sum per thread, a wave sum per
// wave and the four waves' sums after one barrier give r = rsqrt(mean + eps);
// the activation bf16(bf16(s r) w) goes to LDS as the bf16 kernel's does.
// The epilogue stores h = silu(bf16(gate)) * bf16(up) as three bf16 planes.
struct SegNormArgs {
    const uint16_t* resid;   // [K] bf16 residual row
    const uint16_t* delta;   // [K] bf16
    const uint16_t* norm_w;  // [K] bf16
    float eps;
    uint16_t* out_sum;       // [K] bf16: resid + delta (workgroup 0)
    const uint8_t* qweight;  // [2 I][K / 2]
    const uint16_t* scales;  // [2 I][G]
    const uint8_t* zeros;    // [2 I][G / 2] bytes
    uint16_t* planes;        // [3][I] bf16
    int I;   // pairs (gate rows), a multiple of 8
    int K;   // in_features (<= 2048: one activation item per thread)
    int G;
    int P;
    W4G64_TIMELINE_FIELDS
};
constexpr int kNormPairs = 8;
constexpr int kNormPlanesThreads = 256;

// LDS layout (bytes): xs [K] | 64 zero bytes | xsum [G] fp32 | scale chunks of
// the gate span then the up span | zero-byte chunks likewise | red [4][4][4]
// fp32 | wave sums [4] fp32.
struct SegNormLayout {
    int zero, xsum, sc, zb, red, wsum, total;
};
__host__ __device__ inline SegNormLayout seg_norm_layout(int K) {
    const int G = K / 64, P = G / 2;
    SegNormLayout L;
    L.zero = K * 2;
    L.xsum = L.zero + 64;
    L.sc = (L.xsum + G * 4 + 15) & ~15;
    L.zb = L.sc + 2 * ((kNormPairs * G * 2 + 32 + 15) & ~15);
    L.red = L.zb + 2 * ((kNormPairs * P + 32 + 15) & ~15);
    L.wsum = L.red + 4 * 4 * 4 * 4;
    L.total = L.wsum + 4 * 4;
    return L;
}

template <int STEPS, int STAGE>
__global__ __launch_bounds__(kNormPlanesThreads) void gemv_seg_norm_planes_kernel(SegNormArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int SW = 4, R = 4;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int K = a.K, G = a.G, P = a.P, I = a.I;
    const SegNormLayout L = seg_norm_layout(K);
    const int i0 = blockIdx.x * kNormPairs;
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);

    // ---- 1. staging loads ----
    // spans h = 0 (gate rows i0 ..) and 1 (up rows I + i0 ..), 16-byte aligned
    int64_t s_lo[2], z_lo[2];
    int SI[2], ZI[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int64_t r0 = (int64_t)h * I + i0;
        s_lo[h] = (r0 * G * 2) & ~15ll;
        const int64_t s_hi = min(((r0 + kNormPairs) * G * 2 + 15) & ~15ll, (int64_t)2 * I * G * 2);
        z_lo[h] = (r0 * P) & ~15ll;
        const int64_t z_hi = min(((r0 + kNormPairs) * P + 15) & ~15ll, (int64_t)2 * I * P);
        SI[h] = (int)((s_hi - s_lo[h]) >> 4);
        ZI[h] = (int)((z_hi - z_lo[h]) >> 4);
    }
    const int XI = K / 8;  // <= kNormPlanesThreads: activation items are u = 0 only
    const int items = XI + SI[0] + SI[1] + ZI[0] + ZI[1];
    u32x4 xr = {0u, 0u, 0u, 0u}, xd = {0u, 0u, 0u, 0u}, xw = {0u, 0u, 0u, 0u};
    u32x4 sv[STAGE];
#pragma unroll
    for (int u = 0; u < STAGE; ++u) {
        int it = kNormPlanesThreads * u + tid;
        it = it < items ? it : items - 1;
        sv[u] = u32x4{0u, 0u, 0u, 0u};
        if (it < XI) {
            xr = *(const u32x4*)(a.resid + 8 * it);
            xd = *(const u32x4*)(a.delta + 8 * it);
            xw = *(const u32x4*)(a.norm_w + 8 * it);
        } else {
            int c = it - XI;
            const uint8_t* src;
            if (c < SI[0]) src = (const uint8_t*)a.scales + s_lo[0] + 16 * (int64_t)c;
            else if ((c -= SI[0]) < SI[1]) src = (const uint8_t*)a.scales + s_lo[1] + 16 * (int64_t)c;
            else if ((c -= SI[1]) < ZI[0]) src = a.zeros + z_lo[0] + 16 * (int64_t)c;
            else src = a.zeros + z_lo[1] + 16 * (int64_t)(c - ZI[0]);
            sv[u] = *(const u32x4*)src;
        }
    }
    asm volatile("" ::: "memory");

    // ---- 2. weight loads: lane (c, q) -> row r, segment s of row block `wave` ----
    const int c = lane & 15;
    const int q = lane >> 4;
    const int r = c / SW;
    const int s = c % SW;
    const int wrow = wave * R + r;              // 0..15: gate rows 0..7, then up rows
    const int half = wrow >> 3;
    const int row = half * I + i0 + (wrow & 7);
    const uint8_t* wsrc = a.qweight + (int64_t)row * (K / 2) + 16 * q;
    u32x4 wv[STEPS];
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int jj = s + SW * t;
        wv[t] = __builtin_nontemporal_load((const u32x4*)(wsrc + 64 * (jj < P ? jj : 0)));
    }
    asm volatile("" ::: "memory");
    asm volatile("" : "+v"(xr), "+v"(xd), "+v"(xw));
#pragma unroll
    for (int u = 0; u < STAGE; ++u) asm volatile("" : "+v"(sv[u]));
    W4G64_STAMP(1);
    wait_vm<STEPS>();  // everything issued before the weights has landed
    W4G64_STAMP(2);

    // ---- 3. residual add and RMSNorm (model.py:40-44, :149-154) ----
    const bool xitem = tid < XI;
    u32x4 sb;
    float pt = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float sv2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float xv = bf16_bits_to_float(h ? xr[e] >> 16 : xr[e] & 0xFFFFu);
            const float dv = bf16_bits_to_float(h ? xd[e] >> 16 : xd[e] & 0xFFFFu);
            sv2[h] = bf16_round(xv + dv);
            pt += __fmul_rn(sv2[h], sv2[h]);
        }
        sb[e] = float_to_bf16_bits(sv2[0]) | ((uint32_t)float_to_bf16_bits(sv2[1]) << 16);
    }
    pt = xitem ? pt : 0.0f;
    if (xitem && blockIdx.x == 0) *(u32x4*)(a.out_sum + 8 * tid) = sb;
    float* wsum = (float*)(smem + L.wsum);
    const float ws = wave_sum64(pt);
    if (lane == 0) wsum[wave] = ws;
    lds_barrier();
    const float rinv = rsqrtf((((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]) / (float)K + a.eps);
    u32x4 xb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float n0 = bf16_round(bf16_bits_to_float(sb[e] & 0xFFFFu) * rinv) * bf16_bits_to_float(xw[e] & 0xFFFFu);
        const float n1 = bf16_round(bf16_bits_to_float(sb[e] >> 16) * rinv) * bf16_bits_to_float(xw[e] >> 16);
        xb[e] = float_to_bf16_bits(n0) | ((uint32_t)float_to_bf16_bits(n1) << 16);
    }
    // ---- 4. staging into LDS: activations (slot order) with their group sums, scale and zero chunks ----
    {
        float gs = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) gs += __builtin_bit_cast(float, xb[e] << 16) + __builtin_bit_cast(float, xb[e] & 0xFFFF0000u);
        gs = dpp_sum8(gs);  // the 8 items of one group sit in 8 aligned lanes (K / 8 is a multiple of 8)
        float* xsum = (float*)(smem + L.xsum);
        if (xitem) {
            *(u32x4*)(smem + 16 * tid) = permute_slots(xb);
            if ((tid & 7) == 0) xsum[tid >> 3] = gs;
        }
#pragma unroll
        for (int u = 0; u < STAGE; ++u) {
            const int it = kNormPlanesThreads * u + tid;
            if (it >= XI && it < items) {
                const int cc = it - XI;
                const int scs = SI[0] + SI[1];
                *(u32x4*)(smem + (cc < scs ? L.sc + 16 * cc : L.zb + 16 * (cc - scs))) = sv[u];
            }
        }
        if (tid < 16) ((uint32_t*)(smem + L.zero))[tid] = 0u;
    }
    lds_barrier();
    W4G64_STAMP(3);

    // ---- 5. MFMA steps (the bf16 path of gemv_seg_kernel, one activation row) ----
    const int ai = lane & 15;
    const int am = ai / (2 * SW), as = (ai >> 1) % SW, ap = ai & 1;
    const bool a_live = am < 1 && (q >> 1) == ap;
    bool hu[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) hu[h] = (2 * q + h) == s;  // one row: segment s' = 2 q + h
    const uint16_t* sc = (const uint16_t*)(smem + L.sc);
    const uint8_t* zb = smem + L.zb;
    const float* xsum = (const float*)(smem + L.xsum);
    const int sc_row = (half ? 8 * SI[0] : 0) + (int)(((int64_t)row * G * 2 - s_lo[half]) >> 1);
    const int zb_row = (half ? 16 * ZI[0] : 0) + (int)((int64_t)row * P - z_lo[half]);
    float acc[2] = {0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int jj = s + SW * t;
        const int ja = as + SW * t;
        const bool live = jj < P;
        const bool alive = a_live && ja < P;
        const unsigned char* asrc = alive ? smem + (128 * ja + 32 * q) * 2 : smem + L.zero;
        u16x8 av[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) av[u] = *(const u16x8*)(asrc + (alive ? 16 * u : 0));
        float4v d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u)
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[u]), dequant8_bf16_biased(wv[t][u]),
                                                        d, 0, 0, 0);
        const int jc = live ? jj : 0;
        const uint32_t s2 = *(const uint32_t*)(sc + sc_row + 2 * jc);
        const uint32_t z2 = zb[zb_row + jc];
        const float s0 = live ? half_bits_to_float((uint16_t)s2) : 0.0f;
        const float s1 = live ? half_bits_to_float((uint16_t)(s2 >> 16)) : 0.0f;
        int z0 = (int)(z2 & 0xF), z1 = (int)(z2 >> 4);
        z0 -= (z0 & 8) << 1;
        z1 -= (z1 & 8) << 1;
        const float c0 = 136.0f + (float)z0, c1 = 136.0f + (float)z1;
        const float x0 = xsum[2 * jc], x1 = xsum[2 * jc + 1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // halves of other segments accumulate what is never read
            acc[h] = fmaf(s0, fmaf(-c0, x0, d[2 * h]), acc[h]);
            acc[h] = fmaf(s1, fmaf(-c1, x1, d[2 * h + 1]), acc[h]);
        }
    }
    W4G64_STAMP(4);

    // ---- 6. segments summed through LDS; the SiLU product as planes ----
    float* red = (float*)(smem + L.red);  // [wave][r][SW]
#pragma unroll
    for (int h = 0; h < 2; ++h)
        if (hu[h]) red[(wave * R + r) * SW + s] = acc[h];
    lds_barrier();
    W4G64_STAMP(5);
    if (tid < kNormPairs) {
        float g = 0.0f, up = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < SW; ++s2) {
            g += red[tid * SW + s2];                     // row tid: block tid / 4, row tid % 4
            up += red[(kNormPairs + tid) * SW + s2];     // row 8 + tid
        }
        store_silu_planes(a.planes, 0, i0 + tid, 1, I, g, up);
    }
    W4G64_STAMP(6);
    W4G64_TIMELINE_STORE(a);
}

template <int XK, int SW, int NR, int NK, int STEPS>
hipError_t launch_seg3(const SegArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                       hipEvent_t stop) {
    const dim3 grid(plan.n_blocks), block(NR * NK * 64);
    switch (plan.stage) {  // staging loads per lane
        case 1: return launch_kernel(gemv_seg_kernel<XK, SW, NR, NK, STEPS, 1>, grid, block, (size_t)plan.lds_bytes, stream, start, stop, args);
        case 2: return launch_kernel(gemv_seg_kernel<XK, SW, NR, NK, STEPS, 2>, grid, block, (size_t)plan.lds_bytes, stream, start, stop, args);
        case 4: return launch_kernel(gemv_seg_kernel<XK, SW, NR, NK, STEPS, 4>, grid, block, (size_t)plan.lds_bytes, stream, start, stop, args);
        default: return hipErrorInvalidValue;
    }
}

template <int XK, int SW, int NR, int NK>
hipError_t launch_seg2(const SegArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                       hipEvent_t stop) {
    switch (plan.steps) {
#define W4G64_SEG_STEPS(S) \
    case S: return launch_seg3<XK, SW, NR, NK, S>(args, plan, stream, start, stop);
        W4G64_SEG_STEPS(1) W4G64_SEG_STEPS(2) W4G64_SEG_STEPS(3)
#undef W4G64_SEG_STEPS
        default: return hipErrorInvalidValue;
    }
}

template <int XK>
hipError_t launch_seg1(const SegArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                       hipEvent_t stop) {
    const int sw = plan.segments, nr = plan.fblocks, nk = plan.kparts;
#define W4G64_SEG_SHAPE(S, A, B) \
    if (sw == S && nr == A && nk == B) return launch_seg2<XK, S, A, B>(args, plan, stream, start, stop);
    W4G64_SEG_SHAPE(4, 4, 1)
    W4G64_SEG_SHAPE(4, 1, 4)
#undef W4G64_SEG_SHAPE
    return hipErrorInvalidValue;
}

}  // namespace

// (segments, row blocks, K parts) shapes the lean kernel is built for
constexpr int64_t kSegMaxLds = 64 * 1024;

// The planner takes one row: measured with graph replays over cold weight
// copies it is ahead of the segmented kernel for q/k/v/o 1536x1536 and
// 256x1536 (3.4 / 2.95 us against 3.4 / 3.2) and gate/up 8960x1536 (4.9-5.1
// against 5.1-5.2), behind it for the long-K down projection (6.5 against
// 5.6 at four K parts of five steps) and at four rows (gate 5.8 against 5.2),
// so it takes at most three 16-byte steps per lane.  The kernel itself
// handles up to eight rows.
bool plan_seg(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, GemvPlan& plan) {
    if (rows != 1 || (x_kind != kF16 && x_kind != kBF16)) return false;
    const int64_t G = in_features / 64;
    if (G % 2 || out_features % 2 || (out_features * G * 2) % 16 || (out_features * (G / 2)) % 16) return false;
    const int64_t P = G / 2;
    const int sw = 4;  // 4 output rows x 256 contiguous bytes per load instruction
    int nr = 4, nk = 1;
    // fewer than ~256 workgroups with whole rows: split K over the workgroup's waves
    if ((out_features + 4 * (16 / sw) - 1) / (4 * (16 / sw)) < 256) {
        nr = 1;
        nk = 4;
    }
    const int R = 16 / sw, RW = nr * R, W = nr * nk;
    const int64_t PK = (P + nk - 1) / nk;
    const int64_t need = (PK + sw - 1) / sw;
    if (need > 3) return false;
    const int steps = (int)need;
    const int64_t lds = seg_layout((int)rows, (int)in_features, RW, W, R, sw).total;
    if (lds > kSegMaxLds) return false;
    // staging chunks: activations, and the (16-byte rounded) scale and zero spans of RW rows
    const int64_t items = rows * in_features / 8 + (RW * G * 2 + 32) / 16 + (RW * P + 32) / 16 + 2;
    int64_t stage = (items + W * 64 - 1) / (W * 64);
    stage = stage <= 1 ? 1 : stage <= 2 ? 2 : stage <= 4 ? 4 : 0;
    if (!stage) return false;
    plan = GemvPlan{};
    plan.kind = 2;
    plan.segments = sw;
    plan.fblocks = nr;
    plan.kparts = nk;
    plan.stage = (int)stage;
    plan.steps = steps;
    plan.tiles = 1;
    plan.n_blocks = (int)((out_features + RW - 1) / RW);
    plan.splits = 1;
    plan.groups_per_split = (int)PK;
    plan.lds_bytes = lds;
    return true;
}

bool seg_supported(const LinearProblem& p) {
    return ((uintptr_t)p.scales % 16) == 0 && ((uintptr_t)p.zeros % 16) == 0 && ((uintptr_t)p.qweight % 16) == 0 &&
           ((uintptr_t)p.x % 16) == 0 && ((uintptr_t)p.bias % 4) == 0 && !p.paired && p.norm_delta == nullptr;
}

// The one-row RMSNorm + gate|up planes form of the lean kernel: bf16
// residual and delta, no bias, I = out_features / 2 a multiple of 8, in_features
// a multiple of 128 of at most 1536 (three 16-byte weight steps per lane).
bool plan_seg_norm_planes(const LinearProblem& p, GemvPlan& plan) {
    if (p.rows != 1 || p.x_kind != kNormB || !p.paired || p.bias || p.norm_delta_parts != 1) return false;
    if (p.out_features % 16 || p.in_features % 128 || p.in_features > 1536 || p.out_features > kGemvMaxOutFeatures)
        return false;
    if (((uintptr_t)p.scales % 16) || ((uintptr_t)p.zeros % 16) || ((uintptr_t)p.qweight % 16)) return false;
    const int64_t G = p.in_features / 64, P = G / 2, I = p.out_features / 2;
    const int steps = (int)((P + 3) / 4);
    // items: activation chunks, then both spans' scale and zero-byte chunks (a span of
    // L bytes at any offset covers at most (L + 30) / 16 aligned 16-byte chunks)
    const int64_t items = p.in_features / 8 + 2 * ((kNormPairs * G * 2 + 30) / 16) + 2 * ((kNormPairs * P + 30) / 16);
    const int stage = (int)((items + kNormPlanesThreads - 1) / kNormPlanesThreads);
    if (steps < 1 || steps > 3 || stage > 2) return false;
    plan = GemvPlan{};
    plan.kind = 3;
    plan.segments = 4;
    plan.fblocks = 4;
    plan.kparts = 1;
    plan.steps = steps;
    plan.stage = stage;
    plan.tiles = 1;
    plan.n_blocks = (int)(I / kNormPairs);
    plan.splits = 1;
    plan.groups_per_split = (int)P;
    plan.lds_bytes = seg_norm_layout((int)p.in_features).total;
    return true;
}

hipError_t launch_gemv_seg_norm_planes(const LinearProblem& p, const GemvPlan& plan, hipStream_t stream) {
    SegNormArgs a{};
    a.resid = (const uint16_t*)p.x;
    a.delta = (const uint16_t*)p.norm_delta;
    a.norm_w = p.norm_weight;
    a.eps = p.norm_eps;
    a.out_sum = (uint16_t*)p.norm_out_sum;
    a.qweight = p.qweight;
    a.scales = p.scales;
    a.zeros = p.zeros;
    a.planes = (uint16_t*)p.y;
    a.I = (int)(p.out_features / 2);
    a.K = (int)p.in_features;
    a.G = a.K / 64;
    a.P = a.G / 2;
    W4G64_TIMELINE_SET(a);
    const dim3 grid(plan.n_blocks), block(kNormPlanesThreads);
    const size_t lds = (size_t)plan.lds_bytes;
#define W4G64_NORM_PLANES(S, T)                                                                                     \
    if (plan.steps == S && plan.stage == T)                                                                         \
        return launch_kernel(gemv_seg_norm_planes_kernel<S, T>, grid, block, lds, stream, nullptr, nullptr, a);
    W4G64_NORM_PLANES(1, 1) W4G64_NORM_PLANES(2, 1) W4G64_NORM_PLANES(3, 1)
    W4G64_NORM_PLANES(1, 2) W4G64_NORM_PLANES(2, 2) W4G64_NORM_PLANES(3, 2)
#undef W4G64_NORM_PLANES
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_seg(const LinearProblem& p, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                           hipEvent_t stop) {
    SegArgs args{};
    args.x = p.x;
    args.qweight = p.qweight;
    args.scales = p.scales;
    args.zeros = p.zeros;
    args.bias = p.bias;
    args.y = p.y;
    args.bias_kind = p.bias_kind;
    args.M = (int)p.rows;
    args.N = (int)p.out_features;
    args.K = (int)p.in_features;
    args.G = (int)(p.in_features / 64);
    args.P = args.G / 2;
    args.PK = plan.groups_per_split;
    W4G64_TIMELINE_SET(args);
    if (args.M < 1 || args.M > 8 || args.G % 2 || args.PK < 1) return hipErrorInvalidValue;
    switch (p.x_kind) {
        case kF16: return launch_seg1<kF16>(args, plan, stream, start, stop);
        case kBF16: return launch_seg1<kBF16>(args, plan, stream, start, stop);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace w4g64
