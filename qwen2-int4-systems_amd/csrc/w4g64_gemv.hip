// Decode path: fused unpack + dequant + GEMV for 1..16 activation rows.
//
// y[m, n] = sum_g scale[n,g] * sum_{k in g} x[m,k] * (code[n,k] - zero[n,g])   (+ bias[n])
// which is the reference's (x.float() @ W.t() + bias).to(x.dtype)
// (src/qwen_int4/backends.py:73-98) with the group scale applied once per
// 64-wide group in fp32.
//
// MFMA mapping (v_mfma_f32_16x16x32_{f16,bf16}, two per 64-wide group):
//   * B columns j = (row r, segment s), r < 16/SW, s < SW: a wave covers
//     16/SW output features over the workgroup's K range, which is cut into SW
//     segments taking the range's groups round robin (segment s takes groups
//     g0 + s, g0 + s + SW, ...).  Lane (j = lane % 16, q = lane / 16) loads
//     8 packed bytes per group (the 16-value quarter q of the group), so one
//     wave load instruction reads SW consecutive groups of each of its rows.
//   * A rows i = (virtual activation row m, segment s), i = m * SW + s.  Only
//     the block diagonal of D (segment of row i == segment of column j) is
//     used: at M <= 16 the matrix core has far more throughput than the HBM
//     stream needs, so the off-diagonal products are free, and they let one
//     wave own as little as one output feature -- enough workgroups to fill
//     the chip without reducing across workgroups.
//   * fp16 activations: B = (code - zero) exact, built with the 1024+n' magic
//     and one v_pk_add_f16 per pair; the group scale multiplies the MFMA
//     result in fp32.
//   * bf16 activations: B = 128 + n' (exact in bf16); the group result is
//     corrected by -(136 + zero) * sum_{k in g} x[m,k] before scaling.
//   * fp32 activations: every row is split exactly into three bf16 parts
//     (hi + mid + lo == x), staged as three planes; each group step runs the
//     three planes through the MFMA against the same decoded weights, into
//     one fp32 accumulator (the parts lengthen K, not the A rows, so one row
//     still leaves 16 segments per wave).
//   * fused activation form (decode step of the decoder layer): kSwiGLU
//     stages silu(gate) * up (fp32, as three bf16 parts) from a [gate | up]
//     bf16 row; kPlanes stages the three parts from three bf16 planes
//     written by the paired gate|up epilogue (below), with no arithmetic.
//   * paired epilogue (fused gate|up projection of the decoder layer, bf16):
//     a wave's R features are R/2 gate rows i and the R/2 up rows I + i of
//     the same i, so the wave computes h = silu(bf16(gate)) * bf16(up) in
//     fp32 (model.py:133-135) once per value and stores its exact three-way
//     bf16 split (hi + mid + lo == h) as three planes [3][M][I].
//   * every wave first issues its share of the workgroup's activation loads,
//     then every weight, scale and zero load of its steps (raw bits; decoded
//     where the MFMA step uses them).  A wave's loads return in issue order,
//     so the activations arrive first; they go to LDS (with the bf16 group
//     sums reduced across lanes) and a barrier over LDS alone lets every wave
//     start on its first weight step while the rest of the weights stream in.
//   * each wave owns whole output features (all their segments and fp32
//     parts), so the epilogue reduces within the wave, with no workgroup
//     barrier.
//   * optional K split across workgroups (long K at several rows): each
//     workgroup stores its fp32 partial sums, and a second kernel in the same
//     stream adds them in split order (deterministic), adds the bias and
//     stores the output; the kernel boundary makes the partials visible.
//     (An in-kernel last-arriver merge needs an agent-scope release and
//     acquire per workgroup, which measured 3.7-6.3 us per call here against
//     about 2 us for the second launch.)
#include <stdio.h>

#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kMaxSteps = 16;  // group steps per lane in one workgroup
constexpr int kStepBuckets[] = {2, 3, 6, 9, 12, 16};

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

struct GemvArgs {
    const void* x;
    const uint8_t* qweight;
    const uint16_t* scales;
    const uint8_t* zeros;
    const void* bias;
    int bias_kind;
    void* y;
    int M;       // activation rows
    int N;       // out_features
    int K;       // in_features
    int G;       // K / 64
    int gps;     // groups per K split
    int splits;  // K splits across workgroups
    int mv;      // A rows in use (= M)
    float* partials;  // [splits][M][N]
    int paired;          // paired gate|up epilogue (y = bf16 planes [3][M][N/2])
    // RMSNorm prologue (kNormB / kNormF / kNormP): x is the residual stream
    const void* delta;
    int delta_parts;  // kNormP: partial sums [delta_parts][M][K] in delta
    const uint16_t* norm_w;
    float eps;
    uint16_t* out_sum;
    W4G64_TIMELINE_FIELDS
};

// Activation items (8 values each) a lane stages: M x groups-per-split x 8
// items over the workgroup's lanes, where M <= 16 TILES / SW (planes kind:
// 3 M <= 16 TILES / SW) and groups-per-split <= SW STEPS.
// The RMSNorm kinds take one row: SW STEPS groups x 8 items over 256 lanes.
template <int XK, int SW, int STEPS, int TILES>
constexpr int stage_items() {
    if constexpr (XK == kNormB || XK == kNormF || XK == kNormP) return (SW * STEPS + 31) / 32;
    return XK == kPlanes ? (TILES * STEPS + 5) / 6 : (TILES * STEPS + 1) / 2;
}

// Sum over the 8 lanes 8i..8i+7; every one of them gets the same bits.
__device__ __forceinline__ float sum8_lanes(float s) {
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0xB1, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x4E, 0xF, 0xF, false));
    s += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x141, 0xF, 0xF, false));
    return s;
}

template <int XK, int SW, int STEPS, int TILES>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    // fp32-class activations are staged as three bf16 planes; the fp32 and
    // SwiGLU kinds run them along K (three MFMA pairs per group step into
    // separate accumulators), the planes kind as A rows (virtual row p M + m,
    // a third of the LDS reads and MFMAs per weight byte; the epilogue sums
    // the three rows' results)
    constexpr int kStaged = (XK == kF32 || XK == kSwiGLU || XK == kPlanes) ? 3 : 1;
    constexpr int kParts = (XK == kF32 || XK == kSwiGLU) ? 3 : 1;  // along K
    constexpr int kRowParts = XK == kPlanes ? 3 : 1;                // as A rows
    constexpr bool kNorm = XK == kNormB || XK == kNormF || XK == kNormP;
    constexpr int kOut = (XK == kSwiGLU || XK == kPlanes) ? kF32 : (kNorm ? kBF16 : XK);  // output kind
    constexpr int R = 16 / SW;              // output features per wave
    constexpr int kBlockCols = kWaves * R;  // output features per workgroup
    constexpr int kStage = stage_items<XK, SW, STEPS, TILES>();
    // 16-byte loads per item (norm kinds: residual, delta, norm weight)
    // (kNormP: residual, two per partial sum, norm weight)
    constexpr int kVecs = (XK == kF16 || XK == kBF16) ? 1
                          : (XK == kPlanes || XK == kNormB ? 3
                                                           : (XK == kNormF ? 4 : (XK == kNormP ? 2 + 2 * kMaxDeltaParts : 2)));

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    W4G64_TIMELINE_DECL;
    W4G64_STAMP(0);
    const int nb = blockIdx.x;
    const int split = blockIdx.y;
    const int g0 = split * a.gps;
    const int cnt = min(a.gps, a.G - g0);  // groups in this workgroup's K range
    const int row_stride = a.gps * 64 + 8;  // 16-bit elements per staged row (+16 B pad)
    const int planes = kStaged * a.M;       // staged rows: part p of row m is plane row p M + m
    uint16_t* xs = (uint16_t*)smem;         // [planes][row_stride], slot order
    float* sx = (float*)(smem + (size_t)planes * row_stride * 2);  // [planes][gps] group sums (bf16/fp32)
    float* red = sx + planes * a.gps;                               // [M][kBlockCols][SW]

    // ---- this lane's column: output feature n, segment sj ----
    const int j = lane & 15;
    const int q = lane >> 4;
    const int rj = j / SW;
    const int sj = j % SW;
    // Output feature of slot (nb, wave, rj): slot order, or -- paired -- the
    // wave's first R/2 slots are gate rows i and the last R/2 the up rows
    // I + i of the same i (I = N / 2).
    const int half_n = a.N >> 1;
    auto slot_feature = [&](int slot_in_block, int& i_out) {
        const int w = slot_in_block / R, r = slot_in_block % R;
        if (!a.paired) {
            i_out = nb * kBlockCols + slot_in_block;
            return i_out;
        }
        i_out = (nb * kBlockCols + w * R) / 2 + r % (R / 2 > 0 ? R / 2 : 1);
        return (r >= R / 2 ? half_n : 0) + i_out;
    };
    int n_i;
    const int n = slot_feature(wave * R + rj, n_i);
    const bool nvalid = a.paired ? n_i < half_n : n < a.N;
    const int nrow = nvalid ? n : 0;
    u32x2 wq[STEPS];
    // raw scale bits and zero bytes: decoded where used, so that issuing a
    // step's loads never waits for an earlier step's data
    uint32_t sraw[STEPS];
    uint32_t zraw[STEPS];
    const uint8_t* wrow = a.qweight + (int64_t)nrow * (a.K / 2) + 8 * q;
    const int64_t sbase = (int64_t)nrow * a.G;

    // ---- 1. activation loads: item it = kThreads u + tid (8 values of row m) ----
    // Lanes past the last item take the item at the same place in the last
    // group instead, so they load, sum and store exactly what that group's
    // own lanes do (identical bytes to the same addresses): no branch
    // anywhere before the MFMA loop.
    const int kbase = g0 * 64;
    const int items_per_row = cnt * 8;
    const int total = a.M * items_per_row;
    const float inv_items = 1.0f / (float)items_per_row;
    // item -> (row m, item c in the row); it < 2^24, so the float quotient is
    // off by at most one
    auto item_rc = [&](int it, int& m, int& c) {  // branch-free
        m = (int)((float)it * inv_items);
        c = it - m * items_per_row;
        const int adj = (int)(c >= items_per_row) - (int)(c < 0);
        m += adj;
        c -= adj * items_per_row;
    };
    u32x4 v[kStage][kVecs];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
        const int it = kThreads * u + tid;
        int m, c;
        item_rc(it < total ? it : total - 8 + (tid & 7), m, c);
        if constexpr (XK == kF16 || XK == kBF16) {
            v[u][0] = *(const u32x4*)((const uint16_t*)a.x + (int64_t)m * a.K + kbase + 8 * c);
        } else if constexpr (XK == kSwiGLU) {
            // x is [M, 2K]: gate | up (bf16)
            const uint16_t* gu = (const uint16_t*)a.x + (int64_t)m * 2 * a.K + kbase + 8 * c;
            v[u][0] = *(const u32x4*)gu;
            v[u][1] = *(const u32x4*)(gu + a.K);
        } else if constexpr (XK == kPlanes) {
            // x is [3][M][K] bf16: the hi, mid and lo parts
#pragma unroll
            for (int pl = 0; pl < 3; ++pl)
                v[u][pl] = *(const u32x4*)((const uint16_t*)a.x + ((int64_t)pl * a.M + m) * a.K + kbase + 8 * c);
        } else if constexpr (kNorm) {
            // residual (bf16), delta (bf16 or fp32), norm weight (bf16); the K range is the whole row
            v[u][0] = *(const u32x4*)((const uint16_t*)a.x + (int64_t)m * a.K + 8 * c);
            if constexpr (XK == kNormB) {
                v[u][1] = *(const u32x4*)((const uint16_t*)a.delta + (int64_t)m * a.K + 8 * c);
            } else if constexpr (XK == kNormF) {
                const float* dsrc = (const float*)a.delta + (int64_t)m * a.K + 8 * c;
                v[u][1] = *(const u32x4*)dsrc;
                v[u][2] = *(const u32x4*)(dsrc + 4);
            } else {
                // every partial sum's item; parts past delta_parts re-read the last one
#pragma unroll
                for (int pt = 0; pt < kMaxDeltaParts; ++pt) {
                    const int pc = min(pt, a.delta_parts - 1);
                    const float* dsrc = (const float*)a.delta + ((int64_t)pc * a.M + m) * a.K + 8 * c;
                    v[u][1 + 2 * pt] = *(const u32x4*)dsrc;
                    v[u][2 + 2 * pt] = *(const u32x4*)(dsrc + 4);
                }
            }
            v[u][kVecs - 1] = *(const u32x4*)(a.norm_w + 8 * c);
        } else {
            const float* src = (const float*)a.x + (int64_t)m * a.K + kbase + 8 * c;
            v[u][0] = *(const u32x4*)src;
            v[u][1] = *(const u32x4*)(src + 4);
        }
    }
    // (the empty asm statements with a memory clobber fix the issue order)
    asm volatile("" ::: "memory");

    // ---- 2. weight / scale / zero loads of every step ----
    // Unconditional (steps past the K range re-read group g0 and get a zero
    // scale), in step order, so that step t is complete once the lane's first
    // 3 (t + 1) weight-side loads have returned.
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const int gl = sj + SW * t;
        const int g = gl < cnt ? g0 + gl : g0;
        wq[t] = __builtin_nontemporal_load((const u32x2*)(wrow + (int64_t)g * 32));
        sraw[t] = a.scales[sbase + g];
        zraw[t] = a.zeros[(sbase + g) >> 1];
        asm volatile("" ::: "memory");
    }
    // Nothing that uses the activations may move above the last load issue.
#pragma unroll
    for (int u = 0; u < kStage; ++u)
#pragma unroll
        for (int k = 0; k < kVecs; ++k) asm volatile("" : "+v"(v[u][k]));
    W4G64_STAMP(1);

    // ---- 3a. RMSNorm prologue (model.py:40-44, residual adds :149-154) ----
    // s = bf16(x + bf16(delta)); the activation is bf16(bf16(s * r) * w) with
    // r = rsqrt(mean(s^2) + eps) over the whole row (squares rounded before
    // the fp32 sum, as x.pow(2) is).  Workgroup (0, 0) stores s.  One row (the
    // decode step): each thread sums the squares of its items, a wave sum
    // each, the four waves' sums added in order after one barrier.  More
    // rows: per-item sums in LDS, reduced per row by wave 0.
    float r_one = 0.0f;
    if constexpr (kNorm) {
        float* nsq = red + a.mv * kBlockCols * SW;  // [M][items per row] partial sums of squares
        float* rinv = nsq + a.M * items_per_row;    // [M]
        const bool writer = nb == 0 && split == 0;
        const bool one_row = a.M == 1;
        float pt = 0.0f;
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int it = kThreads * u + tid;
            const int itc = it < total ? it : total - 8 + (tid & 7);
            int m, c;
            item_rc(itc, m, c);
            float ps = 0.0f;
            u32x4 sb;
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float sv[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t xw = v[u][0][e / 2];
                    const float xv = bf16_bits_to_float(h ? xw >> 16 : xw & 0xFFFFu);
                    float dv;
                    if constexpr (XK == kNormB) {
                        const uint32_t dw = v[u][1][e / 2];
                        dv = bf16_bits_to_float(h ? dw >> 16 : dw & 0xFFFFu);
                    } else if constexpr (XK == kNormF) {
                        const uint32_t bits = v[u][1 + (e + h) / 4][(e + h) % 4];  // element to a scalar first
                        dv = bf16_round(__builtin_bit_cast(float, bits));
                    } else {
                        // the split-K reduction's sum: parts in order from 0, then + 0 (no bias)
                        float t = 0.0f;
#pragma unroll
                        for (int pt = 0; pt < kMaxDeltaParts; ++pt) {
                            const uint32_t bits = v[u][1 + 2 * pt + (e + h) / 4][(e + h) % 4];
                            t = pt < a.delta_parts ? t + __builtin_bit_cast(float, bits) : t;
                        }
                        dv = bf16_round(t + 0.0f);
                    }
                    sv[h] = bf16_round(xv + dv);
                    ps += __fmul_rn(sv[h], sv[h]);
                }
                sb[e / 2] = float_to_bf16_bits(sv[0]) | ((uint32_t)float_to_bf16_bits(sv[1]) << 16);
            }
            v[u][0] = sb;  // s replaces the residual item
            if (one_row) pt += it < total ? ps : 0.0f;  // clamped items repeat a real one
            else nsq[itc] = ps;
            if (writer) *(u32x4*)(a.out_sum + (int64_t)m * a.K + 8 * c) = sb;
        }
        if (one_row) {
            const float wsum = wave_sum64(pt);
            if (lane == 0) nsq[wave] = wsum;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            float sq = nsq[0];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) sq += nsq[w];
            r_one = rsqrtf(sq / (float)a.K + a.eps);
        } else {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            if (wave == 0) {
                for (int m = 0; m < a.M; ++m) {
                    float sq = 0.0f;
                    for (int l = lane; l < items_per_row; l += 64) sq += nsq[m * items_per_row + l];
#pragma unroll
                    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
                    if (lane == 0) rinv[m] = rsqrtf(sq / (float)a.K + a.eps);
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
#pragma unroll
        for (int u = 0; u < kStage; ++u) {
            const int it = kThreads * u + tid;
            int m, c;
            item_rc(it < total ? it : total - 8 + (tid & 7), m, c);
            const float r = one_row ? r_one : rinv[m];
            u32x4 nbits;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t sw2 = v[u][0][e], ww = v[u][kVecs - 1][e];
                const float n0 = bf16_round(bf16_bits_to_float(sw2 & 0xFFFFu) * r) * bf16_bits_to_float(ww & 0xFFFFu);
                const float n1 = bf16_round(bf16_bits_to_float(sw2 >> 16) * r) * bf16_bits_to_float(ww >> 16);
                nbits[e] = float_to_bf16_bits(n0) | ((uint32_t)float_to_bf16_bits(n1) << 16);
            }
            v[u][0] = nbits;  // the bf16 activation item
        }
    }

    // ---- 3. activations into LDS (slot order) and group sums ----
    // The 8 items of one (row, group) sit in lanes 8i..8i+7 of one u, so a
    // group sum is a reduction over those 8 lanes, and all 8 store it.
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
        const int it = kThreads * u + tid;
        int m, c;
        item_rc(it < total ? it : total - 8 + (tid & 7), m, c);
        const int gl = c >> 3;
        if constexpr (XK == kF16) {
            *(u32x4*)(xs + m * row_stride + 8 * c) = permute_slots(v[u][0]);
        } else if constexpr (XK == kBF16 || kNorm) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                s += __builtin_bit_cast(float, v[u][0][e] << 16) + __builtin_bit_cast(float, v[u][0][e] & 0xFFFF0000u);
            s = sum8_lanes(s);
            *(u32x4*)(xs + m * row_stride + 8 * c) = permute_slots(v[u][0]);
            sx[m * a.gps + gl] = s;
        } else if constexpr (XK == kPlanes) {
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                float ps = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ps += __builtin_bit_cast(float, v[u][pl][e] << 16) + __builtin_bit_cast(float, v[u][pl][e] & 0xFFFF0000u);
                ps = sum8_lanes(ps);
                *(u32x4*)(xs + (pl * a.M + m) * row_stride + 8 * c) = permute_slots(v[u][pl]);
                sx[(pl * a.M + m) * a.gps + gl] = ps;
            }
        } else {
            float h[8];
            if constexpr (XK == kSwiGLU) {
                // h = silu(gate) * up in fp32, silu(g) = g / (1 + exp(-g)) (model.py:133-136)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t gw = v[u][0][e / 2], uw = v[u][1][e / 2];
                    const float g = bf16_bits_to_float(e & 1 ? gw >> 16 : gw & 0xFFFFu);
                    const float up = bf16_bits_to_float(e & 1 ? uw >> 16 : uw & 0xFFFFu);
                    h[e] = (g / (1.0f + expf(-g))) * up;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t bits = v[u][e / 4][e % 4];  // element to a scalar before the cast
                    h[e] = __builtin_bit_cast(float, bits);
                }
            }
            uint16_t hi[8], mid[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) split3_bf16(h[e], hi[e], mid[e], lo[e]);
            u32x4 pp[3];
            float ps[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                pp[0][e] = (uint32_t)hi[2 * e] | ((uint32_t)hi[2 * e + 1] << 16);
                pp[1][e] = (uint32_t)mid[2 * e] | ((uint32_t)mid[2 * e + 1] << 16);
                pp[2][e] = (uint32_t)lo[2 * e] | ((uint32_t)lo[2 * e + 1] << 16);
            }
#pragma unroll
            for (int p = 0; p < 3; ++p) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ps[p] += __builtin_bit_cast(float, pp[p][e] << 16) + __builtin_bit_cast(float, pp[p][e] & 0xFFFF0000u);
                ps[p] = sum8_lanes(ps[p]);
            }
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                *(u32x4*)(xs + (p * a.M + m) * row_stride + 8 * c) = permute_slots(pp[p]);
                sx[(p * a.M + m) * a.gps + gl] = ps[p];
            }
        }
    }
    W4G64_STAMP(2);
    // A barrier over LDS alone: the weight loads stay in flight through it.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    W4G64_STAMP(3);

    // ---- 4. MFMA over the group steps ----
    // One accumulator per fp32 part: the bf16 path's biased codes make each
    // part's group result a difference of two large terms, so the parts are
    // kept apart until the end (their magnitudes differ by 2^8 and 2^16).
    float4v acc[TILES][kParts];
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt)
#pragma unroll
        for (int p = 0; p < kParts; ++p) acc[tt][p] = float4v{0.f, 0.f, 0.f, 0.f};

    // Branch-free: every LDS read is in bounds and unconditional, so the
    // reads of a step need no exec-mask branches around them.  Out-of-range
    // operands read staged (finite) data instead of zeros: A rows past the
    // virtual rows only feed D rows the epilogue drops, and a step past the K
    // range has zero scale.  (Reading several steps ahead measured slower:
    // the registers cost more occupancy than the overlap gained.)
    {
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            // A operands of this step from LDS first (A row il = row m,
            // segment il % SW; one operand pair per fp32 part) ...
            u16x8 a0[TILES][kParts], a1[TILES][kParts];
#pragma unroll
            for (int tt = 0; tt < TILES; ++tt) {
                const int il = 16 * tt + (lane & 15);
                const int m = min(il / SW, a.mv - 1);
                const int ga = min(il % SW + SW * t, cnt - 1);  // the A row's group, local to the K range
#pragma unroll
                for (int p = 0; p < kParts; ++p) {
                    const uint16_t* src = xs + (p * a.M + m) * row_stride + 64 * ga + 16 * q;
                    a0[tt][p] = *(const u16x8*)src;
                    a1[tt][p] = *(const u16x8*)(src + 8);
                }
            }
            // ... then wait for this step's weight, scale and zero alone: the
            // empty asm keeps their decoding here (hoisted next to the loads,
            // it would make the later loads' issue wait for these).
            asm volatile("" : "+v"(wq[t]), "+v"(sraw[t]), "+v"(zraw[t]));
            const uint32_t s_bits = sraw[t], z_bits = zraw[t];
            const int gl = sj + SW * t;  // this lane's group, local to the K range
            const float scale = (nvalid && gl < cnt) ? half_bits_to_float((uint16_t)s_bits) : 0.0f;
            const int gz = gl < cnt ? g0 + gl : g0;  // the group this step loaded
            const int zn = (((sbase + gz) & 1) ? (z_bits >> 4) : z_bits) & 0xF;
            const int zr_t = zn - ((zn & 8) << 1);
            const int glc = min(gl, cnt - 1);
#pragma unroll
            for (int tt = 0; tt < TILES; ++tt) {
                float4v d[kParts];
                if constexpr (XK == kF16) {
                    const _Float16 zl = (_Float16)(1032 + zr_t);
                    const _Float16 zh = (_Float16)(72 + zr_t);
                    const half8 b0 = dequant8_f16_int(wq[t][0], half2v{zl, zl}, half2v{zh, zh});
                    const half8 b1 = dequant8_f16_int(wq[t][1], half2v{zl, zl}, half2v{zh, zh});
                    d[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a0[tt][0]), b0,
                                                                  float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    d[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a1[tt][0]), b1, d[0], 0, 0, 0);
                } else {
                    const bf16x8 b0 = dequant8_bf16_biased(wq[t][0]);
                    const bf16x8 b1 = dequant8_bf16_biased(wq[t][1]);
#pragma unroll
                    for (int p = 0; p < kParts; ++p) {
                        d[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a0[tt][p]), b0,
                                                                       float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        d[p] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1[tt][p]), b1, d[p], 0,
                                                                       0, 0);
                    }
                    // D rows i = 16 tt + 4 q + r.  The rows kept later share this
                    // lane's segment, so their group is this lane's group gl.
                    const float corr = 136.0f + (float)zr_t;
                    if constexpr (SW >= 4) {
                        // the lane's 4 D rows 4q..4q+3 lie in one segment block: one row mi
                        const int mi = min((16 * tt + 4 * q) / SW, a.mv - 1);
#pragma unroll
                        for (int p = 0; p < kParts; ++p) {
                            const float gs = sx[(p * a.M + mi) * a.gps + glc];
#pragma unroll
                            for (int r = 0; r < 4; ++r) d[p][r] = fmaf(-corr, gs, d[p][r]);
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int mi = min((16 * tt + 4 * q + r) / SW, a.mv - 1);
#pragma unroll
                            for (int p = 0; p < kParts; ++p)
                                d[p][r] = fmaf(-corr, sx[(p * a.M + mi) * a.gps + glc], d[p][r]);
                        }
                    }
                }
#pragma unroll
                for (int p = 0; p < kParts; ++p)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[tt][p][r] = fmaf(scale, d[p][r], acc[tt][p][r]);
            }
        }
    }

    W4G64_STAMP(4);
    // ---- 5. epilogue (per wave): keep the block diagonal, sum the segments ----
    // The wave writes and reads only its own features' slots of `red`; LDS
    // operations of one wave complete in order, so no barrier is needed.
#pragma unroll
    for (int tt = 0; tt < TILES; ++tt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * tt + 4 * q + r;
            const int m = i / SW;
            float v = acc[tt][0][r];
#pragma unroll
            for (int p = 1; p < kParts; ++p) v += acc[tt][p][r];
            if (i % SW == sj && m < a.mv) red[(m * kBlockCols + wave * R + rj) * SW + sj] = v;
        }
    }
    W4G64_STAMP(5);
    const int col0 = nb * kBlockCols;
    if constexpr (R >= 2) {  // paired plans keep at most 8 segments (R >= 2)
        if (a.paired && a.splits == 1) {
            // gate and up of the same i are in this wave: h straight to the planes
            for (int idx = lane; idx < a.M * (R / 2); idx += 64) {
                const int m = idx / (R / 2);
                const int c = idx - m * (R / 2);
                int i;
                slot_feature(wave * R + c, i);
                if (i >= half_n) continue;
                float g = 0.0f, up = 0.0f;
#pragma unroll
                for (int s = 0; s < SW; ++s) {
                    g += red[(m * kBlockCols + wave * R + c) * SW + s];
                    up += red[(m * kBlockCols + wave * R + R / 2 + c) * SW + s];
                }
                store_silu_planes(a.y, m, i, a.M, half_n, g + load_bias(a.bias, a.bias_kind, i),
                                  up + load_bias(a.bias, a.bias_kind, half_n + i));
            }
            W4G64_STAMP(6);
            W4G64_TIMELINE_STORE(a);
            return;
        }
    }
    for (int idx = lane; idx < a.M * R; idx += 64) {
        const int m = idx / R;
        const int c = wave * R + (idx - m * R);
        int i;
        const int nn = slot_feature(c, i);
        if (a.paired ? i >= half_n : nn >= a.N) continue;
        float v = 0.0f;
#pragma unroll
        for (int rp = 0; rp < kRowParts; ++rp)
#pragma unroll
            for (int s = 0; s < SW; ++s) v += red[((rp * a.M + m) * kBlockCols + c) * SW + s];
        if (a.splits == 1) {
            v += load_bias(a.bias, a.bias_kind, nn);
            store_out<kOut>(a.y, (int64_t)m * a.N + nn, v);
        } else {
            a.partials[((int64_t)split * a.M + m) * a.N + nn] = v;
        }
    }
    W4G64_STAMP(6);
    W4G64_TIMELINE_STORE(a);
}

// Second kernel of a K-split call: one thread per output (paired: per
// (row, i) pair of gate and up features).
struct SplitReduceArgs {
    const float* partials;
    const void* bias;
    int bias_kind;
    void* y;
    int M;
    int N;
    int splits;
};

template <int OUT, bool PAIRED>
__global__ __launch_bounds__(256) void split_reduce_kernel(SplitReduceArgs r) {
    const int cols = PAIRED ? r.N / 2 : r.N;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)r.M * cols) return;
    const int m = (int)(idx / cols);
    const int c = (int)(idx - (int64_t)m * cols);
    const int64_t stride = (int64_t)r.M * r.N;
    // Up to 8 splits' loads are issued before the first add (a dependent
    // load-add chain would pay one memory latency per split); the adds run in
    // split order, so the sum is deterministic.
    auto total = [&](int nn) {
        const float* src = r.partials + (int64_t)m * r.N + nn;
        float v = 0.0f;
        for (int s0 = 0; s0 < r.splits; s0 += 8) {
            float part[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) part[u] = src[min(s0 + u, r.splits - 1) * stride];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s0 + u < r.splits) v += part[u];
        }
        return v + load_bias(r.bias, r.bias_kind, nn);
    };
    if constexpr (PAIRED) store_silu_planes(r.y, m, c, r.M, cols, total(c), total(cols + c));
    else store_out<OUT>(r.y, (int64_t)m * r.N + c, total(c));
}

template <int XK, int SW, int STEPS, int TILES>
hipError_t launch_typed(const GemvArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                        hipEvent_t stop, bool unreduced) {
    // the staging capacity of this instantiation (the planner never exceeds it)
    if ((int64_t)args.M * args.gps * 8 > (int64_t)stage_items<XK, SW, STEPS, TILES>() * kThreads) return hipErrorInvalidValue;
    constexpr bool kNorm = XK == kNormB || XK == kNormF || XK == kNormP;
    constexpr int kOut = (XK == kSwiGLU || XK == kPlanes) ? kF32 : (kNorm ? kBF16 : XK);
    const bool split = plan.splits > 1 && !unreduced;
    hipError_t err = launch_kernel(gemv_kernel<XK, SW, STEPS, TILES>, dim3(plan.n_blocks, plan.splits),
                                   dim3(kThreads), (size_t)plan.lds_bytes, stream, start, split ? nullptr : stop, args);
    if (err != hipSuccess || !split) return err;
    return launch_split_reduce(args.partials, args.bias, args.bias_kind, args.y, args.M, args.N, args.splits,
                               args.paired != 0, kOut, stream, stop);
}

template <int XK, int SW, int TILES>
hipError_t launch_steps(const GemvArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                        hipEvent_t stop, bool unreduced) {
    switch (plan.steps) {
        case 2: return launch_typed<XK, SW, 2, TILES>(args, plan, stream, start, stop, unreduced);
        case 3: return launch_typed<XK, SW, 3, TILES>(args, plan, stream, start, stop, unreduced);
        case 6: return launch_typed<XK, SW, 6, TILES>(args, plan, stream, start, stop, unreduced);
        case 9: return launch_typed<XK, SW, 9, TILES>(args, plan, stream, start, stop, unreduced);
        case 12: return launch_typed<XK, SW, 12, TILES>(args, plan, stream, start, stop, unreduced);
        default: return launch_typed<XK, SW, 16, TILES>(args, plan, stream, start, stop, unreduced);
    }
}

template <int XK, int TILES>
hipError_t launch_sw(const GemvArgs& args, const GemvPlan& plan, hipStream_t stream, hipEvent_t start,
                     hipEvent_t stop, bool unreduced) {
    switch (plan.segments) {
        case 16: return launch_steps<XK, 16, TILES>(args, plan, stream, start, stop, unreduced);
        case 8: return launch_steps<XK, 8, TILES>(args, plan, stream, start, stop, unreduced);
        case 4: return launch_steps<XK, 4, TILES>(args, plan, stream, start, stop, unreduced);
        case 2: return launch_steps<XK, 2, TILES>(args, plan, stream, start, stop, unreduced);
        default: return launch_steps<XK, 1, TILES>(args, plan, stream, start, stop, unreduced);
    }
}

}  // namespace

constexpr int kRows16Buckets[] = {2, 3, 6, 9, 12, 18};  // steps of the 9..16-row kernel
constexpr int64_t kDeviceCUs = 256;                        // MI355X compute units

// 9..16 fp16/bf16 rows: fblocks 16-feature blocks per workgroup, `waves`
// waves per block taking its K range's groups round robin; the range's
// activations are staged in LDS (at most ~60 KB: 28 groups at 16 rows).
// Measured at 16 rows (fp16, cold weights, eager events): K = 1536 runs best
// as one block of 8 waves (3 steps; q 1536x1536 4.2 us) while that leaves at
// most two workgroups per CU; with more 16-feature blocks (gate 8960x1536:
// 560) as three blocks of 4 waves, one 48-feature workgroup per CU that
// stages the activations once (8.8 -> 8.0 us fp16, 9.2 -> 8.3 us bf16, 8.2 ->
// 8.0 us at 12 rows).  K = 8960 runs as two blocks of 4 waves over the 5 K
// splits the LDS budget needs (down 1536x8960 11.2 us).  More splits, or 8
// waves over 6+ steps (133 VGPRs: one such workgroup per CU, two dispatch
// rounds), measured slower.
bool plan_rows16(int64_t rows, int64_t out_features, int64_t in_features, GemvPlan& plan, int force_fblocks,
                 int force_waves, int force_splits) {
    if (rows < 9 || rows > 16) return false;
    const int64_t groups = in_features / 64;
    plan = GemvPlan{};
    plan.kind = 1;
    plan.segments = 1;
    plan.tiles = 1;
    const bool short_k = groups <= 48;
    const bool wide = (out_features + 15) / 16 > 2 * kDeviceCUs;  // more than two 16-feature blocks per CU
    plan.fblocks = force_fblocks > 0 ? force_fblocks : (short_k ? (wide ? 3 : 1) : 2);
    plan.waves = force_waves > 0 ? force_waves : (plan.fblocks == 1 ? (short_k ? 8 : 4) : 4);
    const int fb = plan.fblocks, kw = plan.waves;
    if (!((fb == 1 && (kw == 4 || kw == 8)) || (fb == 2 && (kw == 2 || kw == 4)) || (fb == 3 && kw == 4) ||
          (fb == 4 && (kw == 1 || kw == 2))))
        return false;
    plan.n_blocks = (int)((out_features + 16 * fb - 1) / (16 * fb));
    auto lds_for = [&](int64_t g) { return rows * (g * 64 + 8) * 2 + rows * g * 4; };
    int64_t splits = force_splits > 0 ? force_splits : 1;
    int64_t gps = (groups + splits - 1) / splits;
    while (lds_for(gps) > 60 * 1024 || (gps + kw - 1) / kw > 18) {
        ++splits;
        gps = (groups + splits - 1) / splits;
    }
    splits = (groups + gps - 1) / gps;
    plan.splits = (int)splits;
    plan.groups_per_split = (int)gps;
    const int64_t need = (gps + kw - 1) / kw;
    plan.steps = 18;
    for (int b : kRows16Buckets)
        if (b >= need) {
            plan.steps = b;
            break;
        }
    plan.lds_bytes = lds_for(gps);
    plan.workspace_bytes = splits > 1 ? splits * rows * out_features * 4 : 0;
    return true;
}

namespace {

// The segmented kernel's plan for `sw` segments and at least `min_splits` K
// splits (more when a lane would need more than kMaxSteps group steps or
// the staged activations would not fit the 60 KB LDS budget).
GemvPlan plan_segmented(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, int64_t sw,
                        int64_t min_splits) {
    GemvPlan plan{};
    const int64_t groups = in_features / 64;
    const int64_t mv = rows * (x_kind == kPlanes ? 3 : 1);
    const int64_t planes = rows * ((x_kind == kF32 || x_kind == kSwiGLU || x_kind == kPlanes) ? 3 : 1);
    const int64_t cols = kWaves * (16 / sw);
    plan.segments = (int)sw;
    plan.tiles = (int)((mv * sw + 15) / 16);
    plan.n_blocks = (int)((out_features + cols - 1) / cols);
    int64_t splits = min_splits > 0 ? min_splits : 1;
    int64_t gps = (groups + splits - 1) / splits;
    // staged activations (virtual rows x split width, 16-bit), the group
    // sums and the epilogue's per-segment results
    // (norm kinds: plus the per-item partial sums of squares and the row factors)
    const int64_t norm_extra =
        (x_kind == kNormB || x_kind == kNormF || x_kind == kNormP) ? rows * (in_features / 64) * 8 * 4 + rows * 4 : 0;
    auto lds_for = [&](int64_t g) {
        return planes * (g * 64 + 8) * 2 + planes * g * 4 + mv * kWaves * 16 * 4 + norm_extra;
    };
    while (lds_for(gps) > 60 * 1024 || (gps + sw - 1) / sw > kMaxSteps) {
        ++splits;
        gps = (groups + splits - 1) / splits;
    }
    splits = (groups + gps - 1) / gps;
    plan.splits = (int)splits;
    plan.groups_per_split = (int)gps;
    const int64_t need = (gps + sw - 1) / sw;
    plan.steps = kMaxSteps;
    for (int b : kStepBuckets)
        if (b >= need) {
            plan.steps = b;
            break;
        }
    plan.lds_bytes = lds_for(gps);
    plan.workspace_bytes = splits > 1 ? splits * rows * out_features * 4 : 0;
    return plan;
}
}  // namespace

GemvPlan plan_gemv(int64_t rows, int64_t out_features, int64_t in_features, int x_kind, int force_segments,
                   int force_splits) {
    GemvPlan plan{};
    if (rows > 8 && rows <= 16 && (x_kind == kF16 || x_kind == kBF16) && force_segments <= 0 && force_splits <= 0 &&
        plan_rows16(rows, out_features, in_features, plan, 0, 0, 0))
        return plan;
    const int64_t groups = in_features / 64;
    const int64_t mv = rows * (x_kind == kPlanes ? 3 : 1);
    const bool fp32_class = x_kind == kF32 || x_kind == kSwiGLU;
    // Segments: as many as fit the 16 MFMA rows (mv * SW <= 16), then fewer
    // while that still leaves >= 1024 column blocks (more features per
    // workgroup = more reuse of the staged activations).
    int64_t sw = 1;
    while (sw < 16 && mv * sw * 2 <= 16) sw *= 2;
    auto blocks_for = [&](int64_t s) {
        const int64_t cols = kWaves * (16 / s);
        return (out_features + cols - 1) / cols;
    };
    while (sw > 1 && blocks_for(sw / 2) >= 1024) sw /= 2;
    // RMSNorm kinds stage the whole residual row (and the delta) in every
    // workgroup: 8 segments (twice the features per workgroup) measured
    // better at one row (q|k|v 2048x1536 with an fp32 delta 4.53 -> 3.89 us,
    // with six fp32 partial sums 5.77 -> 4.75 us; gate|up unchanged)
    if ((x_kind == kNormB || x_kind == kNormF || x_kind == kNormP) && sw > 8) sw = 8;
    if (force_segments > 0 || force_splits > 0)
        return plan_segmented(rows, out_features, in_features, x_kind, force_segments > 0 ? force_segments : sw,
                              force_splits);
    // K splits: a lane holds at most kMaxSteps group steps.  With few column
    // blocks, split further to fill the chip -- but a split adds a cross-
    // workgroup merge, which only pays while each lane keeps >= 5 group steps
    // (fp16/bf16, measured: q at 4 rows 6.3 -> 5.0 us unsplit, down at 4 rows
    // 11.2 -> 9.6 us with 6 splits instead of 3).  The fp32-class kinds stage
    // their activations at a higher cost per workgroup and keep the old rule
    // (the SwiGLU down projection at 1 row: 3 splits 9.9 us, 6 splits 11.2 us).
    int64_t splits = (groups + sw * kMaxSteps - 1) / (sw * kMaxSteps);
    if (!fp32_class) {
        while (blocks_for(sw) * splits < 2 * kDeviceCUs && splits * 2 <= groups && groups >= splits * 2 * sw * 5)
            splits *= 2;
    } else {
        while (blocks_for(sw) * splits < kDeviceCUs && splits * 2 <= groups && groups / (splits * 2) >= sw) splits *= 2;
    }
    return plan_segmented(rows, out_features, in_features, x_kind, sw, splits);
}

GemvPlan plan_gemv(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    return plan_gemv(rows, out_features, in_features, x_kind, 0, 0);
}

GemvPlan plan_gemv_paired(int64_t rows, int64_t out_features, int64_t in_features, int x_kind) {
    GemvPlan plan = plan_gemv(rows, out_features, in_features, x_kind, 0, 0);
    if (plan.kind == 1 || plan.segments > 8)
        plan = plan_gemv(rows, out_features, in_features, x_kind, plan.kind == 1 ? 1 : 8, 0);
    return plan;
}

const char* gemv_kernel_name(const GemvPlan& plan, int x_kind) {
    static thread_local char name[96];
    static const char* kinds[] = {"?", "f16", "bf16", "f32", "?", "swiglu_bf16", "planes_bf16", "rmsnorm_bf16",
                                  "rmsnorm_f32delta"};
    if (plan.kind == 4) {
        // the pipelined kernel's activation form comes from the plan
        static const char* forms[] = {"", "planes_bf16", "rmsnorm_bf16", "rmsnorm_partials"};
        const char* form = plan.form >= 1 && plan.form <= 3 ? forms[plan.form] : kinds[x_kind >= 1 && x_kind <= 8 ? x_kind : 0];
        snprintf(name, sizeof(name), "gemv_pipe_kernel<%s%s%s,%d,%d,%d,%d,%d,%d,%d>", form, plan.pair ? "_gate_up" : "",
                 plan.form == kGrouped ? "_grouped" : "", plan.segments, plan.tiles, plan.fblocks, plan.kparts, plan.rbw, plan.steps, plan.depth);
        return name;
    }
    if (plan.kind == 2) {
        snprintf(name, sizeof(name), "gemv_seg_kernel<%s,%d,%d,%d,%d>", kinds[x_kind >= 1 && x_kind <= 8 ? x_kind : 0],
                 plan.segments, plan.fblocks, plan.kparts, plan.steps);
        return name;
    }
    if (plan.kind == 1) {
        snprintf(name, sizeof(name), "gemv16_kernel<%s,%d,%d,%d>", kinds[x_kind >= 1 && x_kind <= 8 ? x_kind : 0], plan.steps,
                 plan.waves, plan.fblocks);
        return name;
    }
    snprintf(name, sizeof(name), "gemv_kernel<%s,%d,%d,%d>", kinds[x_kind >= 1 && x_kind <= 8 ? x_kind : 0], plan.segments, plan.steps,
             plan.tiles);
    return name;
}

hipError_t launch_gemv(const LinearProblem& p, const GemvPlan& plan, void* workspace, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
    if (plan.kind == 1) return launch_gemv16(p, plan, workspace, stream, start, stop);
    GemvArgs args{};
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
    args.mv = (int)(p.rows * (p.x_kind == kPlanes ? 3 : 1));
    if (plan.tiles != 1 && p.x_kind != kPlanes) return hipErrorInvalidValue;  // rows <= 16 fit one A tile
    args.paired = p.paired;
    const bool norm = p.x_kind == kNormB || p.x_kind == kNormF || p.x_kind == kNormP;
    if (p.paired && ((p.x_kind != kBF16 && !norm) || plan.segments > 8 || (p.out_features & 1)))
        return hipErrorInvalidValue;
    // the norm prologue needs the whole row in every workgroup
    if (norm && (plan.kind != 0 || plan.splits != 1 || !p.norm_delta || !p.norm_weight || !p.norm_out_sum))
        return hipErrorInvalidValue;
    args.delta = p.norm_delta;
    args.delta_parts = p.norm_delta_parts;
    if (p.x_kind == kNormP && (p.norm_delta_parts < 1 || p.norm_delta_parts > kMaxDeltaParts)) return hipErrorInvalidValue;
    args.norm_w = p.norm_weight;
    args.eps = p.norm_eps;
    args.out_sum = (uint16_t*)p.norm_out_sum;
    W4G64_TIMELINE_SET(args);
    // unreduced: the partial sums (or, unsplit, the fp32 result) go to the caller's buffer
    const bool unreduced = p.partials_out != nullptr;
    if (unreduced) {
        constexpr int kNoOut = -1;
        const int out_kind = (p.x_kind == kSwiGLU || p.x_kind == kPlanes || p.x_kind == kF32) ? kF32 : kNoOut;
        if (out_kind != kF32 || p.bias || p.paired) return hipErrorInvalidValue;
        args.y = p.partials_out;
    }
    args.partials = unreduced ? p.partials_out : (float*)workspace;
    switch (p.x_kind) {
        case kF16:
            return launch_sw<kF16, 1>(args, plan, stream, start, stop, unreduced);
        case kBF16:
            return launch_sw<kBF16, 1>(args, plan, stream, start, stop, unreduced);
        case kSwiGLU:
            return launch_sw<kSwiGLU, 1>(args, plan, stream, start, stop, unreduced);
        case kNormB:
            return launch_sw<kNormB, 1>(args, plan, stream, start, stop, unreduced);
        case kNormF:
            return launch_sw<kNormF, 1>(args, plan, stream, start, stop, unreduced);
        case kNormP:
            return launch_sw<kNormP, 1>(args, plan, stream, start, stop, unreduced);
        case kPlanes:
            // 3 rows x rows: more than 16 virtual rows only with one segment per wave
            if (plan.tiles == 1) return launch_sw<kPlanes, 1>(args, plan, stream, start, stop, unreduced);
            if (plan.segments != 1 || plan.tiles > 3) return hipErrorInvalidValue;
            if (plan.tiles == 2) return launch_steps<kPlanes, 1, 2>(args, plan, stream, start, stop, unreduced);
            return launch_steps<kPlanes, 1, 3>(args, plan, stream, start, stop, unreduced);
        default:
            return launch_sw<kF32, 1>(args, plan, stream, start, stop, unreduced);
    }
}

hipError_t launch_split_reduce(const float* partials, const void* bias, int bias_kind, void* y, int M, int N,
                               int splits, bool paired, int out_kind, hipStream_t stream, hipEvent_t stop) {
    SplitReduceArgs r{partials, bias, bias_kind, y, M, N, splits};
    if (!partials || splits < 2 || (paired && (N & 1))) return hipErrorInvalidValue;
    const int64_t items = (int64_t)M * (paired ? N / 2 : N);
    const dim3 grid((unsigned)((items + 255) / 256));
    if (paired) return launch_kernel(split_reduce_kernel<kF32, true>, grid, dim3(256), 0, stream, nullptr, stop, r);
    switch (out_kind) {
        case kF16: return launch_kernel(split_reduce_kernel<kF16, false>, grid, dim3(256), 0, stream, nullptr, stop, r);
        case kBF16: return launch_kernel(split_reduce_kernel<kBF16, false>, grid, dim3(256), 0, stream, nullptr, stop, r);
        case kF32: return launch_kernel(split_reduce_kernel<kF32, false>, grid, dim3(256), 0, stream, nullptr, stop, r);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace w4g64
