/*
 * w4g64_oracle.c -- CPU restatement of the reference's canonical W4G64 codec,
 * quantizers, group-wise dequantization and fp32 linear.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it is linked by the
 * tests, by the smoke check and by the CPU-baseline leg of bench.py, never by
 * the HIP product library.  Every function cites the reference code it
 * restates (paths relative to the reference repository root).
 *
 * Pins (see tests/test_oracle_*.py):
 *   - o_pack_int4 / o_unpack_int4: exhaustive 256-byte and 16x16-pair tables
 *     against the closed form, plus the reference's known-answer vectors.
 *   - o_dequantize_w4g64: exhaustive code x zero table; the closed form is
 *     exact in fp32; reference known-answer vectors.
 *   - o_quantize_symmetric_rtn / o_quantize_asymmetric_rtn: hand-derived
 *     vectors with round-half-even ties and fp32-vs-fp16 scale traps, range
 *     and error-bound invariants, and an independent numpy restatement.
 *   - o_linear_f32: brute-force double accumulation; one-hot/linearity
 *     properties and the reference's exact zero-point boundary case.
 *   - f32<->f16/bf16 conversions: checked against numpy/torch conversions.
 *
 * Build: oracle/Makefile (gcc -O2, no fast-math: IEEE fp32 semantics are
 * part of the contract).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define O_OK 0
#define O_EINVAL 1

/* ------------------------------------------------------------------ */
/* IEEE half / bfloat16 conversions (round to nearest, ties to even), as  */
/* torch's .to(torch.float16) / .to(torch.bfloat16) on CPU.               */
/* ------------------------------------------------------------------ */

uint16_t o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t absx = x & 0x7FFFFFFFu;
    if (absx >= 0x7F800000u) {                 /* inf / nan */
        if (absx > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((absx >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    uint32_t e = absx >> 23;
    uint32_t m = absx & 0x7FFFFFu;
    if (e >= 113) {                            /* normal half range or overflow */
        uint32_t r = ((e - 112) << 10) | (m >> 13);
        uint32_t rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1;
        if (r >= 0x7C00u) r = 0x7C00u;         /* rounds past max -> inf */
        return (uint16_t)(sign | r);
    }
    /* subnormal half (or zero): count of 2^-24 units */
    uint32_t shift = 126 - e;                  /* e<=112 -> shift>=14 */
    if (shift > 31) return (uint16_t)sign;
    uint64_t m24 = (e == 0) ? (uint64_t)m : ((uint64_t)m | 0x800000u);
    uint64_t r = m24 >> shift;
    uint64_t rem = m24 & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (r & 1u))) r += 1;
    return (uint16_t)(sign | (uint32_t)r);
}

float o_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0x1F) {
        x = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else {                                   /* subnormal half: m * 2^-24 */
        float v = (float)m * 5.9604644775390625e-08f;
        memcpy(&x, &v, 4);
        x |= sign;
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t o_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);  /* quiet nan */
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float o_bf16_to_f32(uint16_t b) {
    uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------ */
/* INT4 codec: src/qwen_int4/quantization.py:17-84                      */
/* packing: 0 = CANONICAL (low nibble K-even), 1 = LEGACY_SIGNED_ADD.    */
/* ------------------------------------------------------------------ */

/* pack_int4, quantization.py:30-50 (validation :23-27). */
int o_pack_int4(const int8_t* codes, int64_t count, int packing, uint8_t* out) {
    if (count % 2) return O_EINVAL;
    for (int64_t i = 0; i < count; ++i)
        if (codes[i] < -8 || codes[i] > 7) return O_EINVAL;
    for (int64_t i = 0; i < count / 2; ++i) {
        int32_t first = codes[2 * i], second = codes[2 * i + 1];
        int32_t packed = packing == 1 ? (first << 4) + second            /* :46-47 */
                                      : (first & 0x0F) | ((second & 0x0F) << 4); /* :49 */
        out[i] = (uint8_t)(packed & 0xFF);
    }
    return O_OK;
}

/* unpack_int4, quantization.py:53-84.  `elements` < 0 means "all". */
int o_unpack_int4(const uint8_t* packed, int64_t nbytes, int packing, int64_t elements, int8_t* out) {
    int64_t total = 2 * nbytes;
    if (elements < 0) elements = total;
    if (elements > total) return O_EINVAL;                                  /* :80-82 */
    for (int64_t i = 0; i < nbytes; ++i) {
        int32_t low_u = packed[i] & 0x0F, high_u = packed[i] >> 4;
        if (packing == 1) high_u = (high_u + (low_u >= 8)) & 0x0F;         /* :65-68 */
        int32_t low = low_u >= 8 ? low_u - 16 : low_u;                      /* :70-71 */
        int32_t high = high_u >= 8 ? high_u - 16 : high_u;
        int32_t even = packing == 1 ? high : low, odd = packing == 1 ? low : high;  /* :72-78 */
        if (2 * i < elements) out[2 * i] = (int8_t)even;
        if (2 * i + 1 < elements) out[2 * i + 1] = (int8_t)odd;
    }
    return O_OK;
}

/* dequantize_groupwise, quantization.py:221-258:
 *   W[n,k] = (code[n,k] - zero[n, k/gs]) * f32(scale[n, k/gs]).
 * zeros may be NULL (the `zeros is None` branch, :244-245). */
int o_dequantize_groupwise(const uint8_t* qweight, int64_t qweight_bytes, const uint16_t* scales_f16,
                           const uint8_t* zeros, int64_t zero_bytes, int64_t out_features,
                           int64_t in_features, int64_t group_size, int packing, float* out) {
    if (group_size <= 0 || in_features % group_size) return O_EINVAL;       /* :232-233 */
    int64_t groups = in_features / group_size;
    if (qweight_bytes != out_features * in_features / 2) return O_EINVAL;   /* :239-241 */
    if (zeros && zero_bytes != (out_features * groups + 1) / 2) return O_EINVAL; /* :247-251 */
    for (int64_t n = 0; n < out_features; ++n) {
        for (int64_t k = 0; k < in_features; ++k) {
            int64_t e = n * in_features + k;
            uint8_t b = qweight[e >> 1];
            int32_t low_u = b & 0x0F, high_u = b >> 4;
            if (packing == 1) high_u = (high_u + (low_u >= 8)) & 0x0F;
            int32_t nib = packing == 1 ? ((e & 1) ? low_u : high_u) : ((e & 1) ? high_u : low_u);
            int32_t code = nib >= 8 ? nib - 16 : nib;
            int64_t g = k / group_size;
            int32_t zero = 0;
            if (zeros) {
                int64_t ze = n * groups + g;
                uint8_t zb = zeros[ze >> 1];
                int32_t zl = zb & 0x0F, zh = zb >> 4;
                if (packing == 1) zh = (zh + (zl >= 8)) & 0x0F;
                int32_t zn = packing == 1 ? ((ze & 1) ? zl : zh) : ((ze & 1) ? zh : zl);
                zero = zn >= 8 ? zn - 16 : zn;
            }
            float s = o_f16_to_f32(scales_f16[n * groups + g]);
            out[e] = (float)(code - zero) * s;                               /* :258 */
        }
    }
    return O_OK;
}

/* ------------------------------------------------------------------ */
/* Quantizers                                                           */
/* ------------------------------------------------------------------ */

/* quantize_symmetric_rtn, quantization.py:87-111.
 * s = amax|w|/7 (fp32), s==0 -> 1; q = clamp(rne(w/s), -7, 7); codes use the
 * fp32 scale, the stored scale is fp16(s).  qweight gets N*K/2 bytes. */
int o_quantize_symmetric_rtn(const float* w, int64_t out_features, int64_t in_features,
                             int64_t group_size, int packing, uint8_t* qweight, uint16_t* scales_f16) {
    if (group_size <= 0 || in_features % group_size) return O_EINVAL;       /* :101-102 */
    int64_t groups = in_features / group_size;
    for (int64_t n = 0; n < out_features; ++n) {
        for (int64_t g = 0; g < groups; ++g) {
            const float* row = w + n * in_features + g * group_size;
            float amax = 0.0f;
            for (int64_t i = 0; i < group_size; ++i) {
                float a = fabsf(row[i]);
                if (a > amax || isnan(a)) amax = a;
            }
            float s = amax / 7.0f;                                           /* :107 */
            if (s == 0.0f) s = 1.0f;                                         /* :108 */
            scales_f16[n * groups + g] = o_f32_to_f16(s);                   /* :111 */
            for (int64_t i = 0; i < group_size; i += 2) {
                float q0 = nearbyintf(row[i] / s), q1 = nearbyintf(row[i + 1] / s);  /* :109 */
                q0 = q0 < -7.0f ? -7.0f : (q0 > 7.0f ? 7.0f : q0);
                q1 = q1 < -7.0f ? -7.0f : (q1 > 7.0f ? 7.0f : q1);
                int8_t pair[2] = {(int8_t)q0, (int8_t)q1};
                o_pack_int4(pair, 2, packing, qweight + (n * in_features + g * group_size + i) / 2);
            }
        }
    }
    return O_OK;
}

/* quantize_asymmetric_rtn, quantization.py:114-162 (clip_max optional,
 * :137-147).  Logical u in [0,15] is stored as signed u-8 (:156-157); an odd
 * zero count is padded with a 0 code (:158-159) and the signed zero list is
 * packed with the same packing as the codes (:161).  zeros gets (N*G+1)/2
 * bytes. */
int o_quantize_asymmetric_rtn(const float* w, int64_t out_features, int64_t in_features,
                              int64_t group_size, const float* clip_max, int packing,
                              uint8_t* qweight, uint16_t* scales_f16, uint8_t* zeros) {
    if (group_size <= 0 || in_features % group_size) return O_EINVAL;
    int64_t groups = in_features / group_size;
    if (clip_max)
        for (int64_t i = 0; i < out_features * groups; ++i)
            if (!isfinite(clip_max[i]) || clip_max[i] <= 0.0f) return O_EINVAL;  /* :143-144 */
    int64_t zcount = out_features * groups;
    int64_t zpadded = zcount + (zcount & 1);
    int8_t* signed_zeros = (int8_t*)calloc((size_t)(zpadded > 0 ? zpadded : 1), 1);
    if (!signed_zeros) return O_EINVAL;
    for (int64_t n = 0; n < out_features; ++n) {
        for (int64_t g = 0; g < groups; ++g) {
            const float* row = w + n * in_features + g * group_size;
            float lim = clip_max ? clip_max[n * groups + g] : 0.0f;
            float vmin = INFINITY, vmax = -INFINITY;
            for (int64_t i = 0; i < group_size; ++i) {
                float v = row[i];
                if (clip_max) v = fmaxf(fminf(v, lim), -lim);                 /* :145-147 */
                if (v < vmin) vmin = v;
                if (v > vmax) vmax = v;
            }
            float mn = vmin < 0.0f ? vmin : 0.0f;                            /* :150 */
            float mx = vmax > 0.0f ? vmax : 0.0f;                            /* :151 */
            float range = mx - mn;
            if (range < 1e-5f) range = 1e-5f;
            float s = range / 15.0f;                                         /* :152 */
            float zf = nearbyintf(-mn / s);                                  /* :153 */
            zf = zf < 0.0f ? 0.0f : (zf > 15.0f ? 15.0f : zf);
            int32_t uz = (int32_t)zf;
            scales_f16[n * groups + g] = o_f32_to_f16(s);
            for (int64_t i = 0; i < group_size; i += 2) {
                int8_t pair[2];
                for (int j = 0; j < 2; ++j) {
                    float v = row[i + j];
                    if (clip_max) v = fmaxf(fminf(v, lim), -lim);
                    float u = nearbyintf(v / s) + (float)uz;                 /* :154-155 */
                    u = u < 0.0f ? 0.0f : (u > 15.0f ? 15.0f : u);
                    pair[j] = (int8_t)((int32_t)u - 8);                      /* :156 */
                }
                o_pack_int4(pair, 2, packing, qweight + (n * in_features + g * group_size + i) / 2);
            }
            signed_zeros[n * groups + g] = (int8_t)(uz - 8);                 /* :157 */
        }
    }
    int rc = o_pack_int4(signed_zeros, zpadded, packing, zeros);             /* :158-161 */
    free(signed_zeros);
    return rc;
}

/* ------------------------------------------------------------------ */
/* Linear: backends.py:73-98 (torch_reference_linear).                  */
/*   y = x_f32 @ W^T + bias_f32, accumulated here in double and rounded  */
/*   once to fp32 (the most accurate fp32 answer; the reference's BLAS   */
/*   order is unpinned).  x and y are fp32; callers convert dtypes.      */
/* ------------------------------------------------------------------ */
void o_linear_f32(const float* x, int64_t rows, const float* w, int64_t out_features,
                  int64_t in_features, const float* bias, float* y) {
    for (int64_t m = 0; m < rows; ++m) {
        for (int64_t n = 0; n < out_features; ++n) {
            double acc = 0.0;
            const float* xr = x + m * in_features;
            const float* wr = w + n * in_features;
            for (int64_t k = 0; k < in_features; ++k) acc += (double)xr[k] * (double)wr[k];
            float r = (float)acc;
            if (bias) r = r + bias[n];                                      /* :96-97 */
            y[m * out_features + n] = r;
        }
    }
}

/* Convenience: fp32 array -> fp16 / bf16 bit arrays and back. */
void o_f32_to_f16_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = o_f32_to_f16(in[i]);
}
void o_f32_to_bf16_array(const float* in, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = o_f32_to_bf16(in[i]);
}
void o_f16_to_f32_array(const uint16_t* in, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = o_f16_to_f32(in[i]);
}
