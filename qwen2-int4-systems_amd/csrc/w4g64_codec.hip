// Canonical INT4 unpack and W4G64 dequantization primitives (bit-exact).
//
// unpack:  out[i] = sext4((packed[i >> 1] >> 4*(i & 1)) & 0xF)
//          (reference: src/qwen_int4/quantization.py:53-84; the GPU primitive
//          it mirrors is triton_kernels.py:22-35)
// dequant: out[n,k] = (code[n,k] - zero[n,k/64]) * f32(scale[n,k/64])
//          (quantization.py:221-258; triton_kernels.py:38-63).  (code - zero)
//          is an integer in [-15, 15] and the scale an fp16 value, so the
//          fp32 product is exact and every correct implementation agrees
//          bit for bit.
//
// Both kernels are HBM-bound streams: one packed dword (8 values) per thread
// step, 16-byte vector stores, grid-stride loops sized to fill all CUs.
#include "w4g64_device.h"
#include "w4g64_internal.h"

namespace w4g64 {
namespace {

// Sign-extend the 4 nibbles held in the low half of each byte of v.
__device__ __forceinline__ uint32_t sext_nibbles(uint32_t v) {
    return v | ((v & 0x08080808u) * 0x1Eu);  // 0x08 * 0x1E = 0xF0 per byte, no carries
}

__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t* __restrict__ packed,
                                                      int8_t* __restrict__ out, int64_t elements) {
    const int64_t full_dwords = elements / 8;  // dwords whose 8 values are all in range
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; d < full_dwords; d += stride) {
        const uint8_t* src = packed + 4 * d;
        uint32_t w = (uint32_t)src[0] | ((uint32_t)src[1] << 8) | ((uint32_t)src[2] << 16) |
                     ((uint32_t)src[3] << 24);
        uint32_t lo = sext_nibbles(w & 0x0F0F0F0Fu);         // k even
        uint32_t hi = sext_nibbles((w >> 4) & 0x0F0F0F0Fu);  // k odd
        u32x2 o;
        o[0] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);   // lo.b0 hi.b0 lo.b1 hi.b1
        o[1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);   // lo.b2 hi.b2 lo.b3 hi.b3
        if ((((uintptr_t)out) & 7) == 0) {
            *(u32x2*)(out + 8 * d) = o;
        } else {
            for (int j = 0; j < 8; ++j) out[8 * d + j] = (int8_t)(((j < 4) ? o[0] : o[1]) >> (8 * (j & 3)));
        }
    }
    // Tail: the last (elements % 8) values, one thread each.
    const int64_t tail_start = full_dwords * 8;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t < elements - tail_start) out[tail_start + t] = (int8_t)nibble_at(packed, tail_start + t);
}

__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ qweight,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint8_t* __restrict__ zeros,
                                                       float* __restrict__ out, int64_t out_features,
                                                       int64_t in_features) {
    const int64_t dwords_per_row = in_features / 8;
    const int64_t groups = in_features / 64;
    const int64_t total = out_features * dwords_per_row;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const uint32_t* q32 = (const uint32_t*)qweight;
    for (int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; d < total; d += stride) {
        const int64_t n = d / dwords_per_row;
        const int64_t k0 = (d - n * dwords_per_row) * 8;
        const int64_t g = k0 / 64;
        const float s = half_bits_to_float(scales[n * groups + g]);
        const int z = nibble_at(zeros, n * groups + g);
        const uint32_t w = q32[d];
        float4v a, b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            int nib = (w >> (4 * j)) & 0xF;
            int code = nib - ((nib & 8) << 1);
            float v = (float)(code - z) * s;
            if (j < 4) a[j] = v; else b[j - 4] = v;
        }
        float4v* dst = (float4v*)(out + n * in_features + k0);
        dst[0] = a;
        dst[1] = b;
    }
}

int grid_for(int64_t items) {
    int64_t blocks = (items + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    return (int)blocks;
}

}  // namespace

hipError_t launch_unpack(const uint8_t* packed, int8_t* out, int64_t elements, hipStream_t stream) {
    if (elements == 0) return hipSuccess;
    int64_t items = elements / 8;
    if (items < elements % 8) items = elements % 8;
    hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(items)), dim3(256), 0, stream, packed, out, elements);
    return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros, float* out,
                          int64_t out_features, int64_t in_features, hipStream_t stream) {
    int64_t items = out_features * (in_features / 8);
    if (items == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(items)), dim3(256), 0, stream, qweight, scales, zeros, out,
                       out_features, in_features);
    return hipGetLastError();
}

}  // namespace w4g64
