/*
 * w4g64.h -- C ABI of the MI355X (gfx950) W4G64 INT4 linear backend.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as `void*`, NULL = the default stream) and returns an int status.
 * Nothing here allocates device memory, synchronizes the stream or keeps
 * hidden global state besides the per-thread error string.  Arguments are
 * validated on the host before any launch; on a non-zero status nothing was
 * launched (except W4G64_STATUS_HIP_ERROR, which reports a failed launch).
 *
 * Packed contract (the reference checkpoint layout, unchanged):
 *   qweight  uint8 [out*in/2]  row-major [out, in/2]; byte n*(in/2)+k/2 holds
 *            k even in the low nibble, k odd in the high nibble; signed
 *            two's-complement INT4 codes.
 *   scales   fp16  [out, in/64]
 *   zeros    uint8 [(out*(in/64)+1)/2]  signed INT4 zero points, element
 *            n*(in/64)+g, same nibble order.
 *   dequant  W[n,k] = (code[n,k] - zero[n,k/64]) * scale[n,k/64]
 * Reference: src/qwen_int4/quantization.py:17-84, :221-258 and
 * src/qwen_int4/backends.py:73-98.
 */
#ifndef QWEN_INT4_HIP_W4G64_H
#define QWEN_INT4_HIP_W4G64_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The Python layer maps them onto the reference's exception
 * types: INVALID_VALUE -> ValueError, INVALID_DTYPE -> TypeError,
 * UNSUPPORTED/HIP_ERROR -> RuntimeError. */
#define W4G64_STATUS_OK 0
#define W4G64_STATUS_INVALID_VALUE 1
#define W4G64_STATUS_INVALID_DTYPE 2
#define W4G64_STATUS_WORKSPACE 3
#define W4G64_STATUS_UNSUPPORTED 4
#define W4G64_STATUS_HIP_ERROR 5

/* Element type codes for activations, outputs and bias. */
#define W4G64_DTYPE_NONE 0
#define W4G64_DTYPE_F16 1
#define W4G64_DTYPE_BF16 2
#define W4G64_DTYPE_F32 3

/* Activation form of w4g64_linear_swiglu below, accepted (besides the dtypes
 * above) by w4g64_linear_workspace_bytes and w4g64_linear_kernel_name: the
 * SwiGLU product of a [gate | up] bf16 row (fp32). */
#define W4G64_DTYPE_BF16_SWIGLU 5

/* Decode-step forms (1..16 rows):
 *   W4G64_DTYPE_BF16_PLANES: activation form of w4g64_linear -- x is bf16
 *     [3, rows, in_features], three planes whose fp32 sum (hi + mid + lo) is
 *     the activation, as w4g64_linear_gate_up_planes writes them; y is fp32.
 *   W4G64_DTYPE_BF16_GATE_UP: query code (w4g64_linear_workspace_bytes,
 *     w4g64_linear_kernel_name) for w4g64_linear_gate_up_planes. */
#define W4G64_DTYPE_BF16_PLANES 6
#define W4G64_DTYPE_BF16_GATE_UP 7

/* Residual delta given as `parts` fp32 partial sums [parts][rows][hidden] of a
 * split-K projection (w4g64_linear_partials), accepted as delta_dtype by
 * qwen2_add_rmsnorm (1..255 parts) and w4g64_linear_rmsnorm (1..8 parts): the
 * delta is their sum in order from part 0, exactly the fp32 value the split-K
 * reduction of w4g64_linear stores. */
#define W4G64_DTYPE_F32_PARTIALS(parts) (0x100 | (parts))
#define W4G64_DTYPE_F32_PARTS_OF(code) ((((code) & ~0xFF) == 0x100) ? ((code) & 0xFF) : 0)

/* Version of this ABI (bumped on any signature or contract change). */
int w4g64_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* w4g64_last_error(void);

/* Decode `elements` signed INT4 values (canonical nibble order) from
 * `packed_bytes` bytes into int8.  `elements` may be odd (truncates the last
 * byte) and must be in [0, 2*packed_bytes].
 * Replaces: unpack_canonical_signed_int4_triton
 *           (src/qwen_int4/triton_kernels.py:119-146). */
int w4g64_unpack_canonical_int4(const uint8_t* packed, int64_t packed_bytes, int8_t* out,
                                int64_t elements, void* stream);

/* Dequantize a canonical W4G64 weight to fp32 [out_features, in_features],
 * bit-exact with the closed form above.
 * Replaces: dequantize_canonical_w4g64_triton
 *           (src/qwen_int4/triton_kernels.py:149-203). */
int w4g64_dequantize_canonical(const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros,
                               float* out, int64_t out_features, int64_t in_features, void* stream);

/* Bytes of workspace w4g64_linear needs for this problem (0 = none).
 * It holds fp32 split-K partial sums (decode shapes that split K across
 * workgroups; prefill shapes whose tiles do not fill whole rounds of the
 * device's workgroup slots, up to 64 MiB) -- and, for fp32 activations of the
 * prefill GEMM, their two bf16 planes.  Every call writes what it reads, so a
 * workspace needs no initial contents: a caller allocates one (sized for its
 * largest problem) and reuses it for every shape.  Calls sharing a workspace
 * must be ordered on one stream.  The prefill plan depends on the current
 * device's CU count. */
int64_t w4g64_linear_workspace_bytes(int64_t rows, int64_t out_features, int64_t in_features,
                                     int x_dtype);

/* y[rows, out] = x[rows, in] @ dequant(W)^T (+ bias), fp32 accumulation,
 * stored in x's dtype.  x: fp16/bf16/fp32 contiguous row-major; bias: NONE,
 * fp16, bf16 or fp32 [out]; y: same dtype as x.  rows >= 1; in % 64 == 0.
 * With x_dtype W4G64_DTYPE_BF16_PLANES (1..16 rows) x holds the three bf16
 * planes of an fp32 activation and y is fp32.
 * rows <= 16 runs the decode GEMV, larger rows the MFMA GEMM.
 * Pointers must be 16-byte aligned (scales and bias: element aligned).
 * Replaces: linear_canonical_w4g64_triton (src/qwen_int4/triton_kernels.py:206-268)
 *           and the kernel it launches (:66-116). */
int w4g64_linear(const void* x, int x_dtype, const uint8_t* qweight, const uint16_t* scales,
                 const uint8_t* zeros, const void* bias, int bias_dtype, void* y, int64_t rows,
                 int64_t out_features, int64_t in_features, void* workspace, int64_t workspace_bytes,
                 void* stream);

/* w4g64_linear that also records two hipEvent_t (passed as void*, either may
 * be NULL) at the start and at the end of the kernel itself, so
 * hipEventElapsedTime gives the kernel's own duration -- the figure a
 * profiler reports -- even when the host enqueues slower than the GPU runs.
 * For benchmarking; not usable inside stream capture.
 * No counterpart in the reference (its harness times with CUDA events around
 * the call, scripts/autotune_phase_e_triton_v6.py:44-56). */
int w4g64_linear_timed(const void* x, int x_dtype, const uint8_t* qweight, const uint16_t* scales,
                       const uint8_t* zeros, const void* bias, int bias_dtype, void* y, int64_t rows,
                       int64_t out_features, int64_t in_features, void* workspace, int64_t workspace_bytes,
                       void* stream, void* start_event, void* stop_event);

/* w4g64_linear without a workspace argument and without any allocation:
 * its split-K partial sums live in a file-scope device
 * array of the library (w4g64_static_scratch_bytes() bytes, 4 MiB, one per
 * GPU, held until the process ends), whose address is looked up once per
 * device (hipGetSymbolAddress) on the first call there: make that first call
 * on each device outside stream capture; the calls after it run nothing but
 * the kernels and may be captured.  Problems that need more scratch than that
 * (the split-K prefill GEMM; every decode call of 1..16 rows of the
 * Qwen2-1.5B shapes fits) are rejected with W4G64_STATUS_UNSUPPORTED.  Calls
 * on one GPU share the array: calls that overlap on one GPU (on different
 * streams) race; calls in one stream order are safe, since every call
 * writes the partials it reads.  Same arguments, checks and results as
 * w4g64_linear otherwise.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops that forbid hipMalloc). */
int w4g64_linear_static_scratch(const void* x, int x_dtype, const uint8_t* qweight, const uint16_t* scales,
                                 const uint8_t* zeros, const void* bias, int bias_dtype, void* y, int64_t rows,
                                 int64_t out_features, int64_t in_features, void* stream);
/* Size in bytes of w4g64_linear_static_scratch's per-GPU array. */
int64_t w4g64_static_scratch_bytes(void);

/* Measurement probe; no counterpart in the reference.  One 16-byte
 * nontemporal load per lane over exactly `bytes` of src (16-byte aligned, a
 * multiple of 4096), which practically never stores: the bare-stream floor a
 * decode GEMV launch over the same bytes is measured against (bench.py).
 * sink holds 256 uint32. */
int w4g64_stream_probe(const void* src, int64_t bytes, void* sink, void* stream);

/* Fusion of the SwiGLU product into the down projection: gate_up is
 * [rows, 2 * in_features] bf16 (gate | up), the activation is
 * h = silu(gate) * up in fp32 (silu(g) = g / (1 + exp(-g))), and
 * y[rows, out] = h @ dequant(W)^T (+ bias) in fp32, as w4g64_linear on the
 * fp32 h (decode rows 1..16: formed in the GEMV's activation staging; more
 * rows: written as the GEMM's bf16 planes).  gate_up and qweight 16-byte
 * aligned.
 * Replaces: QwenMLP.forward's product and down projection
 *           (src/qwen_int4/model.py:133-136). */
int w4g64_linear_swiglu(const void* gate_up, const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros,
                        const void* bias, int bias_dtype, float* y, int64_t rows, int64_t out_features,
                        int64_t in_features, void* workspace, int64_t workspace_bytes, void* stream);

/* Fused gate|up projection of a decode step (1..16 rows) with the SwiGLU
 * product in its epilogue.  The weight is the two projections' rows stacked,
 * out_features = 2 I (gate rows 0..I-1, then up rows I..2I-1); x is bf16
 * [rows, in_features].  For every row m and i < I:
 *   gate = bf16(x . W[i] + bias[i]),  up = bf16(x . W[I + i] + bias[I + i])
 *   h    = silu(gate) * up in fp32, silu(v) = v / (1 + exp(-v))
 * stored as its exact three-way bf16 split into planes bf16 [3, rows, I]
 * (planes[0] + planes[1] + planes[2] == h; planes[0] is h truncated to bf16,
 * planes[1] the remainder truncated, planes[2] the rest), the activation form
 * W4G64_DTYPE_BF16_PLANES of the down projection.  Workspace: query with
 * W4G64_DTYPE_BF16_GATE_UP.  x and qweight 16-byte aligned.
 * Replaces: the gate/up projections and the SwiGLU product of
 *           QwenMLP.forward (src/qwen_int4/model.py:133-135). */
int w4g64_linear_gate_up_planes(const void* x, const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros,
                                const void* bias, int bias_dtype, void* planes, int64_t rows, int64_t out_features,
                                int64_t in_features, void* workspace, int64_t workspace_bytes, void* stream);

/* Decode linear (one row, bf16: batch-1 decode) with the decoder's residual add and
 * RMSNorm formed in its activation staging:
 *   s      = bf16(residual + bf16(delta))          (delta bf16, fp32, or 1..8 fp32
 *                                                   partial sums: W4G64_DTYPE_F32_PARTIALS)
 *   x      = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * norm_weight)
 *   y      = x @ dequant(W)^T (+ bias), bf16 [rows, out_features]
 *            -- or, with gate_up_planes != 0, the planes of
 *            w4g64_linear_gate_up_planes (W the stacked [gate; up] rows)
 *   out_sum = s (bf16 [rows, in_features]; must not overlap residual).
 * Squares are rounded before their fp32 sum (as x.pow(2)); the same
 * arithmetic as qwen2_add_rmsnorm followed by w4g64_linear (or the gate|up
 * planes entry).  The whole row is staged by every workgroup, so the plan
 * must not split K (W4G64_STATUS_UNSUPPORTED otherwise); no workspace.
 * Pointers 16-byte aligned.
 * Replaces: RMSNorm.forward (src/qwen_int4/model.py:40-44), the residual adds
 *           of DecoderLayer.forward (:149-154) and the linear that follows
 *           each norm (q/k/v, model.py:70-72; gate/up, :133-135). */
int w4g64_linear_rmsnorm(const void* residual, const void* delta, int delta_dtype, const void* norm_weight, float eps,
                         void* out_sum, const uint8_t* qweight, const uint16_t* scales, const uint8_t* zeros,
                         const void* bias, int bias_dtype, void* y, int gate_up_planes, int64_t rows,
                         int64_t out_features, int64_t in_features, void* workspace, int64_t workspace_bytes,
                         void* stream);

/* Decode linear (one row, bf16: batch-1 decode) whose activation is the
 * decode attention's output, merged in its staging from the per-chunk partial
 * results that qwen2_decode_attention_partials leaves in its workspace:
 *   x[h * 128 + d] = bf16( sum_c exp(m_c - m) acc_c[d] / sum_c exp(m_c - m) l_c ),
 *       m = max_c m_c, over the chunks c of query head h's key/value head
 *   y = x @ dequant(W)^T (+ bias), bf16 [rows, out_features]
 * -- bit for bit qwen2_decode_attention's output followed by w4g64_linear.
 * attention_workspace / attention_workspace_bytes, max_length, num_heads and
 * num_kv_heads are those of the qwen2_decode_attention_partials call (batch
 * = rows = 1); in_features = num_heads * 128.  Takes max_length <= 1024
 * (every chunk's partial is loaded), num_heads <= 12 and in_features a
 * multiple of 256; W4G64_STATUS_UNSUPPORTED otherwise (then use
 * qwen2_decode_attention and w4g64_linear).  qweight 16-byte aligned.
 * Replaces: the softmax-weighted sum of QwenAttention.forward and the o_proj
 *           linear that follows it (src/qwen_int4/model.py:101-122). */
int w4g64_linear_attention_merge(const void* attention_workspace, int64_t attention_workspace_bytes,
                                 int64_t max_length, int64_t num_heads, int64_t num_kv_heads, const uint8_t* qweight,
                                 const uint16_t* scales, const uint8_t* zeros, const void* bias, int bias_dtype,
                                 void* y, int64_t rows, int64_t out_features, void* stream);

/* Number of fp32 partial sums per output w4g64_linear_partials writes for this
 * problem (its K splits; 1 = unsplit), or 0 when the problem does not take
 * that form: x_dtype W4G64_DTYPE_BF16_PLANES or W4G64_DTYPE_F32, 1..16 rows. */
int64_t w4g64_linear_partial_count(int64_t rows, int64_t out_features, int64_t in_features, int x_dtype);

/* The decode linear of w4g64_linear (x_dtype W4G64_DTYPE_BF16_PLANES or
 * W4G64_DTYPE_F32, 1..16 rows, no bias) without its split-K reduction
 * launch: writes the fp32 partial sums partials[s][rows][out_features],
 * s < count = w4g64_linear_partial_count(...), whose sum in order from s = 0
 * is w4g64_linear's output (count 1: that output).  The next residual add
 * takes them as delta_dtype W4G64_DTYPE_F32_PARTIALS(count).  partials 16-byte
 * aligned, partials_bytes >= count * rows * out_features * 4; no workspace.
 * Replaces: the down projection of QwenMLP.forward and the residual add that
 *           consumes it (src/qwen_int4/model.py:136, :149-154), split so that
 *           the add performs the reduction. */
int w4g64_linear_partials(const void* x, int x_dtype, const uint8_t* qweight, const uint16_t* scales,
                          const uint8_t* zeros, float* partials, int64_t partials_bytes, int64_t rows,
                          int64_t out_features, int64_t in_features, void* stream);

/* Name of the kernel w4g64_linear launches for this problem (for profiles
 * and reports); never NULL. */
const char* w4g64_linear_kernel_name(int64_t rows, int64_t out_features, int64_t in_features,
                                     int x_dtype);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_INT4_HIP_W4G64_H */
