"""GPU parity of the HIP W4G64 kernels against the CPU oracle.

Mirrors the reference's GPU gate (tests/test_triton_unpack.py) and extends it
to every benchmark configuration: unpack and dequant must be bit-exact; the
linear must be within the reference's tolerances (fp16 rtol 0.01 / atol
0.0625, bf16 rtol 0.02 / atol 0.25; docs/phase-e-triton.md:48-51) and within
a normwise relative error ||y - r||_inf / ||r||_inf <= 1e-2 of the fp32
oracle.  One-hot activations make the linear output equal to rounded
dequantized weights, which is checked bit for bit.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

from qwen_int4_hip import (  # noqa: E402  (after the skip marker on purpose)
    PackingFormat,
    QuantLinear,
    dequantize_canonical_w4g64_hip,
    hip_w4g64_linear,
    linear_canonical_w4g64_hip,
    unpack_canonical_signed_int4_hip,
)

DEV = "cuda"
TOL = {"fp16": (0.01, 0.0625), "bf16": (0.02, 0.25), "fp32": (1e-4, 1e-4)}
SHAPES = O.QWEN2_SHAPES


def to_dev(arr: np.ndarray, dtype: str) -> torch.Tensor:
    arr = np.ascontiguousarray(arr)
    if dtype == "bf16":
        return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16).to(DEV)
    return torch.from_numpy(arr).to(DEV)


def from_dev(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


@functools.lru_cache(maxsize=None)
def weights(kind: str, n: int, k: int, seed: int):
    if kind == "sym":
        return O.symmetric_weights(n, k, seed)
    if kind == "asym":
        return O.asymmetric_weights(n, k, seed)
    return O.awq_folded_weights(n, k, seed)


def dev_weights(q, s, z):
    return to_dev(q, "u8"), to_dev(s, "fp16"), to_dev(z, "u8")


def check_linear(x_np, q, s, z, bias_np, n, k, dtype, bias_dtype="bf16", normwise=1e-2, tol=None):
    xt = to_dev(x_np, dtype)
    bt = None if bias_np is None else to_dev(bias_np, bias_dtype)
    got = hip_w4g64_linear(xt, *dev_weights(q, s, z), bt, out_features=n, in_features=k, group_size=64,
                           packing=PackingFormat.CANONICAL)
    assert got.dtype == xt.dtype and got.shape == (*x_np.shape[:-1], n)
    ref = O._to_f32(O.reference_linear(x_np, q, s, z, bias_np, out_features=n, in_features=k, x_dtype=dtype,
                                       bias_dtype=bias_dtype), dtype)
    out = from_dev(got)
    assert np.isfinite(out).all()
    rel = float(np.abs(out - ref).max() / max(float(np.abs(ref).max()), 1e-30))
    assert rel <= normwise, f"normwise relative error {rel:.3e} > {normwise}"
    rtol, atol = tol or TOL[dtype]
    np.testing.assert_allclose(out, ref, rtol=rtol, atol=atol)
    return out, ref


# --------------------------------------------------------------------------
# unpack / dequant primitives (bit-exact)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("codes", [[-8, -7, -1, 0, 1, 6, 7, -8], [7, -8, 0, -1, 3, -4, -5, 6]])
def test_unpack_matches_canonical_boundary_patterns(codes):
    codes = np.array(codes, dtype=np.int8)
    got = unpack_canonical_signed_int4_hip(to_dev(O.pack_int4(codes), "u8"))
    np.testing.assert_array_equal(got.cpu().numpy(), codes)


@pytest.mark.parametrize("count", [1025, 1026, 7, 8, 9, 0, 1])
def test_unpack_random_bytes_and_odd_element_count(count):
    torch.manual_seed(20260831)
    packed = torch.randint(0, 256, (513,), dtype=torch.uint8)
    expected = O.unpack_int4(packed.numpy(), elements=count)
    got = unpack_canonical_signed_int4_hip(packed.to(DEV), elements=count)
    np.testing.assert_array_equal(got.cpu().numpy(), expected)


def test_unpack_large_exhaustive_bytes():
    packed = np.tile(np.arange(256, dtype=np.uint8), 4099)  # 1,049,344 bytes, every byte value
    got = unpack_canonical_signed_int4_hip(to_dev(packed, "u8"))
    np.testing.assert_array_equal(got.cpu().numpy(), O.unpack_int4(packed))


def test_unpack_rejects_invalid_tensor_contracts():
    packed = torch.zeros(4, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="dtype"):
        unpack_canonical_signed_int4_hip(packed.to(torch.int8))
    with pytest.raises(ValueError, match="elements"):
        unpack_canonical_signed_int4_hip(packed, elements=9)
    with pytest.raises(ValueError, match="contiguous"):
        unpack_canonical_signed_int4_hip(packed.repeat(2)[::2])


@pytest.mark.parametrize("shape", [(3, 64), (5, 128), (256, 1536)])
def test_dequant_bit_exact_random_asymmetric(shape):
    rng = np.random.default_rng(shape[0] * 10000 + shape[1])
    w = rng.standard_normal(shape, dtype=np.float32) * np.float32(0.1)
    q, s, z = O.quantize_asymmetric_rtn(w, group_size=64)
    expected = O.dequantize_groupwise(q, s, zeros=z, out_features=shape[0], in_features=shape[1], group_size=64,
                                      packing=PackingFormat.CANONICAL)
    got = dequantize_canonical_w4g64_hip(*dev_weights(q, s, z), out_features=shape[0], in_features=shape[1])
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("kind", ["sym", "asym"])
def test_dequant_bit_exact_qwen2_shapes(name, kind):
    n, k = SHAPES[name]
    q, s, z = weights(kind, n, k, O.BASE_SEED + n + k)
    expected = O.dequantize_groupwise(q, s, zeros=z, out_features=n, in_features=k, group_size=64,
                                      packing=PackingFormat.CANONICAL)
    got = dequantize_canonical_w4g64_hip(*dev_weights(q, s, z), out_features=n, in_features=k)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), expected.view(np.uint32))


def test_dequant_rejects_layout_and_dtype_drift():
    qweight = torch.zeros(64, dtype=torch.uint8, device=DEV)
    scales = torch.ones(2, dtype=torch.float16, device=DEV)
    zeros = torch.zeros(1, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="divisible"):
        dequantize_canonical_w4g64_hip(qweight, scales, zeros, out_features=1, in_features=96)
    with pytest.raises(ValueError, match="scales.*dtype"):
        dequantize_canonical_w4g64_hip(qweight, scales.float(), zeros, out_features=1, in_features=128)
    with pytest.raises(ValueError, match="qweight must contain"):
        dequantize_canonical_w4g64_hip(qweight[:-1], scales, zeros, out_features=1, in_features=128)


# --------------------------------------------------------------------------
# linear: reference operator matrix and benchmark configurations
# --------------------------------------------------------------------------

@pytest.mark.parametrize(
    ("rows", "n", "k", "dtype"),
    [(1, 256, 1536, "fp16"), (8, 1536, 1536, "bf16"), (4, 1536, 8960, "fp16")],
    ids=["v-proj-fp16", "q-proj-bf16", "mlp-down-fp16"],
)
def test_linear_matches_reference_operator_matrix(rows, n, k, dtype):
    # docs/phase-e-triton.md:31-37 matrix, asymmetric weights, with bias
    q, s, z = weights("awq", n, k, rows + n + k)
    x = O.activations(rows, k, seed=rows + n + k, dtype=dtype)
    bias = O._from_f32(np.random.default_rng(n).standard_normal(n).astype(np.float32) * np.float32(0.01), dtype)
    check_linear(x, q, s, z, bias, n, k, dtype, bias_dtype=dtype)


@pytest.mark.parametrize("rows", [1, 4, 16])
@pytest.mark.parametrize("name", list(SHAPES))
def test_decode_all_qwen2_shapes_fp16(name, rows):
    # decode configuration: symmetric RTN, fp16 x ~ N(0,1); q/k/v carry a bf16 bias as in the model
    n, k = SHAPES[name]
    q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
    x = O.activations(rows, k, seed=O.BASE_SEED + 7 * rows + n, dtype="fp16")
    bias = (O.f32_to_bf16_bits(np.random.default_rng(n).standard_normal(n).astype(np.float32) * np.float32(0.1))
            if name in ("q_proj", "k_proj", "v_proj") else None)
    out, ref = check_linear(x, q, s, z, bias, n, k, "fp16")
    # exact-integer decode: within one fp16 ulp of the fp32 oracle almost everywhere
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
    assert np.mean(np.abs(out - ref) <= ulp) > 0.99


LEAN_SHAPES = [(2048, 1536, "sym"), (17920, 1536, "asym"), (1536, 8960, "awq"), (200, 256, "asym"),
                  (256, 1536, "sym"), (256, 640, "asym")]


def decode_kernel_prefix(rows: int, k: int) -> str:
    """The decode kernel the planner takes for fp16/bf16 activations with
    16-byte aligned operands: the pipelined GEMV when in_features is a
    multiple of 256, else the lean kernel for one row and the segmented /
    9..16-row kernels for more."""
    if k % 256 == 0:
        return "gemv_pipe_kernel"
    if rows == 1:
        return "gemv_seg_kernel"
    return "gemv16_kernel" if rows > 8 else "gemv_kernel"


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("n,k,kind", LEAN_SHAPES)
def test_lean_decode_kernel(n, k, kind, rows, dtype):
    """Decode shapes through the GEMV kernels: the fused q|k|v and gate|up
    widths, the long-K down projection, a partial last row block (200
    features) and a 256-wide projection take the pipelined kernel at 1..8
    rows; K = 640 (an odd pair count) takes the lean kernel at one row and
    the segmented kernel at more.  Bias, asymmetric and AWQ-folded codes."""
    from qwen_int4_hip import linear_kernel_name

    torch_dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
    assert linear_kernel_name(rows, n, k, torch_dtype).startswith(decode_kernel_prefix(rows, k))
    q, s, z = weights(kind, n, k, O.BASE_SEED + n + k + rows)
    x = O.activations(rows, k, seed=O.BASE_SEED + 13 * rows + n, dtype=dtype, outliers=kind != "sym")
    bias = O.f32_to_bf16_bits(np.random.default_rng(n + rows).standard_normal(n).astype(np.float32) * np.float32(0.1))
    out, ref = check_linear(x, q, s, z, bias, n, k, dtype)
    if dtype == "fp16":  # exact (code - zero) in fp16: within one fp16 ulp almost everywhere
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
        assert np.mean(np.abs(out - ref) <= ulp) > 0.99


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("rows,n,k", [(1, 32768, 1536), (3, 32768, 1536), (1, 33032, 6144)])
def test_pipe_kernel_two_row_blocks_per_wave(rows, n, k, dtype):
    """32768+ output features at 1..4 rows (and at one row over a long K, with
    a last row block that is only partly filled): each wave of the pipelined
    kernel owns two row blocks, so the codes of one block are formed right
    before their MFMAs -- the schedule in which an operand written without
    the MFMA's wait states once corrupted every second block of bf16 rows."""
    from qwen_int4_hip import linear_kernel_name

    torch_dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
    name = linear_kernel_name(rows, n, k, torch_dtype)
    assert name.startswith("gemv_pipe_kernel") and name.split(",")[5] == "2", name  # RBW = 2
    q, s, z = weights("asym", n, k, O.BASE_SEED + 7 * rows)
    x = O.activations(rows, k, seed=O.BASE_SEED + 17 * rows, dtype=dtype, outliers=True)
    check_linear(x, q, s, z, None, n, k, dtype)


@pytest.mark.parametrize("name", ["gate_proj", "q_proj"])
def test_lean_and_segmented_kernels_agree(name):
    """The same problem through the pipelined kernel and, with a scales view
    that is only 2-byte aligned (which neither the pipelined nor the lean
    kernel takes), through the segmented kernel: both round fp32 values that
    differ only by summation order, so they agree within two fp16 ulps."""
    from qwen_int4_hip import linear_kernel_name

    n, k = SHAPES[name]
    assert linear_kernel_name(1, n, k, torch.float16).startswith("gemv_pipe_kernel")
    q, s, z = weights("asym", n, k, O.BASE_SEED + 5)
    xt = to_dev(O.activations(1, k, seed=O.BASE_SEED + 6, dtype="fp16"), "fp16")
    qd, sd, zd = dev_weights(q, s, z)
    fast = linear_canonical_w4g64_hip(xt, qd, sd, zd)
    shifted = torch.empty(sd.numel() + 1, dtype=torch.float16, device=DEV)
    shifted[1:].copy_(sd.reshape(-1))
    slow = linear_canonical_w4g64_hip(xt, qd, shifted[1:].view(sd.shape), zd)
    diff = (fast.float() - slow.float()).abs().cpu()
    big = torch.maximum(fast.float().abs(), slow.float().abs()).cpu().numpy().astype(np.float16)
    ulp = torch.from_numpy(np.spacing(big).astype(np.float32))
    assert bool((diff <= 2 * ulp).all()), float((diff / ulp).max())


def output_ulp(v: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "fp16":
        return np.spacing(np.abs(v).astype(np.float16)).astype(np.float32)
    return np.ldexp(np.float32(1), np.frexp(np.abs(v).astype(np.float32))[1] - 8).astype(np.float32)  # bf16


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("rows,name,kind", [(2048, "gate_proj", "sym"), (512, "down_proj", "asym"),
                                            (128, "q_proj", "awq"), (40, "k_proj", "sym")])
def test_gemm_multiplies_exact_weights(rows, name, kind, dtype):
    """The prefill GEMM's products are those of the exact fp32 weights
    (code - zero) * scale, as in the reference's dequantize-then-matmul
    (backends.py:86-98): against the fp32 oracle rounded to the output type,
    at least 99% of the outputs are identical and every one is within an
    ulp (plus 1e-6 of the largest output, for outputs near zero, where the
    fp32 summation orders differ by more than their ulp).  Weights rounded to
    the activation type before the multiply miss this by a wide margin."""
    from qwen_int4_hip import linear_kernel_name

    n, k = SHAPES[name]
    torch_dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
    assert linear_kernel_name(rows, n, k, torch_dtype).startswith("gemm_kernel")
    q, s, z = weights(kind, n, k, O.BASE_SEED + 17 * rows + n)
    x = O.activations(rows, k, seed=O.BASE_SEED + 19 * rows + k, dtype=dtype, outliers=kind != "sym")
    out, ref = check_linear(x, q, s, z, None, n, k, dtype)
    diff = np.abs(out - ref)
    bound = output_ulp(np.maximum(np.abs(out), np.abs(ref)), dtype) + 1e-6 * float(np.abs(ref).max())
    assert bool((diff <= bound).all()), float((diff / bound).max())
    assert float(np.mean(diff == 0)) >= 0.99, float(np.mean(diff == 0))


@pytest.mark.parametrize("rows", [128, 512, 2048])
@pytest.mark.parametrize("name", ["gate_proj", "down_proj"])
def test_prefill_mlp_shapes_bf16(name, rows):
    n, k = SHAPES[name]
    q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
    x = O.activations(rows, k, seed=O.BASE_SEED + rows + n, dtype="bf16")
    check_linear(x, q, s, z, None, n, k, "bf16")


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
def test_gemm_eight_wave_workgroups(dtype):
    """gate_proj 8960x1536 at 512 rows: 140 unsplit tiles, at most one
    workgroup per CU, so each workgroup runs 8 waves of 32 output features
    (two per SIMD on one tile); fp32 rows take the two-plane staging and the
    fp32-output epilogue."""
    from qwen_int4_hip import linear_kernel_name

    n, k = SHAPES["gate_proj"]
    torch_dtype = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}[dtype]
    assert "8 waves" in linear_kernel_name(512, n, k, torch_dtype)
    q, s, z = weights("asym", n, k, O.BASE_SEED + 41)
    x = O.activations(512, k, seed=O.BASE_SEED + 43, dtype=dtype)
    if dtype == "fp32":
        bias = np.linspace(-1, 1, n, dtype=np.float32)
        check_linear(x, q, s, z, bias, n, k, "fp32", bias_dtype="fp32", normwise=1e-5, tol=(1e-4, 1e-4))
    else:
        bias = O.f32_to_bf16_bits(np.linspace(-1, 1, n, dtype=np.float32))
        check_linear(x, q, s, z, bias, n, k, dtype)


@pytest.mark.parametrize("rows", [1, 2048])
@pytest.mark.parametrize("name", list(SHAPES))
def test_asymmetric_awq_shapes_fp16_with_outliers(name, rows):
    n, k = SHAPES[name]
    q, s, z = weights("asym", n, k, O.BASE_SEED + 3 * n + k)
    x = O.activations(rows, k, seed=O.BASE_SEED + 11 * rows + n, dtype="fp16", outliers=True)
    check_linear(x, q, s, z, None, n, k, "fp16")


@pytest.mark.parametrize("rows", [1, 16, 256])
def test_awq_folded_weights_bf16(rows):
    n, k = SHAPES["up_proj"]
    q, s, z = weights("awq", n, k, O.BASE_SEED + 99)
    x = O.activations(rows, k, seed=O.BASE_SEED + rows, dtype="bf16", outliers=True)
    check_linear(x, q, s, z, None, n, k, "bf16")


@pytest.mark.parametrize("rows", [1, 3, 5, 6, 16, 17, 64, 200, 512])
def test_fp32_activations_run_natively(rows):
    # the reference routes fp32 to its torch oracle (backends.py:172-177); here it runs on the kernels
    n, k = SHAPES["down_proj"]
    q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
    x = O.activations(rows, k, seed=O.BASE_SEED + 5 * rows, dtype="fp32")
    bias = np.linspace(-1, 1, n, dtype=np.float32)
    # decode splits fp32 exactly into three bf16 parts; the GEMM into two
    # (|x - hi - lo| <= 2^-17 |x|) against exact weights: near-fp32 accuracy
    check_linear(x, q, s, z, bias, n, k, "fp32", bias_dtype="fp32", normwise=1e-5, tol=(1e-4, 1e-4))


@pytest.mark.parametrize("n,k,rows", [(200, 192, 40), (1000, 64, 300), (4, 128, 33)])
def test_fp32_gemm_ragged_shapes(n, k, rows):
    # output widths that are not a multiple of 4 (scalar fp32 stores), K = 64,
    # and a single column tile
    q, s, z = weights("awq", n, k, O.BASE_SEED + 3 * n + k)
    x = O.activations(rows, k, seed=O.BASE_SEED + rows + n, dtype="fp32")
    check_linear(x, q, s, z, None, n, k, "fp32", normwise=1e-5, tol=(1e-4, 1e-4))


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_lean_kernel_with_an_empty_k_part_ignores_lds_leftovers(dtype):
    """K = 384 (3 group pairs) over the lean kernel's 4 K parts leaves the
    last part empty; its steps must read only in-range staged data.  A GEMM
    over NaN activations first fills the LDS of every CU with NaN, which an
    out-of-range read of the group sums would turn into NaN outputs (0 * NaN)."""
    from qwen_int4_hip import linear_kernel_name

    torch_dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
    poison = torch.full((2048, 1536), float("nan"), dtype=torch_dtype, device=DEV)
    q8, s8, z8 = weights("sym", 8960, 1536, O.BASE_SEED + 5)
    for n in (384, 128):
        kind = "f16" if dtype == "fp16" else "bf16"
        assert linear_kernel_name(1, n, 384, torch_dtype).startswith(f"gemv_seg_kernel<{kind},4,1,4,")
        q, s, z = weights("asym", n, 384, O.BASE_SEED + n)
        x = O.activations(1, 384, seed=O.BASE_SEED + 3 * n, dtype=dtype)
        bias = O._from_f32(np.linspace(-1, 1, n, dtype=np.float32), "bf16")
        for _ in range(3):
            hip_w4g64_linear(poison, *dev_weights(q8, s8, z8), None, out_features=8960, in_features=1536,
                             group_size=64, packing=PackingFormat.CANONICAL)
            check_linear(x, q, s, z, bias, n, 384, dtype)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("rows", [1, 2, 3, 4, 6, 12])
@pytest.mark.parametrize("n,k", [(264, 4096), (1000, 3328), (40, 256), (264, 13824), (100, 6144)])
def test_pipe_kernel_k_splits_and_pairs_past_the_range(n, k, rows, dtype):
    """The pipelined GEMV with K split across workgroups whose last split is
    mostly pairs past the range (K = 4096: spans of 12 pairs over 32 pairs;
    K = 3328: 26 pairs, the last split 2 real pairs; at 2..4 rows the long-K
    spans of 72 and 80 pairs: K = 13824 in two splits, K = 6144 in one span
    a third past the range), a partial last row
    block (n = 264, 1000, 40), and LDS left full of NaN by a GEMM over NaN
    activations: steps past the range must add exactly nothing (their scales,
    activations and, bf16, group sums are never taken from stale LDS)."""
    from qwen_int4_hip import linear_kernel_name

    torch_dtype = torch.float16 if dtype == "fp16" else torch.bfloat16
    assert linear_kernel_name(rows, n, k, torch_dtype).startswith("gemv_pipe_kernel")
    poison = torch.full((2048, 1536), float("nan"), dtype=torch_dtype, device=DEV)
    q8, s8, z8 = weights("sym", 8960, 1536, O.BASE_SEED + 5)
    q, s, z = weights("asym", n, k, O.BASE_SEED + n + k + rows)
    x = O.activations(rows, k, seed=O.BASE_SEED + 5 * rows + n, dtype=dtype, outliers=True)
    bias = O._from_f32(np.linspace(-1, 1, n, dtype=np.float32), "fp16")
    for _ in range(2):
        hip_w4g64_linear(poison, *dev_weights(q8, s8, z8), None, out_features=8960, in_features=1536,
                         group_size=64, packing=PackingFormat.CANONICAL)
        check_linear(x, q, s, z, bias, n, k, dtype, bias_dtype="fp16")


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
@pytest.mark.parametrize("k", [1536, 16448])
def test_gemm_row_scaling_keeps_every_row_exact(dtype, k):
    """The GEMM stages each activation row as fp16 times a power of two
    chosen from the row's largest magnitude.  Rows whose magnitudes lie far
    outside fp16's range (1e-30, 1e30 -- representable in bf16 and fp32), a
    zero row and rows with one large outlier must each match the oracle to
    the same per-row relative error as ordinary rows.  k = 16448 stages rows
    longer than a staging thread holds (a second read of the row)."""
    n, rows = 72, 24
    q, s, z = weights("asym", n, k, O.BASE_SEED + k)
    base = np.random.default_rng(k).standard_normal((rows, k)).astype(np.float32)
    factors = np.array([1e-30, 1e30, 0.0, 1.0, 3e-8, 6e4, 1e-3, 1e5] * 3, dtype=np.float32)
    x32 = base * factors[:, None]
    x32[3, 17] = np.float32(5e4)  # one outlier: the rest of its row sits 2^15..2^20 below it
    x = O._from_f32(x32, dtype)
    xt = to_dev(x, dtype)
    got = from_dev(hip_w4g64_linear(xt, *dev_weights(q, s, z), None, out_features=n, in_features=k, group_size=64,
                                    packing=PackingFormat.CANONICAL))
    ref = O._to_f32(O.reference_linear(x, q, s, z, None, out_features=n, in_features=k, x_dtype=dtype,
                                       bias_dtype="bf16"), dtype)
    assert np.isfinite(got).all()
    assert not got[2].any() and not ref[2].any()
    for r in range(rows):
        scale = float(np.abs(ref[r]).max())
        if scale == 0.0:
            continue
        err = float(np.abs(got[r] - ref[r]).max()) / scale
        # bf16 outputs: half an output ulp plus summation order; fp32: near-fp32
        assert err <= (5e-3 if dtype == "bf16" else 1e-5), (r, err)


@pytest.mark.parametrize("rows", [2, 40])
@pytest.mark.parametrize("input_kind", ["zero", "alternating", "bounded_large"])
def test_linear_matches_adversarial_inputs(input_kind, rows):
    # tests/test_triton_unpack.py:133-154 (plus a GEMM-sized variant)
    rng = np.random.default_rng(81)
    n, k = 64, 128
    q, s, z = O.quantize_asymmetric_rtn(rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.05), 64)
    if input_kind == "zero":
        x = np.zeros((rows, k), np.float16)
    elif input_kind == "alternating":
        x = np.tile(np.array([1.0, -1.0], np.float16), (rows, k // 2))
    else:
        x = np.tile(np.linspace(-8, 8, k, dtype=np.float32).astype(np.float16), (rows, 1))
    check_linear(x, q, s, z, None, n, k, "fp16")


@pytest.mark.parametrize("rows", [1, 32])
def test_linear_boundary_zero_points_exact(rows):
    # tests/test_backends.py:91-104, worked out by hand to [[-360, -1440]]
    codes = np.tile(np.array([-8, 7], dtype=np.int8), 2 * 128 // 2)
    q = O.pack_int4(codes)
    z = O.pack_int4(np.array([-8, 7, 7, -8], dtype=np.int8))
    s = np.array([[0.25, 0.5], [1.0, 2.0]], dtype=np.float16)
    x = np.tile(np.array([1.0, -1.0], np.float16), (rows, 64))
    for dtype in ("fp16", "bf16"):
        xd = O._from_f32(x.astype(np.float32), dtype)
        got = linear_canonical_w4g64_hip(to_dev(xd, dtype), *dev_weights(q, s, z))
        np.testing.assert_array_equal(from_dev(got), np.tile(np.array([[-360.0, -1440.0]], np.float32), (rows, 1)))


@pytest.mark.parametrize("rows", [1, 7, 16, 48, 200])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_one_hot_activations_reproduce_dequantized_weights_exactly(rows, dtype):
    """x = e_k gives y[m, n] = round(W[n, k_m]) -- pins the MFMA operand and
    accumulator layouts, the nibble order and the scale/zero indexing."""
    n, k = 200, 640
    q, s, z = weights("asym", n, k, 4242)
    w = O.dequantize_groupwise(q, s, zeros=z, out_features=n, in_features=k, group_size=64,
                               packing=PackingFormat.CANONICAL)
    ks = np.random.default_rng(rows).integers(0, k, size=rows)
    x = np.zeros((rows, k), np.float32)
    x[np.arange(rows), ks] = 1.0
    got = linear_canonical_w4g64_hip(to_dev(O._from_f32(x, dtype), dtype), *dev_weights(q, s, z))
    expected = O._to_f32(O._from_f32(w[:, ks].T.copy(), dtype), dtype)
    np.testing.assert_array_equal(from_dev(got), expected)


@pytest.mark.parametrize(
    ("rows", "n", "k"),
    [(1, 6, 128), (3, 100, 64), (4, 7, 192), (16, 200, 640), (17, 64, 128), (33, 1000, 192), (127, 130, 256),
     (129, 72, 512)],
)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_ragged_shapes(rows, n, k, dtype):
    """Ragged feature counts and K: the scale and zero-point arrays end
    mid-way through a 16-byte chunk (6 x 2 groups, 7 x 3 groups), which the
    decode kernels stage per workgroup in 16-byte chunks."""
    q, s, z = weights("asym", n, k, rows * 1000 + n + k)
    x = O.activations(rows, k, seed=rows + n, dtype=dtype)
    bias = O._from_f32(np.linspace(-0.3, 0.3, n, dtype=np.float32), "fp16")
    check_linear(x, q, s, z, bias, n, k, dtype, bias_dtype="fp16")


@pytest.mark.parametrize(
    ("rows", "n", "k"),
    [(9, 1536, 1536), (12, 256, 1536), (16, 8960, 1536), (16, 1536, 8960), (13, 72, 3072), (16, 40, 9280),
     (10, 96, 64), (9, 8200, 512), (12, 7, 192), (16, 13, 8960)],
)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_decode_nine_to_sixteen_rows(rows, n, k, dtype):
    """Rows 9..16: K a multiple of 256 runs the pipelined kernel (two A tiles;
    long K (8960) split across workgroups; n = 13, 72: one partial row
    block), other K the 16-row kernel that stages the activations in LDS and
    splits K across the waves of each 16-feature block (K = 9280 also across
    workgroups; n = 40: the second block is partly past N)."""
    from qwen_int4_hip import linear_kernel_name

    assert linear_kernel_name(rows, n, k, torch.float16 if dtype == "fp16" else torch.bfloat16).startswith(
        decode_kernel_prefix(rows, k))
    q, s, z = weights("asym", n, k, rows * 7 + n + k)
    x = O.activations(rows, k, seed=rows + 2 * n, dtype=dtype, outliers=True)
    bias = O._from_f32(np.linspace(-0.5, 0.5, n, dtype=np.float32), dtype)
    check_linear(x, q, s, z, bias, n, k, dtype, bias_dtype=dtype)


def test_leading_dims_noncontiguous_and_empty_inputs():
    n, k = 96, 256
    q, s, z = weights("asym", n, k, 17)
    x = O.activations(6, k, seed=3, dtype="bf16").reshape(2, 3, k)
    check_linear(x, q, s, z, None, n, k, "bf16")
    # non-contiguous activations (tests/test_backends.py:79-88)
    xt = torch.arange(4 * k, dtype=torch.float32).reshape(k, 4).t().to(torch.bfloat16).to(DEV) / 100
    assert not xt.is_contiguous()
    got = hip_w4g64_linear(xt, *dev_weights(q, s, z), None, out_features=n, in_features=k, group_size=64,
                           packing=PackingFormat.CANONICAL)
    ref = O.reference_linear(O.f32_to_bf16_bits(xt.float().cpu().numpy()), q, s, z, None, out_features=n,
                             in_features=k, x_dtype="bf16")
    np.testing.assert_allclose(from_dev(got), O.bf16_bits_to_f32(ref), rtol=0.02, atol=0.25)
    empty = hip_w4g64_linear(torch.zeros(0, k, dtype=torch.float16, device=DEV), *dev_weights(q, s, z), None,
                             out_features=n, in_features=k, group_size=64, packing=PackingFormat.CANONICAL)
    assert empty.shape == (0, n)


def test_linear_rejects_noncanonical_contract():
    values = torch.zeros((1, 64), dtype=torch.float16, device=DEV)
    qweight = torch.zeros(32, dtype=torch.uint8, device=DEV)
    scales = torch.ones(1, dtype=torch.float16, device=DEV)
    zeros = torch.zeros(1, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="qweight size"):
        linear_canonical_w4g64_hip(values, qweight[:-1], scales, zeros)
    with pytest.raises(ValueError, match="activations"):
        linear_canonical_w4g64_hip(values.unsqueeze(0), qweight, scales, zeros)
    with pytest.raises(ValueError, match="W4G64"):
        hip_w4g64_linear(values, qweight, scales, zeros, None, out_features=1, in_features=64, group_size=128,
                         packing=PackingFormat.CANONICAL)


def test_determinism_and_workspace_reuse_across_shapes():
    """Split-K partial sums are reduced in a fixed order and every call writes
    the partials it reads: repeated, interleaved calls on one workspace are
    bitwise equal."""
    cases = []
    for (name, rows) in [("down_proj", 1), ("q_proj", 4), ("gate_proj", 1), ("k_proj", 16), ("down_proj", 16)]:
        n, k = SHAPES[name]
        q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
        x = to_dev(O.activations(rows, k, seed=rows, dtype="fp16"), "fp16")
        cases.append((x, dev_weights(q, s, z)))
    first = [linear_canonical_w4g64_hip(x, *w) for x, w in cases]
    for _ in range(3):
        again = [linear_canonical_w4g64_hip(x, *w) for x, w in cases]
        for a, b in zip(first, again):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_linearity_at_full_size():
    n, k = SHAPES["gate_proj"]
    q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
    w = dev_weights(q, s, z)
    rng = np.random.default_rng(1)
    x1 = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32)).to(DEV)
    x2 = torch.from_numpy(rng.standard_normal((4, k)).astype(np.float32)).to(DEV)
    y12 = linear_canonical_w4g64_hip(x1 + 2 * x2, *w)
    y1, y2 = linear_canonical_w4g64_hip(x1, *w), linear_canonical_w4g64_hip(x2, *w)
    torch.testing.assert_close(y12, y1 + 2 * y2, rtol=1e-4, atol=1e-4)


def test_quantlinear_dispatch_matches_oracle():
    # tests/test_triton_unpack.py:157-189 (bias, leading dims, fp32 input)
    rng = np.random.default_rng(117)
    q, s, z = O.quantize_asymmetric_rtn(rng.standard_normal((64, 128)).astype(np.float32) * np.float32(0.1), 64)
    layer = QuantLinear(128, 64, group_size=64, bias=True, packing=PackingFormat.CANONICAL).to(DEV)
    layer.qweight.copy_(torch.from_numpy(q))
    layer.scales.copy_(torch.from_numpy(s))
    layer.zeros.copy_(torch.from_numpy(z))
    bias = O.f32_to_bf16_bits(rng.standard_normal(64).astype(np.float32) * np.float32(0.01))
    layer.bias.copy_(to_dev(bias, "bf16"))
    x = O.activations(6, 128, seed=118, dtype="bf16").reshape(2, 3, 128)
    got = layer(to_dev(x, "bf16"))
    ref = O.reference_linear(x, q, s, z, bias, out_features=64, in_features=128, x_dtype="bf16")
    np.testing.assert_allclose(from_dev(got), O.bf16_bits_to_f32(ref), rtol=0.02, atol=0.25)
    x32 = O.activations(2, 128, seed=119, dtype="fp32")
    got32 = layer(to_dev(x32, "fp32"))
    ref32 = O.reference_linear(x32, q, s, z, bias, out_features=64, in_features=128, x_dtype="fp32")
    np.testing.assert_allclose(from_dev(got32), ref32, rtol=1e-5, atol=1e-5)


def test_hip_graph_capture_replays_match_eager():
    """The decode GEMV (split-K: partials, then the split-reduce kernel) and the GEMM inside a
    captured HIP graph: several replays, with eager work and synchronizations
    between them, each equal to the eager result bit for bit."""
    calls = []
    for name, rows in (("down_proj", 1), ("gate_proj", 4), ("q_proj", 16), ("down_proj", 200)):
        n, k = SHAPES[name]
        q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
        dtype = "fp16" if rows <= 16 else "bf16"
        calls.append((to_dev(O.activations(rows, k, seed=rows + 5, dtype=dtype), dtype), dev_weights(q, s, z)))
    eager = [linear_canonical_w4g64_hip(x, *w) for x, w in calls]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        for x, w in calls:  # warm-up on the capture stream: its workspace exists before capture
            linear_canonical_w4g64_hip(x, *w)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = [linear_canonical_w4g64_hip(x, *w) for x, w in calls]
    for replay in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(captured, eager):
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"replay {replay} differs"
        # eager work on the default stream between replays
        again = [linear_canonical_w4g64_hip(x, *w) for x, w in calls]
        torch.cuda.synchronize()
        for got, ref in zip(again, eager):
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_graphs_captured_before_and_after_workspace_growth_both_replay():
    """A small-row graph captured on a stream, then (after an eager call grows
    that stream's workspace) a large-row graph on the same stream: both keep
    replaying correctly, interleaved -- the first graph's workspace was not
    freed when the buffer grew."""
    n, k = SHAPES["down_proj"]
    q, s, z = weights("sym", n, k, O.BASE_SEED + n + k)
    w = dev_weights(q, s, z)
    small = to_dev(O.activations(4, k, seed=31, dtype="fp16"), "fp16")  # split-K GEMV: partials
    large = to_dev(O.activations(200, k, seed=32, dtype="bf16"), "bf16")  # split-K GEMM: tens of MB of partials
    want_small = linear_canonical_w4g64_hip(small, *w)
    want_large = linear_canonical_w4g64_hip(large, *w)
    from qwen_int4_hip import kernels

    side = torch.cuda.Stream()
    graphs, outs, buffers = [], [], []
    for x in (small, large):
        with torch.cuda.stream(side):
            linear_canonical_w4g64_hip(x, *w)  # warm-up: grows this stream's workspace outside capture
        torch.cuda.synchronize()
        buffers.append(kernels._workspaces[(torch.cuda.current_device(), side.cuda_stream)])
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            outs.append(linear_canonical_w4g64_hip(x, *w))
        graphs.append(graph)
    assert buffers[1] is not buffers[0] and any(b is buffers[0] for b in kernels._retired)  # the buffer grew in between
    for replay in range(3):
        for graph in (graphs[1], graphs[0]):
            graph.replay()
            torch.cuda.synchronize()
            linear_canonical_w4g64_hip(large, *w)  # eager work on the default stream between replays
        assert torch.equal(outs[0].view(torch.int16), want_small.view(torch.int16)), f"replay {replay}"
        assert torch.equal(outs[1].view(torch.int16), want_large.view(torch.int16)), f"replay {replay}"
