"""The reference's backend arms kept in this package's registry
(src/qwen_int4/backends.py:11, :73-98, :101-150, :153-181): ``"torch"`` and
``"lpu"`` against the oracle's restatements of the same functions, the
``"triton"`` arm's failure, and QuantLinear's dispatch by name
(tests/test_backends.py:140-143 style).  CPU only."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from qwen_int4_hip import PackingFormat, QuantLinear
from qwen_int4_hip.backends import lpu_w4g64_linear, torch_w4g64_linear


def _case(n, k, rows, dtype, asym, seed):
    if asym:
        qweight, scales, zeros = O.asymmetric_weights(n, k, seed=seed)
    else:
        qweight, scales, zeros = O.symmetric_weights(n, k, seed=seed)
    x = O.activations(rows, k, seed=seed + 1, dtype=dtype)
    bias = O.f32_to_bf16_bits(np.linspace(-0.25, 0.25, n, dtype=np.float32))
    return x, qweight, scales, zeros, bias


def _torch_x(x, dtype):
    if dtype == "bf16":
        return torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(x))


def _tensors(qweight, scales, zeros, bias):
    return (torch.from_numpy(qweight), torch.from_numpy(scales), torch.from_numpy(zeros),
            torch.from_numpy(bias.view(np.int16)).view(torch.bfloat16))


def _f32(t):
    return t.to(torch.float32).numpy()


@pytest.mark.parametrize("dtype", ["fp16", "bf16", "fp32"])
@pytest.mark.parametrize("asym", [False, True])
def test_torch_arm_matches_oracle_reference_linear(dtype, asym):
    n, k, rows = 96, 256, 3
    x, qweight, scales, zeros, bias = _case(n, k, rows, dtype, asym, O.BASE_SEED + 31)
    q, s, z, b = _tensors(qweight, scales, zeros, bias)
    got = torch_w4g64_linear(_torch_x(x, dtype), q, s, z, b, out_features=n, in_features=k, group_size=64,
                             packing=PackingFormat.CANONICAL)
    ref = O.reference_linear(x, qweight, scales, zeros, bias, out_features=n, in_features=k, x_dtype=dtype,
                             bias_dtype="bf16", return_f32=True)
    # same dequantized fp32 weight and fp32 accumulation; only the matmul's summation order may differ
    got32 = _f32(got)
    ref_cast = O._to_f32(O._from_f32(ref, dtype), dtype)
    err = np.abs(got32 - ref_cast).max() / max(np.abs(ref_cast).max(), 1e-30)
    assert got.dtype == _torch_x(x, dtype).dtype and got.shape == (rows, n)
    assert err <= {"fp16": 2e-3, "bf16": 1e-2, "fp32": 1e-5}[dtype]


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_lpu_arm_matches_oracle_lpu_functional_linear(dtype):
    n, k, rows = 64, 192, 2
    x, qweight, scales, zeros, bias = _case(n, k, rows, dtype, True, O.BASE_SEED + 37)
    q, s, z, b = _tensors(qweight, scales, zeros, bias)
    got = lpu_w4g64_linear(_torch_x(x, dtype), q, s, z, b, out_features=n, in_features=k, group_size=64,
                           packing="canonical")
    ref = O.lpu_functional_linear(x, qweight, scales, zeros, bias, out_features=n, in_features=k,
                                  x_dtype=dtype, bias_dtype="bf16")
    ref32 = O._to_f32(ref, dtype)
    err = np.abs(_f32(got) - ref32).max() / max(np.abs(ref32).max(), 1e-30)
    assert err <= {"fp16": 2e-3, "bf16": 1e-2}[dtype]


def test_lpu_arm_fails_closed_like_the_reference():
    n, k = 8, 64
    x, qweight, scales, zeros, bias = _case(n, k, 1, "fp16", False, O.BASE_SEED + 41)
    q, s, z, b = _tensors(qweight, scales, zeros, bias)
    s = s.clone()
    s[0, 0] = 0
    with pytest.raises(ValueError, match="finite and strictly positive"):
        lpu_w4g64_linear(_torch_x(x, "fp16"), q, s, z, b, out_features=n, in_features=k, group_size=64,
                         packing="canonical")


def test_quantlinear_dispatches_by_name_and_triton_arm_raises():
    n, k = 32, 128
    x, qweight, scales, zeros, bias = _case(n, k, 2, "fp16", False, O.BASE_SEED + 43)
    layer = QuantLinear(k, n, group_size=64, bias=True, backend="torch", packing=PackingFormat.CANONICAL)
    q, s, z, b = _tensors(qweight, scales, zeros, bias)
    layer.qweight.copy_(q.reshape(-1, 1))
    layer.scales.copy_(s)
    layer.zeros.copy_(z.reshape(-1, 1))
    layer.bias.copy_(b)
    xt = _torch_x(x, "fp16")
    via_torch = layer(xt)
    layer.set_backend("lpu")
    via_lpu = layer(xt)
    ref = O._to_f32(O.reference_linear(x, qweight, scales, zeros, bias, out_features=n, in_features=k,
                                       x_dtype="fp16", bias_dtype="bf16"), "fp16")
    for got in (via_torch, via_lpu):
        assert np.abs(_f32(got) - ref).max() <= 2e-3 * np.abs(ref).max()
    layer.set_backend("triton")
    with pytest.raises(RuntimeError, match="Triton backend requires"):
        layer(xt)
