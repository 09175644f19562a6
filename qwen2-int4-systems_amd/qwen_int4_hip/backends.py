"""Operator backends for quantized linear layers: the reference's registry
(src/qwen_int4/backends.py:11) plus the ``"hip"`` backend.

Counterpart of the reference's backend registry and dispatch shims
(src/qwen_int4/backends.py:11, :14-70, :73-98, :101-150, :153-181).
Selection stays explicit: a module picks a backend by name, there is no
environment switch and no silent fallback between arms.
  * ``"hip"``: the MI355X kernels; fails loudly without a ROCm GPU and the
    built library.  fp32 activations, which the reference's Triton arm routes
    to its torch path (backends.py:172-177), run natively here.
  * ``"torch"``: dequantize the whole weight to fp32, then one fp32 matmul
    (backends.py:73-98) -- plain PyTorch on whatever device the tensors live.
  * ``"lpu"``: the reference's A/B/C-dataflow emulation (backends.py:101-150):
    validated inputs, one fp32 product per 64-wide K group, accumulated in
    group order.
  * ``"triton"``: kept in the registry for configuration compatibility; this
    build has no Triton, so the arm raises (as the reference's does without a
    Triton installation, backends.py:166-167).
"""

from __future__ import annotations

import torch

from .kernels import hip_available, linear_canonical_w4g64_hip
from .quantization import PackingFormat, dequantize_groupwise, unpack_int4

SUPPORTED_BACKENDS = ("torch", "lpu", "triton", "hip")


def validate_canonical_w4g64_inputs(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    out_features: int,
    in_features: int,
    group_size: int,
    packing: PackingFormat | str,
    check_values: bool = True,
) -> PackingFormat:
    """Fail closed on inputs outside the frozen canonical W4G64 contract.

    Same checks, order, exception types and messages as the reference's
    ``_validate_lpu_functional_inputs`` (backends.py:14-70).  With
    ``check_values`` the scales are scanned for non-finite/non-positive
    values, which needs a device-to-host sync; the per-call HIP path skips it
    (as the reference's Triton path does) and loaders call it once.
    """
    packing = PackingFormat(packing)
    if packing is not PackingFormat.CANONICAL:
        raise ValueError("HIP backend supports only canonical INT4 packing")
    if group_size != 64:
        raise ValueError("HIP backend supports only canonical W4G64 tensors")
    if in_features <= 0 or out_features <= 0 or in_features % group_size:
        raise ValueError("linear dimensions must be positive and divisible by group size 64")
    if x.ndim < 1 or x.shape[-1] != in_features:
        raise ValueError("activation feature dimension does not match QuantLinear")
    if x.dtype not in {torch.float16, torch.bfloat16, torch.float32}:
        raise TypeError("HIP activations must use FP16, BF16, or FP32")
    if qweight.dtype != torch.uint8 or zeros.dtype != torch.uint8:
        raise TypeError("canonical packed weights and zero points must use uint8 storage")
    if scales.dtype != torch.float16:
        raise TypeError("canonical group scales must use FP16 storage")
    groups = in_features // group_size
    expected_weight_bytes = out_features * in_features // 2
    expected_zero_bytes = (out_features * groups + 1) // 2
    if qweight.numel() != expected_weight_bytes:
        raise ValueError(f"qweight must contain {expected_weight_bytes} bytes, got {qweight.numel()}")
    if tuple(scales.shape) != (out_features, groups):
        raise ValueError(f"scales must have shape {(out_features, groups)}, got {tuple(scales.shape)}")
    if zeros.numel() != expected_zero_bytes:
        raise ValueError(f"zeros must contain {expected_zero_bytes} bytes, got {zeros.numel()}")
    if bias is not None and tuple(bias.shape) != (out_features,):
        raise ValueError(f"bias must have shape {(out_features,)}, got {tuple(bias.shape)}")
    tensors = (qweight, scales, zeros) + (() if bias is None else (bias,))
    if any(tensor.device != x.device for tensor in tensors):
        raise ValueError("all HIP backend inputs must be on the same device")
    if check_values:
        if not torch.isfinite(scales).all() or torch.any(scales <= 0):
            raise ValueError("canonical group scales must be finite and strictly positive")
        if bias is not None and not torch.isfinite(bias).all():
            raise ValueError("bias values must be finite")
    return packing


def hip_w4g64_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    out_features: int,
    in_features: int,
    group_size: int,
    packing: PackingFormat | str,
) -> torch.Tensor:
    """Dispatch canonical W4G64 linear to the MI355X kernels.

    Signature and result contract of the reference backends
    (backends.py:153-181): ``x`` is ``[..., in_features]`` fp16/bf16/fp32,
    the result is ``[..., out_features]`` in ``x.dtype``.
    """
    if not hip_available():
        raise RuntimeError("HIP backend requires a ROCm GPU and the built libw4g64_hip library")
    validate_canonical_w4g64_inputs(
        x, qweight, scales, zeros, bias, out_features=out_features, in_features=in_features,
        group_size=group_size, packing=packing, check_values=False,
    )
    rows = x.numel() // in_features
    if rows == 0:
        return x.new_empty((*x.shape[:-1], out_features))
    output = linear_canonical_w4g64_hip(x.reshape(-1, in_features).contiguous(), qweight, scales, zeros, bias)
    return output.reshape(*x.shape[:-1], out_features)


def torch_w4g64_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    out_features: int,
    in_features: int,
    group_size: int,
    packing: PackingFormat | str,
) -> torch.Tensor:
    """The reference's correctness-first arm (backends.py:73-98): the fp32
    weight (code - zero) * scale, one fp32 matmul, fp32 bias, cast to
    ``x.dtype``."""
    weight = dequantize_groupwise(qweight, scales, zeros=zeros, out_features=out_features,
                                  in_features=in_features, group_size=group_size, packing=packing)
    out = torch.matmul(x.reshape(-1, in_features).to(torch.float32), weight.t())
    if bias is not None:
        out = out + bias.to(torch.float32)
    return out.reshape(*x.shape[:-1], out_features).to(x.dtype)


def lpu_w4g64_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bias: torch.Tensor | None,
    *,
    out_features: int,
    in_features: int,
    group_size: int,
    packing: PackingFormat | str,
) -> torch.Tensor:
    """The reference's LPU-style dataflow emulation (backends.py:101-150):
    validated canonical inputs, then per K group an fp32 A tile times the
    group's dequantized B tile, added into an fp32 C buffer in group order,
    then the fp32 bias."""
    packing = validate_canonical_w4g64_inputs(
        x, qweight, scales, zeros, bias, out_features=out_features, in_features=in_features,
        group_size=group_size, packing=packing,
    )
    groups = in_features // group_size
    codes = unpack_int4(qweight, packing=packing).reshape(out_features, groups, group_size).to(torch.float32)
    zero_points = unpack_int4(zeros, packing=packing, elements=out_features * groups).reshape(
        out_features, groups).to(torch.float32)
    a = x.reshape(-1, in_features).to(torch.float32)
    c = torch.zeros((a.shape[0], out_features), dtype=torch.float32, device=x.device)
    for g in range(groups):
        b_tile = (codes[:, g, :] - zero_points[:, g:g + 1]) * scales[:, g:g + 1].to(torch.float32)
        c.add_(torch.matmul(a[:, g * group_size:(g + 1) * group_size], b_tile.t()))
    if bias is not None:
        c.add_(bias.to(torch.float32))
    return c.reshape(*x.shape[:-1], out_features).to(x.dtype)


def triton_w4g64_linear(x, qweight, scales, zeros, bias, **kwargs) -> torch.Tensor:
    """Registry arm of the reference's Triton operator (backends.py:153-181).
    This build carries no Triton: the arm raises, as the reference's does
    without a Triton installation (backends.py:166-167)."""
    raise RuntimeError("Triton backend requires CUDA and a Triton installation; this build provides the 'hip' backend")


BACKEND_IMPLEMENTATIONS = {
    "torch": torch_w4g64_linear,
    "lpu": lpu_w4g64_linear,
    "triton": triton_w4g64_linear,
    "hip": hip_w4g64_linear,
}
