"""Packed INT4 storage format and the offline quantizers of the W4G64 contract.

Mirrors src/qwen_int4/quantization.py: the packing-format identity
(:17-20), pack / unpack (:23-84), symmetric and asymmetric RTN quantizers
(:87-162) and group-wise dequantization (:221-258), with the same arguments,
results and error messages.  Unlike the reference, which moves every input to
the CPU, these run on the device of their input, so a GPU caller can generate
and check full-size layers without a host round trip; the arithmetic is the
same IEEE fp32 sequence (correctly rounded division, round half to even), so
results are bit-identical on every device.

Only the canonical format reaches the HIP kernels; ``LEGACY_SIGNED_ADD`` is
kept so the enum values (and therefore module state and checkpoint metadata)
match the reference, and so the kernels can reject it by name.
"""

from __future__ import annotations

from enum import Enum

import torch


class PackingFormat(str, Enum):
    # Canonical v1: byte = q[k] in low nibble | q[k+1] in high nibble.
    CANONICAL = "canonical"
    LEGACY_SIGNED_ADD = "legacy_signed_add"


# Format identity strings of the canonical W4G64 checkpoint metadata
# (src/qwen_int4/export.py:38-57; scripts/quantize_model.py:148-162).
CANONICAL_PACKING_METADATA = "canonical_low_nibble_k_even_high_nibble_k_odd"
WEIGHT_LAYOUT_METADATA = "row_major_[out_features,in_features]"
SCALE_LAYOUT_METADATA = "[out_features,in_features/group_size]"


def pack_int4(codes: torch.Tensor, *, packing: PackingFormat | str = PackingFormat.CANONICAL) -> torch.Tensor:
    """Two signed INT4 codes per byte (quantization.py:30-50): canonical puts
    the even element in the low nibble; legacy stores ``(first << 4) + second``."""
    packing = PackingFormat(packing)
    flat = codes.reshape(-1).to(torch.int16)
    if flat.numel() % 2:
        raise ValueError("INT4 packing requires an even number of elements")
    if flat.numel() and (int(flat.min()) < -8 or int(flat.max()) > 7):
        raise ValueError("signed INT4 codes must be in [-8, 7]")
    even, odd = flat[0::2], flat[1::2]
    if packing is PackingFormat.LEGACY_SIGNED_ADD:
        byte = even * 16 + odd
    else:
        byte = (even & 0xF) + (odd & 0xF) * 16
    return (byte & 0xFF).to(torch.uint8)


def unpack_int4(packed: torch.Tensor, *, packing: PackingFormat | str = PackingFormat.CANONICAL,
                elements: int | None = None) -> torch.Tensor:
    """Interleaved int8 codes from packed bytes (quantization.py:53-84); the
    legacy format first undoes the borrow a negative low nibble took from the
    high one."""
    packing = PackingFormat(packing)
    byte = packed.reshape(-1).to(torch.uint8).to(torch.int16)
    lo = byte & 0xF
    hi = byte >> 4
    if packing is PackingFormat.LEGACY_SIGNED_ADD:
        hi = (hi + (lo >> 3)) & 0xF
    lo = lo - ((lo & 8) << 1)  # sign extension of a nibble
    hi = hi - ((hi & 8) << 1)
    first, second = (hi, lo) if packing is PackingFormat.LEGACY_SIGNED_ADD else (lo, hi)
    out = torch.stack((first, second), dim=1).reshape(-1).to(torch.int8)
    if elements is not None:
        if elements < 0 or elements > out.numel():
            raise ValueError(f"invalid element count {elements} for {out.numel()} decoded values")
        out = out[:elements]
    return out


def _div(a: torch.Tensor, b) -> torch.Tensor:
    """Correctly rounded fp32 quotient on any device: the fp64 quotient of two
    fp32 values rounded to fp32 equals the correctly rounded fp32 quotient
    (53 >= 2 * 24 + 2 makes the double rounding innocuous), whereas a device's
    fast fp32 division may be off by one unit in the last place."""
    b64 = b.to(torch.float64) if isinstance(b, torch.Tensor) else float(b)
    return (a.to(torch.float64) / b64).to(torch.float32)


def _grouped(weight: torch.Tensor, group_size: int) -> torch.Tensor:
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2D, got shape={tuple(weight.shape)}")
    out_features, in_features = weight.shape
    if in_features % group_size:
        raise ValueError(f"in_features={in_features} is not divisible by group_size={group_size}")
    return weight.detach().to(torch.float32).reshape(out_features, in_features // group_size, group_size)


def quantize_symmetric_rtn(weight: torch.Tensor, *, group_size: int = 128,
                           packing: PackingFormat | str = PackingFormat.CANONICAL) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-(row, group) symmetric RTN (quantization.py:87-111): fp32 scale
    max|w| / 7 (1 for an all-zero group), codes round-half-even(w / scale)
    clamped to [-7, 7]; the codes use the fp32 scale, the stored scale is its
    fp16 rounding.  Returns (packed [N*K/2, 1] uint8, scales fp16 [N, G])."""
    grouped = _grouped(weight, group_size)
    scale = _div(grouped.abs().amax(dim=-1), 7.0)
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    codes = torch.round(_div(grouped, scale.unsqueeze(-1))).clamp(-7, 7).to(torch.int8)
    return pack_int4(codes, packing=packing).reshape(-1, 1), scale.to(torch.float16)


def quantize_asymmetric_rtn(weight: torch.Tensor, *, group_size: int = 128, clip_max: torch.Tensor | None = None,
                            packing: PackingFormat | str = PackingFormat.CANONICAL
                            ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Asymmetric RTN with unsigned codes and zero points in [0, 15] stored
    shifted by -8 as signed nibbles (quantization.py:114-162).  Returns
    (packed weights [N*K/2, 1], scales fp16 [N, G], packed zeros
    [(N*G+1)//2, 1]); an odd zero count is padded with one zero nibble."""
    grouped = _grouped(weight, group_size)
    out_features, groups, _ = grouped.shape
    if clip_max is not None:
        limit = clip_max.detach().to(device=grouped.device, dtype=torch.float32)
        if tuple(limit.shape) != (out_features, groups):
            raise ValueError(f"clip_max must have shape {(out_features, groups)}, got {tuple(limit.shape)}")
        if not bool(torch.isfinite(limit).all()) or bool((limit <= 0).any()):
            raise ValueError("clip_max values must be finite and positive")
        limit = limit.unsqueeze(-1)
        grouped = torch.maximum(torch.minimum(grouped, limit), -limit)
    zero = torch.zeros((), dtype=torch.float32, device=grouped.device)
    low = torch.minimum(grouped.amin(dim=-1), zero)
    high = torch.maximum(grouped.amax(dim=-1), zero)
    scale = _div((high - low).clamp_min(1e-5), 15.0)
    zero_point = torch.round(_div(-low, scale)).clamp(0, 15)
    codes = (torch.round(_div(grouped, scale.unsqueeze(-1))) + zero_point.unsqueeze(-1)).clamp(0, 15)
    signed_codes = (codes.to(torch.int16) - 8).to(torch.int8)
    signed_zeros = (zero_point.to(torch.int16) - 8).to(torch.int8).reshape(-1)
    if signed_zeros.numel() % 2:
        signed_zeros = torch.cat((signed_zeros, signed_zeros.new_zeros(1)))
    return (pack_int4(signed_codes, packing=packing).reshape(-1, 1), scale.to(torch.float16),
            pack_int4(signed_zeros, packing=packing).reshape(-1, 1))


def dequantize_groupwise(qweight: torch.Tensor, scales: torch.Tensor, *, out_features: int, in_features: int,
                         group_size: int, packing: PackingFormat | str = PackingFormat.LEGACY_SIGNED_ADD,
                         zeros: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 [N, K] = (code - zero) * scale, group-wise along K
    (quantization.py:221-258; note the reference's LEGACY default packing)."""
    if in_features % group_size:
        raise ValueError(f"in_features={in_features} is not divisible by group_size={group_size}")
    groups = in_features // group_size
    if tuple(scales.shape) != (out_features, groups):
        raise ValueError(f"scale shape must be {(out_features, groups)}, got {tuple(scales.shape)}")
    if qweight.numel() != out_features * in_features // 2:
        raise ValueError(f"qweight must contain {out_features * in_features // 2} bytes, got {qweight.numel()}")
    codes = unpack_int4(qweight, packing=packing).reshape(out_features, groups, group_size).to(torch.float32)
    if zeros is None:
        zero_points = torch.zeros((out_features, groups), dtype=torch.float32, device=codes.device)
    else:
        if zeros.numel() != (out_features * groups + 1) // 2:
            raise ValueError(f"zeros must contain {(out_features * groups + 1) // 2} bytes, got {zeros.numel()}")
        zero_points = unpack_int4(zeros, packing=packing, elements=out_features * groups).reshape(
            out_features, groups).to(torch.float32)
    weight = (codes - zero_points.unsqueeze(-1)) * scales.to(torch.float32).unsqueeze(-1)
    return weight.reshape(out_features, in_features)
