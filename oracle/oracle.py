"""CPU oracle for the canonical W4G64 linear path -- TEST INFRASTRUCTURE ONLY.

This module is the checker.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the CPU-baseline leg of ``bench.py`` import it; the HIP product package never
does, and nothing here is ever used as a fallback for the product path.

It holds two independent restatements of the reference algorithm:

* numpy (this file): vectorised codec, quantizers, dequantization, the
  fp32 linear, the LPU K-streaming emulation and the tensor metrics;
* C (``w4g64_oracle.c``, built by ``oracle/Makefile`` into
  ``oracle/_build/libw4g64_oracle.so``), loaded here through ctypes.

The tests pin both against the reference's known-answer vectors, exhaustive
byte tables, hand-derived quantization ties, closed forms and each other.

bfloat16 arrays are carried as ``uint16`` bit patterns (numpy has no bf16);
fp16 arrays are ``numpy.float16``.
"""

from __future__ import annotations

import ctypes
import os
from enum import Enum
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
C_LIBRARY = ORACLE_DIR / "_build" / "libw4g64_oracle.so"


class PackingFormat(str, Enum):
    """quantization.py:17-20."""

    CANONICAL = "canonical"
    LEGACY_SIGNED_ADD = "legacy_signed_add"


# ---------------------------------------------------------------------------
# dtype helpers (fp32 <-> bf16 bits, round to nearest even; torch semantics)
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(values: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (x & 0x7FFFFFFF) > 0x7F800000
    rounded = ((x + 0x7FFF + ((x >> 16) & 1)) >> 16).astype(np.uint16)
    quiet = ((x >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# INT4 codec: quantization.py:23-84
# ---------------------------------------------------------------------------

def pack_int4(codes: np.ndarray, packing: PackingFormat | str = PackingFormat.CANONICAL) -> np.ndarray:
    """quantization.py:30-50: consecutive signed INT4 pairs -> uint8."""
    packing = PackingFormat(packing)
    flat = np.asarray(codes).reshape(-1).astype(np.int16)
    if flat.size % 2:                                                   # :24-25
        raise ValueError("INT4 packing requires an even number of elements")
    if flat.size and (flat.min() < -8 or flat.max() > 7):               # :26-27
        raise ValueError("signed INT4 codes must be in [-8, 7]")
    first, second = flat[0::2], flat[1::2]
    if packing is PackingFormat.LEGACY_SIGNED_ADD:
        packed = (first << 4) + second                                   # :46-47
    else:
        packed = (first & 0x0F) | ((second & 0x0F) << 4)                 # :49
    return (packed & 0xFF).astype(np.uint8)


def unpack_int4(
    packed: np.ndarray,
    packing: PackingFormat | str = PackingFormat.CANONICAL,
    elements: int | None = None,
) -> np.ndarray:
    """quantization.py:53-84: uint8 -> interleaved signed int8."""
    packing = PackingFormat(packing)
    byte = np.asarray(packed).reshape(-1).astype(np.uint8)
    low_u = (byte & 0x0F).astype(np.int16)
    high_u = (byte >> 4).astype(np.int16)
    if packing is PackingFormat.LEGACY_SIGNED_ADD:
        high_u = (high_u + (low_u >= 8).astype(np.int16)) & 0x0F         # :65-68
    low = np.where(low_u >= 8, low_u - 16, low_u)                       # :70
    high = np.where(high_u >= 8, high_u - 16, high_u)                   # :71
    result = np.empty(byte.size * 2, dtype=np.int8)
    if packing is PackingFormat.LEGACY_SIGNED_ADD:
        result[0::2], result[1::2] = high, low                          # :73-75
    else:
        result[0::2], result[1::2] = low, high                          # :76-78
    if elements is not None:
        if elements < 0 or elements > result.size:                      # :80-82
            raise ValueError(f"invalid element count {elements} for {result.size} decoded values")
        result = result[:elements]
    return result


# ---------------------------------------------------------------------------
# Quantizers: quantization.py:87-162 (IEEE fp32 arithmetic, round half even)
# ---------------------------------------------------------------------------

def quantize_symmetric_rtn(
    weight: np.ndarray, group_size: int = 128, packing: PackingFormat | str = PackingFormat.CANONICAL
) -> tuple[np.ndarray, np.ndarray]:
    """quantization.py:87-111.  Returns (qweight uint8 [N*K/2, 1], scales fp16 [N, G])."""
    weight = np.asarray(weight, dtype=np.float32)
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2D, got shape={weight.shape}")
    out_features, in_features = weight.shape
    if in_features % group_size:
        raise ValueError(f"in_features={in_features} is not divisible by group_size={group_size}")
    groups = in_features // group_size
    grouped = weight.reshape(out_features, groups, group_size)
    scales = (np.abs(grouped).max(axis=-1) / np.float32(7.0)).astype(np.float32)   # :107
    scales = np.where(scales == 0, np.float32(1.0), scales).astype(np.float32)      # :108
    codes = np.clip(np.rint(grouped / scales[..., None]), -7, 7).astype(np.int8)    # :109
    packed = pack_int4(codes, packing).reshape(-1, 1)                                # :110
    return packed, scales.astype(np.float16)                                         # :111


def quantize_asymmetric_rtn(
    weight: np.ndarray,
    group_size: int = 128,
    clip_max: np.ndarray | None = None,
    packing: PackingFormat | str = PackingFormat.CANONICAL,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """quantization.py:114-162.  Returns (qweight, scales fp16 [N, G], zeros uint8 [(N*G+1)//2, 1])."""
    weight = np.asarray(weight, dtype=np.float32)
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2D, got shape={weight.shape}")
    out_features, in_features = weight.shape
    if in_features % group_size:
        raise ValueError(f"in_features={in_features} is not divisible by group_size={group_size}")
    groups = in_features // group_size
    grouped = weight.reshape(out_features, groups, group_size)
    if clip_max is not None:                                                         # :137-147
        limits = np.asarray(clip_max, dtype=np.float32)
        if limits.shape != (out_features, groups):
            raise ValueError(f"clip_max must have shape {(out_features, groups)}, got {limits.shape}")
        if not np.isfinite(limits).all() or np.any(limits <= 0):
            raise ValueError("clip_max values must be finite and positive")
        grouped = np.maximum(np.minimum(grouped, limits[..., None]), -limits[..., None])
    zero = np.float32(0.0)
    minimum = np.minimum(grouped.min(axis=-1), zero)                                # :150
    maximum = np.maximum(grouped.max(axis=-1), zero)                                # :151
    scales = (np.maximum(maximum - minimum, np.float32(1e-5)) / np.float32(15.0)).astype(np.float32)  # :152
    unsigned_zeros = np.clip(np.rint(-minimum / scales), 0, 15).astype(np.int16)    # :153
    unsigned_codes = np.rint(grouped / scales[..., None]).astype(np.float32)        # :154
    unsigned_codes = np.clip(unsigned_codes + unsigned_zeros[..., None].astype(np.float32), 0, 15)  # :155
    signed_codes = (unsigned_codes.astype(np.int16) - 8).astype(np.int8)            # :156
    signed_zeros = (unsigned_zeros - 8).astype(np.int8).reshape(-1)                 # :157
    if signed_zeros.size % 2:                                                       # :158-159
        signed_zeros = np.concatenate((signed_zeros, np.zeros(1, dtype=np.int8)))
    qweight = pack_int4(signed_codes, packing).reshape(-1, 1)                       # :160
    zeros = pack_int4(signed_zeros, packing).reshape(-1, 1)                         # :161
    return qweight, scales.astype(np.float16), zeros


# ---------------------------------------------------------------------------
# Dequantization and linear: quantization.py:221-258, backends.py:73-150
# ---------------------------------------------------------------------------

def dequantize_groupwise(
    qweight: np.ndarray,
    scales: np.ndarray,
    *,
    out_features: int,
    in_features: int,
    group_size: int,
    packing: PackingFormat | str = PackingFormat.LEGACY_SIGNED_ADD,
    zeros: np.ndarray | None = None,
) -> np.ndarray:
    """quantization.py:221-258.  Note the reference default packing is LEGACY (:228)."""
    if in_features % group_size:
        raise ValueError(f"in_features={in_features} is not divisible by group_size={group_size}")
    groups = in_features // group_size
    scales = np.asarray(scales)
    if tuple(scales.shape) != (out_features, groups):
        raise ValueError(f"scale shape must be {(out_features, groups)}, got {tuple(scales.shape)}")
    expected_bytes = out_features * in_features // 2
    if np.asarray(qweight).size != expected_bytes:
        raise ValueError(f"qweight must contain {expected_bytes} bytes, got {np.asarray(qweight).size}")
    codes = unpack_int4(qweight, packing).reshape(out_features, in_features)
    expanded_scales = np.repeat(scales.astype(np.float32), group_size, axis=1)       # :243
    if zeros is None:
        expanded_zeros = np.zeros_like(expanded_scales)
    else:
        expected_zero_bytes = (out_features * groups + 1) // 2
        if np.asarray(zeros).size != expected_zero_bytes:
            raise ValueError(f"zeros must contain {expected_zero_bytes} bytes, got {np.asarray(zeros).size}")
        zero_values = unpack_int4(zeros, packing, elements=out_features * groups).reshape(out_features, groups)
        expanded_zeros = np.repeat(zero_values.astype(np.float32), group_size, axis=1)  # :255-257
    return (codes.astype(np.float32) - expanded_zeros) * expanded_scales             # :258


def _to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return bf16_bits_to_f32(x)
    return np.asarray(x).astype(np.float32)


def _from_f32(y: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return f32_to_bf16_bits(y)
    if dtype == "fp16":
        return y.astype(np.float16)
    return y.astype(np.float32)


def reference_linear(
    x: np.ndarray,
    qweight: np.ndarray,
    scales: np.ndarray,
    zeros: np.ndarray,
    bias: np.ndarray | None,
    *,
    out_features: int,
    in_features: int,
    group_size: int = 64,
    packing: PackingFormat | str = PackingFormat.CANONICAL,
    x_dtype: str = "fp16",
    bias_dtype: str = "bf16",
    return_f32: bool = False,
) -> np.ndarray:
    """backends.py:73-98 (torch_reference_linear): dequantize, fp32 matmul, add
    fp32 bias, cast to the activation dtype.

    ``x`` is ``[..., K]`` in ``x_dtype`` ("fp16" numpy float16, "bf16" uint16
    bits, "fp32"); the result has the same leading dims and dtype.
    """
    weight = dequantize_groupwise(
        qweight, scales, zeros=zeros, out_features=out_features, in_features=in_features,
        group_size=group_size, packing=packing,
    )
    x = np.asarray(x)
    lead = x.shape[:-1]
    activation = _to_f32(x, x_dtype).reshape(-1, in_features)
    output = activation @ weight.T                                                   # :95
    if bias is not None:
        output = output + _to_f32(np.asarray(bias), bias_dtype)                       # :96-97
    output = output.astype(np.float32).reshape(*lead, out_features)
    return output if return_f32 else _from_f32(output, x_dtype)                      # :98


def lpu_functional_linear(
    x: np.ndarray, qweight, scales, zeros, bias, *, out_features: int, in_features: int,
    group_size: int = 64, x_dtype: str = "fp16", bias_dtype: str = "bf16",
) -> np.ndarray:
    """backends.py:101-150: K-streaming emulation, fp32 accumulate per group."""
    groups = in_features // group_size
    codes = unpack_int4(qweight, PackingFormat.CANONICAL).reshape(out_features, in_features)
    zero_values = unpack_int4(zeros, PackingFormat.CANONICAL, elements=out_features * groups).reshape(
        out_features, groups)
    x = np.asarray(x)
    lead = x.shape[:-1]
    activation = _to_f32(x, x_dtype).reshape(-1, in_features)
    accumulator = np.zeros((activation.shape[0], out_features), dtype=np.float32)
    scales32 = np.asarray(scales).astype(np.float32)
    for group in range(groups):                                                      # :139-146
        start, stop = group * group_size, (group + 1) * group_size
        b_tile = codes[:, start:stop].astype(np.float32) - zero_values[:, group].astype(np.float32)[:, None]
        b_tile = b_tile * scales32[:, group][:, None]
        accumulator += activation[:, start:stop] @ b_tile.T
    if bias is not None:
        accumulator += _to_f32(np.asarray(bias), bias_dtype)
    return _from_f32(accumulator.reshape(*lead, out_features), x_dtype)


def tensor_metrics(reference: np.ndarray, candidate: np.ndarray) -> dict:
    """validation.py:112-134 (max_abs, mean_abs, rmse, mean_relative, cosine)."""
    ref = np.asarray(reference, dtype=np.float32).reshape(-1)
    got = np.asarray(candidate, dtype=np.float32).reshape(-1)
    if ref.shape != got.shape:
        raise ValueError(f"shape mismatch: reference={ref.shape}, candidate={got.shape}")
    if ref.size == 0:
        raise ValueError("cannot compare empty tensors")
    difference = np.abs(ref - got)
    relative = difference / np.maximum(np.abs(ref), np.float32(1e-6))
    ref_norm = float(np.linalg.norm(ref.astype(np.float64)))
    got_norm = float(np.linalg.norm(got.astype(np.float64)))
    denominator = ref_norm * got_norm
    if denominator == 0:
        cosine = 1.0 if np.array_equal(ref, got) else 0.0
    else:
        cosine = float(np.dot(ref.astype(np.float64), got.astype(np.float64)) / denominator)
    return {
        "max_abs": float(difference.max()),
        "mean_abs": float(difference.mean()),
        "rmse": float(np.sqrt(np.mean((ref.astype(np.float64) - got) ** 2))),
        "mean_relative": float(relative.mean()),
        "cosine": cosine,
        "normwise_relative": float(difference.max() / max(float(np.abs(ref).max()), 1e-30)),
    }


# ---------------------------------------------------------------------------
# Seeded synthetic workloads (the shapes and recipes of the benchmark configs)
# ---------------------------------------------------------------------------

BASE_SEED = 20260831

QWEN2_SHAPES = {            # name: (out_features N, in_features K)
    "q_proj": (1536, 1536),
    "k_proj": (256, 1536),
    "v_proj": (256, 1536),
    "o_proj": (1536, 1536),
    "gate_proj": (8960, 1536),
    "up_proj": (8960, 1536),
    "down_proj": (1536, 8960),
}


def symmetric_weights(out_features: int, in_features: int, seed: int):
    """fp32 N(0, 0.02) weights, symmetric RTN W4G64, zeros all 0."""
    rng = np.random.default_rng(seed)
    weight = (rng.standard_normal((out_features, in_features), dtype=np.float32) * np.float32(0.02))
    qweight, scales = quantize_symmetric_rtn(weight, group_size=64)
    zeros = np.zeros(((out_features * (in_features // 64) + 1) // 2, 1), dtype=np.uint8)
    return qweight, scales, zeros


def asymmetric_weights(out_features: int, in_features: int, seed: int):
    """AWQ-style direct draws: u ~ U{0..15}, z ~ U{4..11}, log-normal scales
    (mu = ln 0.003, sigma = 0.5); stored as signed u-8 / z-8."""
    rng = np.random.default_rng(seed)
    groups = in_features // 64
    codes = rng.integers(0, 16, size=(out_features, in_features), dtype=np.int16) - 8
    zeros_u = rng.integers(4, 12, size=(out_features * groups,), dtype=np.int16)
    scales = np.exp(rng.normal(np.log(0.003), 0.5, size=(out_features, groups))).astype(np.float16)
    signed_zeros = (zeros_u - 8).astype(np.int8)
    if signed_zeros.size % 2:
        signed_zeros = np.concatenate((signed_zeros, np.zeros(1, dtype=np.int8)))
    return (pack_int4(codes.astype(np.int8)).reshape(-1, 1), scales,
            pack_int4(signed_zeros).reshape(-1, 1))


def awq_folded_weights(out_features: int, in_features: int, seed: int):
    """W = N(0, 0.02) * a[k], a ~ U[0.5, 2] (input-channel AWQ vector folded in
    before packing), asymmetric RTN W4G64 (quantization.py:114-162)."""
    rng = np.random.default_rng(seed)
    weight = rng.standard_normal((out_features, in_features), dtype=np.float32) * np.float32(0.02)
    awq = rng.uniform(0.5, 2.0, size=(in_features,)).astype(np.float32)
    return quantize_asymmetric_rtn(weight * awq[None, :], group_size=64)


def activations(rows: int, in_features: int, seed: int, dtype: str = "fp16", outliers: bool = False):
    """x ~ N(0, 1) in ``dtype``; with ``outliers`` 1 % of channels are x20."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, in_features), dtype=np.float32)
    if outliers:
        channels = rng.choice(in_features, size=max(1, in_features // 100), replace=False)
        x[:, channels] *= np.float32(20.0)
    return _from_f32(x, dtype)


# ---------------------------------------------------------------------------
# C restatement through ctypes
# ---------------------------------------------------------------------------

class COracle:
    """ctypes view of ``oracle/_build/libw4g64_oracle.so``."""

    def __init__(self, path: Path | str = C_LIBRARY) -> None:
        if not Path(path).exists():
            raise FileNotFoundError(f"C oracle not built: {path} (run `make -C oracle`)")
        lib = ctypes.CDLL(str(path))
        i64, p = ctypes.c_int64, ctypes.c_void_p
        lib.o_pack_int4.argtypes = [p, i64, ctypes.c_int, p]
        lib.o_unpack_int4.argtypes = [p, i64, ctypes.c_int, i64, p]
        lib.o_dequantize_groupwise.argtypes = [p, i64, p, p, i64, i64, i64, i64, ctypes.c_int, p]
        lib.o_quantize_symmetric_rtn.argtypes = [p, i64, i64, i64, ctypes.c_int, p, p]
        lib.o_quantize_asymmetric_rtn.argtypes = [p, i64, i64, i64, p, ctypes.c_int, p, p, p]
        lib.o_linear_f32.argtypes = [p, i64, p, i64, i64, p, p]
        lib.o_linear_f32.restype = None
        for name in ("o_f32_to_f16_array", "o_f32_to_bf16_array", "o_f16_to_f32_array"):
            getattr(lib, name).argtypes = [p, i64, p]
            getattr(lib, name).restype = None
        self.lib = lib

    @staticmethod
    def _ptr(a: np.ndarray | None):
        return None if a is None else a.ctypes.data_as(ctypes.c_void_p)

    @staticmethod
    def _packing(packing) -> int:
        return 1 if PackingFormat(packing) is PackingFormat.LEGACY_SIGNED_ADD else 0

    def pack_int4(self, codes, packing=PackingFormat.CANONICAL) -> np.ndarray:
        codes = np.ascontiguousarray(np.asarray(codes).reshape(-1), dtype=np.int8)
        out = np.zeros(codes.size // 2, dtype=np.uint8)
        if self.lib.o_pack_int4(self._ptr(codes), codes.size, self._packing(packing), self._ptr(out)):
            raise ValueError("invalid INT4 codes")
        return out

    def unpack_int4(self, packed, packing=PackingFormat.CANONICAL, elements=None) -> np.ndarray:
        packed = np.ascontiguousarray(np.asarray(packed).reshape(-1), dtype=np.uint8)
        count = packed.size * 2 if elements is None else elements
        out = np.zeros(max(count, 0), dtype=np.int8)
        if count < 0 or self.lib.o_unpack_int4(self._ptr(packed), packed.size, self._packing(packing),
                                               count, self._ptr(out)):
            raise ValueError("invalid element count")
        return out

    def dequantize_groupwise(self, qweight, scales, zeros, out_features, in_features, group_size=64,
                             packing=PackingFormat.CANONICAL) -> np.ndarray:
        qweight = np.ascontiguousarray(np.asarray(qweight).reshape(-1), dtype=np.uint8)
        scales = np.ascontiguousarray(np.asarray(scales, dtype=np.float16)).view(np.uint16)
        zeros_arr = None if zeros is None else np.ascontiguousarray(np.asarray(zeros).reshape(-1), dtype=np.uint8)
        out = np.zeros((out_features, in_features), dtype=np.float32)
        rc = self.lib.o_dequantize_groupwise(
            self._ptr(qweight), qweight.size, self._ptr(scales), self._ptr(zeros_arr),
            0 if zeros_arr is None else zeros_arr.size, out_features, in_features, group_size,
            self._packing(packing), self._ptr(out))
        if rc:
            raise ValueError("invalid dequantization arguments")
        return out

    def quantize_symmetric_rtn(self, weight, group_size=64, packing=PackingFormat.CANONICAL):
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        n, k = weight.shape
        q = np.zeros((n * k // 2, 1), dtype=np.uint8)
        s = np.zeros((n, k // group_size), dtype=np.uint16)
        if self.lib.o_quantize_symmetric_rtn(self._ptr(weight), n, k, group_size, self._packing(packing),
                                             self._ptr(q), self._ptr(s)):
            raise ValueError("invalid quantization arguments")
        return q, s.view(np.float16)

    def quantize_asymmetric_rtn(self, weight, group_size=64, clip_max=None, packing=PackingFormat.CANONICAL):
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        n, k = weight.shape
        g = k // group_size
        q = np.zeros((n * k // 2, 1), dtype=np.uint8)
        s = np.zeros((n, g), dtype=np.uint16)
        z = np.zeros(((n * g + 1) // 2, 1), dtype=np.uint8)
        clip = None if clip_max is None else np.ascontiguousarray(clip_max, dtype=np.float32)
        if self.lib.o_quantize_asymmetric_rtn(self._ptr(weight), n, k, group_size, self._ptr(clip),
                                              self._packing(packing), self._ptr(q), self._ptr(s), self._ptr(z)):
            raise ValueError("invalid quantization arguments")
        return q, s.view(np.float16), z

    def linear_f32(self, x32: np.ndarray, w32: np.ndarray, bias32: np.ndarray | None = None) -> np.ndarray:
        x32 = np.ascontiguousarray(x32, dtype=np.float32)
        w32 = np.ascontiguousarray(w32, dtype=np.float32)
        rows, k = x32.reshape(-1, x32.shape[-1]).shape
        n = w32.shape[0]
        y = np.zeros((rows, n), dtype=np.float32)
        b = None if bias32 is None else np.ascontiguousarray(bias32, dtype=np.float32)
        self.lib.o_linear_f32(self._ptr(x32), rows, self._ptr(w32), n, k, self._ptr(b), self._ptr(y))
        return y

    def f32_to_f16_bits(self, values) -> np.ndarray:
        values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        out = np.zeros(values.size, dtype=np.uint16)
        self.lib.o_f32_to_f16_array(self._ptr(values), values.size, self._ptr(out))
        return out

    def f32_to_bf16_bits(self, values) -> np.ndarray:
        values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        out = np.zeros(values.size, dtype=np.uint16)
        self.lib.o_f32_to_bf16_array(self._ptr(values), values.size, self._ptr(out))
        return out

    def f16_bits_to_f32(self, bits) -> np.ndarray:
        bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
        out = np.zeros(bits.size, dtype=np.float32)
        self.lib.o_f16_to_f32_array(self._ptr(bits), bits.size, self._ptr(out))
        return out


def build_c_oracle() -> Path:
    """Compile the C oracle with its Makefile (checker build, not the product)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True, env=dict(os.environ))
    return C_LIBRARY


# ---------------------------------------------------------------------------
# torch CPU restatement of the reference's "torch" backend, used as the CPU
# baseline (same library and arithmetic as the reference path).
# ---------------------------------------------------------------------------

def reference_linear_torch(x, qweight, scales, zeros, bias, *, out_features: int, in_features: int,
                           group_size: int = 64, return_f32: bool = False):
    """backends.py:73-98 over quantization.py:53-84 / :221-258, canonical
    packing, with torch tensors on any device: dequantize the whole weight to fp32,
    fp32 matmul, fp32 bias, cast to ``x.dtype`` (or kept in fp32 with
    ``return_f32``, for error measurements)."""
    import torch

    groups = in_features // group_size

    def signed_nibbles(packed, count):
        byte = packed.reshape(-1).to(torch.uint8)
        low = (byte & 0x0F).to(torch.int16)
        high = (byte >> 4).to(torch.int16)
        out = torch.empty(byte.numel() * 2, dtype=torch.int8, device=byte.device)
        out[0::2] = torch.where(low >= 8, low - 16, low).to(torch.int8)
        out[1::2] = torch.where(high >= 8, high - 16, high).to(torch.int8)
        return out[:count]

    codes = signed_nibbles(qweight, out_features * in_features).reshape(out_features, in_features)
    zero_values = signed_nibbles(zeros, out_features * groups).reshape(out_features, groups)
    expanded_scales = scales.to(torch.float32).repeat_interleave(group_size, dim=1)
    expanded_zeros = zero_values.to(torch.float32).repeat_interleave(group_size, dim=1)
    weight = (codes.to(torch.float32) - expanded_zeros) * expanded_scales
    output = x.reshape(-1, in_features).to(torch.float32) @ weight.t()
    if bias is not None:
        output = output + bias.to(torch.float32)
    output = output.reshape(*x.shape[:-1], out_features)
    return output if return_f32 else output.to(x.dtype)
