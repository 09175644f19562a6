"""HIP (gfx950) W4G64 primitives -- the counterparts of the reference's Triton
wrappers in src/qwen_int4/triton_kernels.py.

Each wrapper validates its tensors on the host, with the reference's
messages, before anything is launched, allocates its output with torch's
caching allocator and launches on torch's current stream through the C ABI
of ``libw4g64_hip.so``.  There is no other implementation behind them: a
missing library or GPU raises.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def hip_available() -> bool:
    """Return whether this process can run the HIP primitives
    (mirrors triton_available, triton_kernels.py:15-17)."""
    return _lib.library_built() and torch.cuda.is_available()


def _require_library() -> ctypes.CDLL:
    if not torch.cuda.is_available():
        raise RuntimeError("HIP W4G64 backend requires a ROCm GPU")
    return _lib.load()


def _stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _aligned(tensor: torch.Tensor, bytes_: int) -> torch.Tensor:
    """Return ``tensor`` or a contiguous copy whose storage starts on a
    ``bytes_`` boundary (views into a larger buffer may start anywhere)."""
    if tensor.data_ptr() % bytes_ == 0:
        return tensor
    copy = torch.empty_like(tensor, memory_format=torch.contiguous_format)
    copy.copy_(tensor)
    return copy


# ---------------------------------------------------------------------------
# Workspace: split-K partial sums of the decode GEMV and the GEMM (and the
# GEMM's bf16 planes of fp32 activations).  One buffer per (device, stream),
# grown on demand; every call writes what it reads, so its contents between
# calls do not matter.
# A HIP graph captured on a stream keeps the raw address of the buffer it was
# captured with, so a buffer is never freed once replaced: it moves to
# ``_retired`` and lives as long as the process.  Growing (or creating) a
# buffer while the stream is being captured is refused -- run the same call
# once before the capture, as the warm-up of every capture in this package
# does.
# ---------------------------------------------------------------------------

_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_retired: list[torch.Tensor] = []
_workspace_lock = threading.Lock()


def _grow_workspace(key, nbytes: int, device, capturing: bool) -> torch.Tensor:
    """The buffer for ``key`` with at least ``nbytes`` bytes (the dict logic
    of ``_workspace``; device-independent, so it is testable on the CPU)."""
    with _workspace_lock:
        buffer = _workspaces.get(key)
        if buffer is not None and buffer.numel() >= nbytes:
            return buffer
        if capturing:
            raise RuntimeError(
                f"W4G64 workspace of {nbytes} bytes is not allocated for this stream; HIP graph capture cannot "
                "allocate it -- run the same call on the capture stream once before capturing")
        size = max(nbytes, 2 * (0 if buffer is None else buffer.numel()), 1 << 20)
        if buffer is not None:
            _retired.append(buffer)  # a captured graph may still point at it
        buffer = torch.zeros(size, dtype=torch.uint8, device=device)
        _workspaces[key] = buffer
        return buffer


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes <= 0:
        return None
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(device)
    return _grow_workspace((index, stream.cuda_stream), nbytes, device, torch.cuda.is_current_stream_capturing())


# ---------------------------------------------------------------------------
# Primitives
# ---------------------------------------------------------------------------

def unpack_canonical_signed_int4_hip(packed: torch.Tensor, *, elements: int | None = None) -> torch.Tensor:
    """Decode canonical low-even/high-odd packed signed INT4 values on the GPU
    (triton_kernels.py:119-146).  ``elements`` may truncate the final byte."""
    lib = _require_library()
    if not packed.is_cuda:
        raise ValueError("HIP canonical INT4 unpack requires a GPU tensor")
    if packed.dtype != torch.uint8:
        raise ValueError("packed canonical INT4 values must have dtype torch.uint8")
    if not packed.is_contiguous():
        raise ValueError("packed canonical INT4 values must be contiguous")
    available = packed.numel() * 2
    count = available if elements is None else elements
    if not isinstance(count, int) or isinstance(count, bool) or count < 0 or count > available:
        raise ValueError(f"elements must be in [0, {available}], got {count!r}")
    output = torch.empty(count, device=packed.device, dtype=torch.int8)
    if count == 0:
        return output
    with torch.cuda.device(packed.device):
        _lib.check(lib.w4g64_unpack_canonical_int4(_ptr(packed), packed.numel(), _ptr(output), count,
                                                   _stream_handle(packed.device)))
    return output


def dequantize_canonical_w4g64_hip(
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    *,
    out_features: int,
    in_features: int,
) -> torch.Tensor:
    """Dequantize canonical W4G64 tensors to an fp32 GPU weight, bit-exact
    with (code - zero) * scale (triton_kernels.py:149-203)."""
    lib = _require_library()
    if not isinstance(out_features, int) or out_features <= 0:
        raise ValueError("out_features must be a positive integer")
    if not isinstance(in_features, int) or in_features <= 0 or in_features % 64:
        raise ValueError("canonical W4G64 dequantization requires in_features divisible by 64")
    for name, tensor, dtype in (
        ("qweight", qweight, torch.uint8),
        ("scales", scales, torch.float16),
        ("zeros", zeros, torch.uint8),
    ):
        if not tensor.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if tensor.dtype != dtype:
            raise ValueError(f"{name} must have dtype {dtype}")
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    groups_per_row = in_features // 64
    expected_qweight = out_features * in_features // 2
    expected_scales = out_features * groups_per_row
    expected_zeros = (expected_scales + 1) // 2
    if qweight.numel() != expected_qweight:
        raise ValueError(f"qweight must contain {expected_qweight} bytes, got {qweight.numel()}")
    if scales.numel() != expected_scales:
        raise ValueError(f"scales must contain {expected_scales} values, got {scales.numel()}")
    if zeros.numel() != expected_zeros:
        raise ValueError(f"zeros must contain {expected_zeros} bytes, got {zeros.numel()}")
    if not (qweight.device == scales.device == zeros.device):
        raise ValueError("qweight, scales and zeros must be on the same device")
    qweight = _aligned(qweight, 16)
    output = torch.empty((out_features, in_features), device=qweight.device, dtype=torch.float32)
    with torch.cuda.device(qweight.device):
        _lib.check(lib.w4g64_dequantize_canonical(_ptr(qweight), _ptr(scales), _ptr(zeros), _ptr(output),
                                                  out_features, in_features, _stream_handle(qweight.device)))
    return output


def linear_canonical_w4g64_hip(
    activations: torch.Tensor,
    qweight: torch.Tensor,
    scales: torch.Tensor,
    zeros: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused canonical W4G64 linear on MI355X (triton_kernels.py:206-268).

    ``activations`` is a contiguous rank-2 fp16/bf16/fp32 GPU tensor; the
    result has its dtype.  Rows <= 16 run the decode GEMV, more rows the MFMA
    GEMM; fp32 activations run natively (no torch fallback).
    """
    lib = _require_library()
    if activations.ndim != 2 or not activations.is_cuda or not activations.is_contiguous():
        raise ValueError("activations must be a contiguous rank-2 GPU tensor")
    if activations.dtype not in _DTYPE_CODE:
        raise ValueError("activations must have dtype torch.float16, torch.bfloat16, or torch.float32")
    rows, in_features = activations.shape
    if rows <= 0 or in_features <= 0 or in_features % 64:
        raise ValueError("activations require a positive W4G64-compatible feature dimension")
    for name, tensor, dtype in (
        ("qweight", qweight, torch.uint8),
        ("scales", scales, torch.float16),
        ("zeros", zeros, torch.uint8),
    ):
        if not tensor.is_cuda or not tensor.is_contiguous() or tensor.dtype != dtype:
            raise ValueError(f"{name} must be a contiguous GPU tensor with dtype {dtype}")
    groups_per_row = in_features // 64
    if scales.numel() % groups_per_row:
        raise ValueError("scales do not encode an integral number of output rows")
    out_features = scales.numel() // groups_per_row
    if out_features <= 0 or qweight.numel() != out_features * in_features // 2:
        raise ValueError("qweight size does not match the canonical W4G64 layout")
    if zeros.numel() != (out_features * groups_per_row + 1) // 2:
        raise ValueError("zeros size does not match the canonical W4G64 layout")
    bias_code = _lib.DTYPE_NONE
    if bias is not None:
        if not bias.is_cuda or not bias.is_contiguous() or bias.ndim != 1 or bias.numel() != out_features:
            raise ValueError("bias must be a contiguous GPU vector matching out_features")
        if bias.dtype not in _DTYPE_CODE:
            raise ValueError("bias must have dtype torch.float16, torch.bfloat16, or torch.float32")
        bias_code = _DTYPE_CODE[bias.dtype]
    device = activations.device
    tensors = (qweight, scales, zeros) + (() if bias is None else (bias,))
    if any(t.device != device for t in tensors):
        raise ValueError("all W4G64 inputs must be on the same device")
    activations = _aligned(activations, 16)
    qweight = _aligned(qweight, 16)
    x_code = _DTYPE_CODE[activations.dtype]
    output = torch.empty((rows, out_features), device=device, dtype=activations.dtype)
    with torch.cuda.device(device):
        ws_bytes = lib.w4g64_linear_workspace_bytes(rows, out_features, in_features, x_code)
        workspace = _workspace(device, ws_bytes)
        _lib.check(lib.w4g64_linear(
            _ptr(activations), x_code, _ptr(qweight), _ptr(scales), _ptr(zeros), _ptr(bias), bias_code,
            _ptr(output), rows, out_features, in_features, _ptr(workspace),
            0 if workspace is None else workspace.numel(), _stream_handle(device)))
    return output


def linear_kernel_name(rows: int, out_features: int, in_features: int, dtype: torch.dtype) -> str:
    """Name of the kernel the linear launches for this shape (for profiles)."""
    return _lib.load().w4g64_linear_kernel_name(rows, out_features, in_features, _DTYPE_CODE[dtype]).decode()
