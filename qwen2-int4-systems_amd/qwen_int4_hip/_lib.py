"""ctypes binding of ``libw4g64_hip.so`` (C ABI declared in include/w4g64.h and
include/qwen2_decode.h).

The library is loaded from the package directory only.  If it is missing the
HIP backend is unavailable and every entry point raises -- there is no other
implementation to fall back to.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().parent / "libw4g64_hip.so"

STATUS_OK = 0
STATUS_INVALID_VALUE = 1
STATUS_INVALID_DTYPE = 2
STATUS_WORKSPACE = 3
STATUS_UNSUPPORTED = 4
STATUS_HIP_ERROR = 5

DTYPE_NONE = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_F32 = 3
DTYPE_BF16_SWIGLU = 5  # activation form of w4g64_linear_swiglu (workspace / kernel-name queries)
DTYPE_BF16_PLANES = 6  # three bf16 planes of an fp32 activation (w4g64_linear, 1..16 rows, fp32 out)
DTYPE_BF16_GATE_UP = 7  # workspace / kernel-name queries of w4g64_linear_gate_up_planes


def dtype_f32_partials(parts: int) -> int:
    """Residual-delta code of ``parts`` fp32 partial sums (W4G64_DTYPE_F32_PARTIALS)."""
    if not 1 <= parts <= 255:
        raise ValueError(f"partial sum count must be in [1, 255], got {parts}")
    return 0x100 | parts


# (name, restype, argtypes) for every symbol include/*.h declares.
_p, _i64, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
SIGNATURES = {
    "w4g64_abi_version": (_int, []),
    "w4g64_last_error": (ctypes.c_char_p, []),
    "w4g64_unpack_canonical_int4": (_int, [_p, _i64, _p, _i64, _p]),
    "w4g64_dequantize_canonical": (_int, [_p, _p, _p, _p, _i64, _i64, _p]),
    "w4g64_linear_workspace_bytes": (_i64, [_i64, _i64, _i64, _int]),
    "w4g64_linear": (_int, [_p, _int, _p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "w4g64_linear_timed": (_int, [_p, _int, _p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _p, _i64, _p, _p, _p]),
    "w4g64_linear_kernel_name": (ctypes.c_char_p, [_i64, _i64, _i64, _int]),
    "w4g64_linear_partial_count": (_i64, [_i64, _i64, _i64, _int]),
    "w4g64_linear_partials": (_int, [_p, _int, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "w4g64_linear_static_scratch": (_int, [_p, _int, _p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _p]),
    "w4g64_static_scratch_bytes": (_i64, []),
    "w4g64_stream_probe": (_int, [_p, _i64, _p, _p]),
    "w4g64_linear_swiglu": (_int, [_p, _p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "w4g64_linear_gate_up_planes": (_int, [_p, _p, _p, _p, _p, _int, _p, _i64, _i64, _i64, _p, _i64, _p]),
    "w4g64_linear_rmsnorm": (_int, [_p, _p, _int, _p, ctypes.c_float, _p, _p, _p, _p, _p, _int, _p, _int, _i64, _i64,
                                    _i64, _p, _i64, _p]),
    "w4g64_linear_attention_merge": (_int, [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _int, _p, _i64, _i64, _p]),
    # include/qwen2_decode.h
    "qwen2_decode_prologue": (_int, [_p] * 8 + [ctypes.c_float, _p] + [_i64] * 4 + [_p]),
    "qwen2_add_rmsnorm": (_int, [_p, _p, _int, _p, ctypes.c_float, _p, _p, _i64, _i64, _p]),
    "qwen2_decode_attention_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qwen2_decode_attention": (_int, [_p] * 7 + [_i64] * 5 + [ctypes.c_float, _p, _i64, _p]),
    "qwen2_decode_attention_partials": (_int, [_p] * 6 + [_i64] * 5 + [ctypes.c_float, _p, _i64, _p]),
    "qwen2_prefill_attention_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qwen2_prefill_attention": (_int, [_p] * 6 + [_i64] * 6 + [ctypes.c_float, _p, _i64, _p]),
    "qwen2_silu_mul": (_int, [_p, _p, _i64, _i64, _p]),
    "qwen2_lm_head_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "qwen2_lm_head": (_int, [_p, _p, _p, _p, _i64, _i64, _i64, _p, _i64, _p]),
}

_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library_built() -> bool:
    return LIBRARY_PATH.exists()


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if not built."""
    global _library
    if _library is not None:
        return _library
    with _lock:
        if _library is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"HIP W4G64 library is not built ({LIBRARY_PATH}); run __graft_entry__.build()"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _library = lib
    return _library


def check(status: int) -> None:
    """Raise the reference's exception type for a non-zero C status."""
    if status == STATUS_OK:
        return
    message = (load().w4g64_last_error() or b"").decode("utf-8", "replace")
    if status == STATUS_INVALID_DTYPE:
        raise TypeError(message)
    if status in (STATUS_INVALID_VALUE, STATUS_WORKSPACE):
        raise ValueError(message)
    raise RuntimeError(message)
