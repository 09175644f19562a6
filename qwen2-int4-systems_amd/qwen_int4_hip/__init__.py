"""MI355X (gfx950) W4G64 INT4 linear backend for Qwen2 -- HIP kernels behind
the reference's explicit backend selection (src/qwen_int4/backends.py,
src/qwen_int4/linear.py)."""

from .backends import (
    SUPPORTED_BACKENDS,
    hip_w4g64_linear,
    lpu_w4g64_linear,
    torch_w4g64_linear,
    validate_canonical_w4g64_inputs,
)
from .kernels import (
    dequantize_canonical_w4g64_hip,
    hip_available,
    linear_canonical_w4g64_hip,
    linear_kernel_name,
    unpack_canonical_signed_int4_hip,
)
from .linear import QuantLinear
from .quantization import (
    PackingFormat,
    dequantize_groupwise,
    pack_int4,
    quantize_asymmetric_rtn,
    quantize_symmetric_rtn,
    unpack_int4,
)

__all__ = [
    "PackingFormat",
    "QuantLinear",
    "dequantize_groupwise",
    "pack_int4",
    "quantize_asymmetric_rtn",
    "quantize_symmetric_rtn",
    "unpack_int4",
    "SUPPORTED_BACKENDS",
    "dequantize_canonical_w4g64_hip",
    "hip_available",
    "hip_w4g64_linear",
    "lpu_w4g64_linear",
    "torch_w4g64_linear",
    "linear_canonical_w4g64_hip",
    "linear_kernel_name",
    "unpack_canonical_signed_int4_hip",
    "validate_canonical_w4g64_inputs",
]
