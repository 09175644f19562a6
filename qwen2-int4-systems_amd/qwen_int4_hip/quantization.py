"""Packed INT4 storage-format identity (src/qwen_int4/quantization.py:17-20).

Only the canonical format reaches the HIP kernels; ``LEGACY_SIGNED_ADD`` is
kept so the enum values (and therefore module state and checkpoint
metadata) match the reference, and so the kernels can reject it by name.
"""

from __future__ import annotations

from enum import Enum


class PackingFormat(str, Enum):
    # Canonical v1: byte = q[k] in low nibble | q[k+1] in high nibble.
    CANONICAL = "canonical"
    LEGACY_SIGNED_ADD = "legacy_signed_add"


# Format identity strings of the canonical W4G64 checkpoint metadata
# (src/qwen_int4/export.py:38-57; scripts/quantize_model.py:148-162).
CANONICAL_PACKING_METADATA = "canonical_low_nibble_k_even_high_nibble_k_odd"
WEIGHT_LAYOUT_METADATA = "row_major_[out_features,in_features]"
SCALE_LAYOUT_METADATA = "[out_features,in_features/group_size]"
