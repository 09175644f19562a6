"""Packed W4G64 checkpoints: metadata contracts, strict loading, export.

Restates the reference's checkpoint contract so that its RTN-v4 and AWQ-v6
safetensors files load drop-in into ``QwenInt4ForCausalLM``:

  * metadata of the symmetric RTN export (scripts/quantize_model.py:148-162)
    and of the canonical asymmetric AWQ export (src/qwen_int4/export.py:38-57);
  * ``load_quantized_checkpoint`` (the contract of src/qwen_int4/
    checkpoint.py:51-118): the quantized tensors must match the model's
    buffers name for name and shape for shape, AWQ files also carry their
    transformed norms and v_proj bias, and non-zero zero points require an
    asymmetric contract, with the reference's error messages.  Everything is
    checked from the file header before any tensor is read, and the tensors
    are then streamed one at a time onto the device of the model's buffers
    (no host copy of the whole file); buffers that
    ``decode.fuse_projections`` turned into views of fused q|k|v and gate|up
    buffers are written through;
  * the frozen canonical AWQ v6 manifest and the checks on a v6 file's bytes
    and metadata before it loads (src/qwen_int4/artifact_contract.py:52-167,
    src/qwen_int4/checkpoint.py:121-140);
  * the base-model tensors the checkpoint does not carry (embedding, norms,
    q/k/v biases, tied LM head) -- src/qwen_int4/checkpoint.py:143-175.

Loading uses safetensors only (no pickle).
"""

from __future__ import annotations

import hashlib
import json
import re
from dataclasses import dataclass
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .quantization import (
    CANONICAL_PACKING_METADATA,
    SCALE_LAYOUT_METADATA,
    WEIGHT_LAYOUT_METADATA,
    PackingFormat,
)

# Pinned upstream identity of the reference's exports (src/qwen_int4/provenance.py:3-6).
HF_MODEL_ID = "Qwen/Qwen2-1.5B"
HF_MODEL_REVISION = "8a16abf2848eda07cc5253dec660bf1ce007ad7a"
HF_TOKENIZER_REVISION = HF_MODEL_REVISION

RTN_FORMAT_VERSION = "qwen-int4-v1"
AWQ_FORMAT_VERSION = "qwen-int4-awq-v1"
AWQ_TRANSFORMED_SUFFIXES = ("input_layernorm.weight", "post_attention_layernorm.weight", "v_proj.bias")
QUANTIZED_SUFFIXES = (".qweight", ".scales", ".zeros")
ZERO_LAYOUT_METADATA = "packed_row_major_[out_features,in_features/group_size]"
ASYMMETRIC_ZERO_POINT_CONTRACTS = {
    "canonical_signed_packed_per_group",
    "asymmetric_canonical_signed_packed_per_group",
}


@dataclass(frozen=True)
class LoadReport:
    loaded_keys: int
    skipped_non_quantized_keys: int


def is_quantized_key(name: str) -> bool:
    return name.endswith(QUANTIZED_SUFFIXES)


def canonical_rtn_metadata(*, group_size: int = 64, method: str = "symmetric_rtn",
                           source_model: str = HF_MODEL_ID, source_model_revision: str = HF_MODEL_REVISION,
                           tokenizer_revision: str = HF_TOKENIZER_REVISION) -> dict[str, str]:
    """Metadata of a symmetric RTN export (scripts/quantize_model.py:148-162)."""
    if method not in ("symmetric_rtn", "activation_weighted_clip_rtn"):
        raise ValueError(f"unknown RTN method {method!r}")
    return {
        "format_version": RTN_FORMAT_VERSION,
        "source_model": source_model,
        "source_model_revision": source_model_revision,
        "tokenizer_revision": tokenizer_revision,
        "quantization": method,
        "bits": "4",
        "activation_dtype": "bf16_or_fp16",
        "group_size": str(group_size),
        "code_range": "[-7,7]",
        "packing": CANONICAL_PACKING_METADATA,
        "weight_layout": WEIGHT_LAYOUT_METADATA,
        "scale_layout": SCALE_LAYOUT_METADATA,
        "zero_point": "none_symmetric",
    }


def canonical_awq_metadata(*, group_size: int = 128) -> dict[str, str]:
    """Metadata of a canonical asymmetric AWQ export (src/qwen_int4/export.py:38-57)."""
    if group_size not in {64, 128}:
        raise ValueError("canonical AWQ supports group sizes 64 and 128")
    return {
        "format_version": AWQ_FORMAT_VERSION,
        "source_model": HF_MODEL_ID,
        "source_model_revision": HF_MODEL_REVISION,
        "tokenizer_revision": HF_TOKENIZER_REVISION,
        "quantization": "canonical_awq_w4a16_asymmetric",
        "bits": "4",
        "activation_dtype": "bf16_or_fp16",
        "group_size": str(group_size),
        "code_range": "[-8,7]",
        "packing": CANONICAL_PACKING_METADATA,
        "weight_layout": WEIGHT_LAYOUT_METADATA,
        "scale_layout": SCALE_LAYOUT_METADATA,
        "zero_point": "canonical_signed_packed_per_group",
        "zero_layout": ZERO_LAYOUT_METADATA,
        "status": "awaiting_gpu_reference",
    }


def checkpoint_metadata(path: str | Path) -> dict[str, str]:
    with safe_open(str(path), framework="pt", device="cpu") as handle:
        return handle.metadata() or {}


def packing_from_checkpoint(path: str | Path) -> PackingFormat:
    """Canonical only when the file says so; an unversioned file is legacy
    (src/qwen_int4/checkpoint.py:36-41)."""
    if checkpoint_metadata(path).get("packing", "") == CANONICAL_PACKING_METADATA:
        return PackingFormat.CANONICAL
    return PackingFormat.LEGACY_SIGNED_ADD


def group_size_from_checkpoint(path: str | Path, default: int = 128) -> int:
    value = checkpoint_metadata(path).get("group_size")
    return default if value is None else int(value)


def _buffer_device(model: torch.nn.Module) -> torch.device:
    for name, tensor in model.state_dict().items():
        if is_quantized_key(name):
            return tensor.device
    return torch.device("cpu")


def _file_header(path: Path) -> tuple[dict[str, tuple[int, ...]], dict[str, str]]:
    """Tensor shapes and metadata from the safetensors header alone."""
    with safe_open(str(path), framework="pt", device="cpu") as handle:
        shapes = {key: tuple(handle.get_slice(key).get_shape()) for key in handle.keys()}
        return shapes, handle.metadata() or {}


def _key_set_problems(want: dict[str, tuple], have: dict[str, tuple]) -> tuple[list, list, dict]:
    """(missing, unexpected, shape mismatches) of a file's keys against a model's."""
    missing = sorted(set(want) - set(have))
    unexpected = sorted(set(have) - set(want))
    shapes = {key: (want[key], have[key]) for key in sorted(set(want) & set(have)) if want[key] != have[key]}
    return missing, unexpected, shapes


def load_quantized_checkpoint(model: torch.nn.Module, path: str | Path, *,
                              device: torch.device | str | None = None) -> LoadReport:
    """Load a W4G64 checkpoint's quantized tensors -- and, for the AWQ format,
    its transformed norms and v_proj biases -- into ``model``, strictly
    (the contract of src/qwen_int4/checkpoint.py:51-118).

    Three phases, so that a rejected file leaves the model untouched:
      1. the file's header alone (names and shapes, no tensor data) is
         checked against the model: the quantized key sets must be equal
         with equal shapes, and an AWQ file must carry exactly the model's
         transformed-state keys;
      2. unless the metadata names an asymmetric zero-point contract, every
         ``.zeros`` tensor of the file must be all zero;
      3. each tensor is read onto ``device`` (default: where the model's
         quantized buffers live) and copied into its buffer -- buffers that
         are views of fused projection buffers receive the data in place.
    Returns the count of loaded keys and of file keys left unused."""
    path = Path(path)
    if not path.is_file():
        raise FileNotFoundError(path)
    shapes, metadata = _file_header(path)
    targets = model.state_dict()
    want = {key: tuple(t.shape) for key, t in targets.items() if is_quantized_key(key)}
    have = {key: shape for key, shape in shapes.items() if is_quantized_key(key)}
    missing, unexpected, mismatched = _key_set_problems(want, have)
    if missing or unexpected or mismatched:
        raise RuntimeError(f"checkpoint contract mismatch:\n  missing={missing}\n  unexpected={unexpected}\n"
                           f"  shape_mismatches={mismatched}")
    keys = sorted(want)
    if metadata.get("format_version") == AWQ_FORMAT_VERSION:
        t_want = {key: tuple(t.shape) for key, t in targets.items() if key.endswith(AWQ_TRANSFORMED_SUFFIXES)}
        t_have = {key: shape for key, shape in shapes.items() if key.endswith(AWQ_TRANSFORMED_SUFFIXES)}
        t_missing, t_unexpected, t_shapes = _key_set_problems(t_want, t_have)
        if t_missing or t_unexpected:
            raise RuntimeError(f"AWQ transformed-state contract mismatch:\n  missing={t_missing}\n"
                               f"  unexpected={t_unexpected}")
        if t_shapes:
            # the reference loads these with load_state_dict, which rejects a
            # shape that differs (torch's message); copy_ would broadcast
            raise RuntimeError("Error(s) in loading state_dict:\n" + "\n".join(
                f"\tsize mismatch for {key}: copying a param with shape {torch.Size(have_shape)} from checkpoint, "
                f"the shape in current model is {torch.Size(want_shape)}."
                for key, (want_shape, have_shape) in t_shapes.items()))
        keys += sorted(t_want)
    target = torch.device(device) if device is not None else _buffer_device(model)
    with safe_open(str(path), framework="pt", device=str(target)) as handle:
        if metadata.get("zero_point", "") not in ASYMMETRIC_ZERO_POINT_CONTRACTS:
            nonzero = [key for key in keys if key.endswith(".zeros") and bool(handle.get_tensor(key).any())]
            if nonzero:
                raise RuntimeError("non-zero zero-points found without an asymmetric checkpoint contract: "
                                   + ", ".join(nonzero))
        with torch.no_grad():
            for key in keys:
                targets[key].copy_(handle.get_tensor(key))
    return LoadReport(len(keys), len(shapes) - len(keys))


# Non-quantized tensors every model needs from its base model (the checkpoint
# carries only the quantized linears and, for AWQ, the transformed norms and
# v_proj bias) -- src/qwen_int4/checkpoint.py:157-165.
_REQUIRED_BASE_KEYS = ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight")
_REQUIRED_BASE_SUFFIXES = ("layernorm.weight", "q_proj.bias", "k_proj.bias", "v_proj.bias")


def extract_non_quantized_state(base_model: torch.nn.Module, target_model: torch.nn.Module) -> dict[str, torch.Tensor]:
    """The base model's tensors that `target_model` holds outside its quantized
    buffers (embedding, norms, q/k/v biases, tied LM head), as host copies,
    matched by name and shape; fails if a required one is absent
    (src/qwen_int4/checkpoint.py:143-169)."""
    source = base_model.state_dict()
    wanted = [key for key in target_model.state_dict() if not is_quantized_key(key)]
    target_shapes = {key: tensor.shape for key, tensor in target_model.state_dict().items()}
    state = {key: source[key].detach().to("cpu").clone() for key in wanted
             if key in source and source[key].shape == target_shapes[key]}
    required = {key for key in wanted
                if key in _REQUIRED_BASE_KEYS or key.endswith(_REQUIRED_BASE_SUFFIXES)}
    missing = sorted(required - set(state))
    if missing:
        raise RuntimeError(f"HF base model is missing required non-quantized tensors: {missing}")
    return state


def load_non_quantized_state(model: torch.nn.Module, state: dict[str, torch.Tensor]) -> None:
    """Copy base-model tensors into `model` (src/qwen_int4/checkpoint.py:172-175)."""
    incompatible = model.load_state_dict(state, strict=False)
    if incompatible.unexpected_keys:
        raise RuntimeError(f"unexpected HF base keys: {sorted(incompatible.unexpected_keys)}")


def save_quantized_checkpoint(model: torch.nn.Module, path: str | Path, metadata: dict[str, str]) -> Path:
    """Write ``model``'s quantized tensors (plus, for the AWQ format, its
    transformed norms and v_proj biases) with ``metadata``; never overwrites."""
    path = Path(path)
    if path.exists():
        raise FileExistsError(f"refusing to overwrite {path}")
    awq = metadata.get("format_version") == AWQ_FORMAT_VERSION
    tensors = {
        key: value.detach().to("cpu").contiguous()
        for key, value in model.state_dict().items()
        if is_quantized_key(key) or (awq and key.endswith(AWQ_TRANSFORMED_SUFFIXES))
    }
    if not any(is_quantized_key(key) for key in tensors):
        raise ValueError("model has no quantized tensors")
    path.parent.mkdir(parents=True, exist_ok=True)
    save_file(tensors, str(path), metadata=dict(metadata))
    return path


def sha256_file(path: str | Path) -> str:
    """SHA-256 of a file, read in 1 MiB blocks (src/qwen_int4/artifact_contract.py:31-37)."""
    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        for block in iter(lambda: handle.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


AWQ_V6_ARTIFACT_ID = "qwen2-1.5b-w4g64-awq-canonical-v6"


@dataclass(frozen=True)
class CanonicalAWQV6Contract:
    """What the frozen v6 manifest pins about the checkpoint file."""
    manifest_path: Path
    checkpoint_sha256: str
    checkpoint_size_bytes: int
    group_size: int
    model_id: str
    model_revision: str
    tokenizer_revision: str


# (dotted manifest field, required value, message on mismatch): the frozen
# v6 manifest's fixed fields (src/qwen_int4/artifact_contract.py:60-101).
_V6_MANIFEST_FIXED = (
    ("schema_version", "qwen-int4-awq-artifact-manifest-v1", "unsupported canonical AWQ manifest schema"),
    ("artifact_id", AWQ_V6_ARTIFACT_ID, "manifest is not the canonical AWQ v6 artifact"),
    ("status", "frozen_phase_d_candidate", "canonical AWQ v6 manifest must remain frozen"),
    ("quantization_contract.format_version", AWQ_FORMAT_VERSION, "canonical AWQ v6 format version mismatch"),
    ("quantization_contract.bits", 4, "canonical AWQ v6 requires W4G64"),
    ("quantization_contract.group_size", 64, "canonical AWQ v6 requires W4G64"),
    ("quantization_contract.quantization", "canonical_awq_asymmetric",
     "canonical AWQ v6 requires asymmetric quantization"),
    ("quantization_contract.zero_point", "per-group asymmetric",
     "canonical AWQ v6 requires per-group asymmetric zero points"),
    ("quantization_contract.packing", "canonical signed INT4 packing",
     "canonical AWQ v6 requires canonical signed INT4 packing"),
    ("selection.selected_variant", "v6", "canonical AWQ v6 selection record mismatch"),
    ("selection.rejected_variant", "v7", "canonical AWQ v6 selection record mismatch"),
    ("selection.phase_e_eligibility", "correctness-only work; no performance claim is authorized by this manifest",
     "manifest must retain the Phase E correctness-only restriction"),
)


def _manifest_field(manifest: object, dotted: str) -> object:
    node = manifest
    parts = dotted.split(".")
    for depth, part in enumerate(parts):
        if not isinstance(node, dict):
            raise ValueError(f"manifest field {'.'.join(parts[:depth]) or 'root'!r} must be an object")
        node = node.get(part)
    return node


def _manifest_string(manifest: object, dotted: str) -> str:
    value = _manifest_field(manifest, dotted)
    if not isinstance(value, str) or not value:
        raise ValueError(f"manifest field {dotted!r} must be a non-empty string")
    return value


def load_canonical_awq_v6_contract(manifest_path: str | Path) -> CanonicalAWQV6Contract:
    """Read the frozen v6 manifest and reject any drift from it
    (src/qwen_int4/artifact_contract.py:52-111).  The manifest's evidence
    records (the reference repository's own result files) are not checked."""
    path = Path(manifest_path)
    try:
        manifest = json.loads(path.read_text(encoding="utf-8"))
    except json.JSONDecodeError as error:
        raise ValueError(f"invalid manifest JSON: {path}") from error
    if not isinstance(manifest, dict):
        raise ValueError("manifest field 'root' must be an object")
    for field, value, message in _V6_MANIFEST_FIXED:
        got = _manifest_field(manifest, field)
        if got != value:
            raise ValueError(message)
    digest = _manifest_string(manifest, "artifact.sha256")
    if re.fullmatch(r"[0-9a-f]{64}", digest) is None:
        raise ValueError("artifact.sha256 must be a lowercase SHA-256 digest")
    size = _manifest_field(manifest, "artifact.size_bytes")
    if type(size) is not int or size <= 0:
        raise ValueError("artifact.size_bytes must be a positive integer")
    remote = _manifest_string(manifest, "artifact.remote_path")
    if not (remote.startswith("/") and remote.endswith("/model.safetensors")):
        raise ValueError("artifact.remote_path must be an absolute model.safetensors path")
    return CanonicalAWQV6Contract(
        manifest_path=path,
        checkpoint_sha256=digest,
        checkpoint_size_bytes=size,
        group_size=64,
        model_id=_manifest_string(manifest, "upstream.model_id"),
        model_revision=_manifest_string(manifest, "upstream.model_revision"),
        tokenizer_revision=_manifest_string(manifest, "upstream.tokenizer_revision"),
    )


def validate_canonical_awq_v6_checkpoint(path: str | Path, contract: CanonicalAWQV6Contract) -> dict[str, str]:
    """Fail closed on the v6 checkpoint's bytes and metadata before any load
    (src/qwen_int4/artifact_contract.py:140-167)."""
    path = Path(path)
    if not path.is_file():
        raise FileNotFoundError(path)
    if path.stat().st_size != contract.checkpoint_size_bytes:
        raise ValueError("checkpoint size does not match the frozen v6 manifest")
    if sha256_file(path) != contract.checkpoint_sha256:
        raise ValueError("checkpoint SHA-256 does not match the frozen v6 manifest")
    metadata = checkpoint_metadata(path)
    # the export's metadata (export.py:38-57) minus its free-form fields,
    # with the identity the manifest pins
    expected = canonical_awq_metadata(group_size=contract.group_size)
    del expected["activation_dtype"], expected["status"]
    expected.update(source_model=contract.model_id, source_model_revision=contract.model_revision,
                    tokenizer_revision=contract.tokenizer_revision)
    mismatch = {key: (value, metadata.get(key)) for key, value in expected.items() if metadata.get(key) != value}
    if mismatch:
        raise ValueError(f"checkpoint metadata does not satisfy canonical AWQ v6: {mismatch}")
    return metadata


def _layers_outside(model: torch.nn.Module, group_size: int) -> list[str]:
    """Quantized layers of ``model`` that are not canonical W4G``group_size``."""
    return [name for name, module in model.named_modules()
            if hasattr(module, "qweight") and not (getattr(module, "group_size", None) == group_size
                                                   and getattr(module, "packing", None) is PackingFormat.CANONICAL)]


def load_canonical_awq_v6_checkpoint(model: torch.nn.Module, path: str | Path, contract: CanonicalAWQV6Contract, *,
                                     device: torch.device | str | None = None) -> LoadReport:
    """The frozen v6 file into a W4G64 canonical model: the file's bytes and
    metadata against the manifest's contract first, then the model's layers,
    then the strict load (src/qwen_int4/checkpoint.py:121-140)."""
    validate_canonical_awq_v6_checkpoint(path, contract)
    outside = _layers_outside(model, contract.group_size)
    if outside:
        raise RuntimeError("model does not satisfy canonical AWQ v6 W4G64 packing: " + ", ".join(outside))
    return load_quantized_checkpoint(model, path, device=device)
