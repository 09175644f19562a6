"""Checkpoint contract: metadata, strict loading, export, v6 manifest checks.

Mirrors the reference's loader tests (tests/test_awq_export.py:19-96,
tests/test_phase_e_correctness.py:33-101) and pins the metadata and tensor
inventory against the reference's own records of its RTN-v4 export and AWQ-v6
manifest (fixtures under tests/golden/, made by make_checkpoint_fixtures.py).
All on the CPU: nothing here launches a kernel.
"""

import json
import re
from dataclasses import replace
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from safetensors.torch import save_file
from torch import nn

from qwen_int4_hip.checkpoint import (
    AWQ_FORMAT_VERSION,
    CanonicalAWQV6Contract,
    LoadReport,
    canonical_awq_metadata,
    canonical_rtn_metadata,
    checkpoint_metadata,
    extract_non_quantized_state,
    group_size_from_checkpoint,
    is_quantized_key,
    load_canonical_awq_v6_checkpoint,
    load_canonical_awq_v6_contract,
    load_non_quantized_state,
    load_quantized_checkpoint,
    packing_from_checkpoint,
    save_quantized_checkpoint,
    sha256_file,
    validate_canonical_awq_v6_checkpoint,
)
from qwen_int4_hip.decode import fuse_projections
from qwen_int4_hip.linear import QuantLinear
from qwen_int4_hip.model import QwenInt4ForCausalLM
from qwen_int4_hip.quantization import PackingFormat, pack_int4

GOLDEN = Path(__file__).resolve().parent / "golden"
RTN_V4 = json.loads((GOLDEN / "rtn_v4_contract.json").read_text())
V6_MANIFEST = GOLDEN / "awq_canonical_v6_manifest.json"
QWEN2_1_5B = dict(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2, head_dim=128,
                  intermediate_size=8960, vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1_000_000.0)


class ToyQuantModel(nn.Module):
    """The reference's toy: one norm and one W4 linear (tests/test_awq_export.py:27-33)."""

    def __init__(self, group_size: int = 64, in_features: int = 128, out_features: int = 4) -> None:
        super().__init__()
        self.input_layernorm = nn.LayerNorm(in_features, elementwise_affine=True, bias=False)
        self.proj = QuantLinear(in_features, out_features, group_size=group_size, packing=PackingFormat.CANONICAL)


def _fill(model: nn.Module, seed: int, *, zeros: bool = True) -> nn.Module:
    generator = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, tensor in model.state_dict().items():
            if tensor.dtype == torch.uint8 and (zeros or not name.endswith(".zeros")):
                tensor.copy_(torch.randint(0, 256, tensor.shape, generator=generator, dtype=torch.uint8))
            elif tensor.is_floating_point():
                tensor.copy_((torch.rand(tensor.shape, generator=generator) + 0.5).to(tensor.dtype))
    return model


def _assert_same_state(a: nn.Module, b: nn.Module, keys) -> None:
    sa, sb = a.state_dict(), b.state_dict()
    for key in keys:
        assert torch.equal(sa[key], sb[key]), key


# --- metadata ---------------------------------------------------------------

def test_rtn_metadata_matches_the_reference_v4_export_record():
    """The v4 file predates the revision fields; everything else must agree
    byte for byte with what the reference recorded of the file it wrote."""
    ours = canonical_rtn_metadata(group_size=64)
    recorded = RTN_V4["safetensors_metadata"]
    assert set(ours) - set(recorded) == {"source_model_revision", "tokenizer_revision"}
    assert {key: ours[key] for key in recorded} == recorded
    assert canonical_rtn_metadata(method="activation_weighted_clip_rtn")["quantization"] == "activation_weighted_clip_rtn"
    with pytest.raises(ValueError):
        canonical_rtn_metadata(method="gptq")


def test_awq_metadata_satisfies_the_frozen_v6_contract(tmp_path: Path):
    metadata = canonical_awq_metadata(group_size=64)
    assert metadata["format_version"] == AWQ_FORMAT_VERSION
    assert metadata["zero_point"] == "canonical_signed_packed_per_group"
    assert metadata["status"] == "awaiting_gpu_reference"
    assert canonical_awq_metadata()["group_size"] == "128"
    with pytest.raises(ValueError, match="group sizes"):
        canonical_awq_metadata(group_size=32)
    checkpoint, contract = _v6_checkpoint(tmp_path, metadata)
    assert validate_canonical_awq_v6_checkpoint(checkpoint, contract) == metadata


def test_packing_and_group_size_come_from_metadata(tmp_path: Path):
    canonical = tmp_path / "canonical.safetensors"
    legacy = tmp_path / "legacy.safetensors"
    save_file({"x": torch.zeros(1)}, str(canonical), metadata=canonical_rtn_metadata(group_size=64))
    save_file({"x": torch.zeros(1)}, str(legacy))
    assert packing_from_checkpoint(canonical) is PackingFormat.CANONICAL
    assert packing_from_checkpoint(legacy) is PackingFormat.LEGACY_SIGNED_ADD
    assert group_size_from_checkpoint(canonical) == 64
    assert group_size_from_checkpoint(legacy) == 128
    assert group_size_from_checkpoint(legacy, default=64) == 64
    assert checkpoint_metadata(legacy) == {}


def test_quantized_key_suffixes():
    assert is_quantized_key("model.layers.0.mlp.down_proj.qweight")
    assert is_quantized_key("a.scales") and is_quantized_key("a.zeros")
    assert not is_quantized_key("model.norm.weight") and not is_quantized_key("a.bias")


# --- model inventory against the reference's v4 record -----------------------

def test_model_quantized_tensors_match_the_reference_v4_inventory():
    config = SimpleNamespace(num_hidden_layers=28, **QWEN2_1_5B)
    with torch.device("meta"):
        model = QwenInt4ForCausalLM(config, packing="canonical", group_size=64)
    state = model.state_dict()
    quantized = {key: tuple(value.shape) for key, value in state.items() if is_quantized_key(key)}
    inventory = RTN_V4["tensor_inventory"]
    assert len(quantized) == inventory["total"] == 3 * RTN_V4["num_linear_layers"]
    for suffix in ("qweight", "scales", "zeros"):
        assert sum(key.endswith("." + suffix) for key in quantized) == inventory[suffix]
    for name, (out_features, in_features) in RTN_V4["linear_shapes"].items():
        groups = in_features // 64
        assert quantized[f"{name}.qweight"] == (out_features * in_features // 2, 1)
        assert quantized[f"{name}.scales"] == (out_features, groups)
        assert quantized[f"{name}.zeros"] == ((out_features * groups + 1) // 2, 1)
    # every v_proj has a bias, as the AWQ transformed state requires
    assert all(f"model.layers.{i}.self_attn.v_proj.bias" in state for i in range(28))


# --- strict loading ----------------------------------------------------------

def test_awq_round_trip_restores_quantized_and_transformed_state(tmp_path: Path):
    source = _fill(ToyQuantModel(), 10)
    source.input_layernorm.weight.data.fill_(0.625)
    path = save_quantized_checkpoint(source, tmp_path / "toy-awq" / "model.safetensors",
                                     canonical_awq_metadata(group_size=64))
    target = ToyQuantModel()
    report = load_quantized_checkpoint(target, path)
    assert report == LoadReport(loaded_keys=4, skipped_non_quantized_keys=0)
    _assert_same_state(source, target, ["proj.qweight", "proj.scales", "proj.zeros", "input_layernorm.weight"])
    assert torch.count_nonzero(target.proj.zeros).item() > 0
    with pytest.raises(FileExistsError):
        save_quantized_checkpoint(source, path, canonical_awq_metadata(group_size=64))


def test_rtn_round_trip_leaves_non_quantized_state_alone(tmp_path: Path):
    source = _fill(ToyQuantModel(), 11, zeros=False)
    path = save_quantized_checkpoint(source, tmp_path / "rtn.safetensors", canonical_rtn_metadata(group_size=64))
    target = ToyQuantModel()
    target.input_layernorm.weight.data.fill_(3.0)
    report = load_quantized_checkpoint(target, path)
    assert report.loaded_keys == 3
    _assert_same_state(source, target, ["proj.qweight", "proj.scales", "proj.zeros"])
    assert torch.all(target.input_layernorm.weight == 3.0)


def test_loader_counts_skipped_non_quantized_keys(tmp_path: Path):
    source = _fill(ToyQuantModel(), 12, zeros=False)
    tensors = {k: v for k, v in source.state_dict().items() if is_quantized_key(k)}
    tensors["lm_head.weight"] = torch.zeros(2, 2)
    path = tmp_path / "extra.safetensors"
    save_file(tensors, str(path), metadata=canonical_rtn_metadata(group_size=64))
    assert load_quantized_checkpoint(ToyQuantModel(), path) == LoadReport(3, 1)


def test_loader_rejects_a_tensor_shape_mismatch(tmp_path: Path):
    tensors = _fill(ToyQuantModel(), 13).state_dict()
    tensors["proj.qweight"] = tensors["proj.qweight"][:-1]
    path = tmp_path / "bad-shape.safetensors"
    save_file(dict(tensors), str(path), metadata=canonical_awq_metadata(group_size=64))
    with pytest.raises(RuntimeError, match="shape_mismatches"):
        load_quantized_checkpoint(ToyQuantModel(), path)


@pytest.mark.parametrize("edit,field", [("drop", "missing=\\['proj.zeros'\\]"),
                                        ("add", "unexpected=\\['other.scales'\\]")])
def test_loader_rejects_missing_and_unexpected_quantized_keys(tmp_path: Path, edit: str, field: str):
    tensors = {k: v for k, v in _fill(ToyQuantModel(), 14, zeros=False).state_dict().items() if is_quantized_key(k)}
    if edit == "drop":
        del tensors["proj.zeros"]
    else:
        tensors["other.scales"] = torch.zeros(1, 1, dtype=torch.float16)
    path = tmp_path / "bad-keys.safetensors"
    save_file(tensors, str(path), metadata=canonical_rtn_metadata(group_size=64))
    with pytest.raises(RuntimeError, match="checkpoint contract mismatch") as error:
        load_quantized_checkpoint(ToyQuantModel(), path)
    assert re.search(field, str(error.value))


def test_awq_loader_requires_the_transformed_state(tmp_path: Path):
    source = _fill(ToyQuantModel(), 15)
    tensors = {k: v for k, v in source.state_dict().items() if is_quantized_key(k)}
    path = tmp_path / "no-norm.safetensors"
    save_file(tensors, str(path), metadata=canonical_awq_metadata(group_size=64))
    with pytest.raises(RuntimeError, match="AWQ transformed-state contract mismatch"):
        load_quantized_checkpoint(ToyQuantModel(), path)


@pytest.mark.parametrize("norm_shape", [(1,), (64,)])
def test_awq_loader_rejects_a_transformed_tensor_shape_before_any_copy(tmp_path: Path, norm_shape):
    """A transformed norm of the wrong shape -- broadcastable ([1]) or not
    ([64]) -- is a size mismatch, as the reference's load_state_dict reports
    it, and the model is left untouched (quantized buffers included)."""
    tensors = dict(_fill(ToyQuantModel(), 18).state_dict())
    tensors["input_layernorm.weight"] = torch.full(norm_shape, 7.0)
    path = tmp_path / "bad-norm.safetensors"
    save_file(tensors, str(path), metadata=canonical_awq_metadata(group_size=64))
    target = _fill(ToyQuantModel(), 19)
    before = {k: v.clone() for k, v in target.state_dict().items()}
    with pytest.raises(RuntimeError, match="size mismatch for input_layernorm.weight"):
        load_quantized_checkpoint(target, path)
    for key, value in target.state_dict().items():
        assert torch.equal(value, before[key]), key


def test_nonzero_zero_points_need_an_asymmetric_contract(tmp_path: Path):
    source = _fill(ToyQuantModel(), 16)
    source.proj.zeros.copy_(pack_int4(torch.tensor([-7, 5], dtype=torch.int8), packing=PackingFormat.CANONICAL)
                            .reshape(-1, 1))
    path = save_quantized_checkpoint(source, tmp_path / "rtn-with-zeros.safetensors",
                                     canonical_rtn_metadata(group_size=64))
    with pytest.raises(RuntimeError, match="non-zero zero-points found without an asymmetric"):
        load_quantized_checkpoint(ToyQuantModel(), path)


def test_loader_rejects_a_missing_file(tmp_path: Path):
    with pytest.raises(FileNotFoundError):
        load_quantized_checkpoint(ToyQuantModel(), tmp_path / "absent.safetensors")


def test_export_refuses_a_model_without_quantized_tensors(tmp_path: Path):
    with pytest.raises(ValueError, match="no quantized tensors"):
        save_quantized_checkpoint(nn.Linear(2, 2), tmp_path / "x.safetensors", canonical_rtn_metadata())


def test_load_writes_through_fused_projection_views(tmp_path: Path):
    """A model whose q|k|v and gate|up were fused for decode still loads: the
    per-projection buffers are views into the fused buffers, and those views
    receive the file's bytes."""
    config = SimpleNamespace(num_hidden_layers=2, **dict(QWEN2_1_5B, hidden_size=128, num_attention_heads=2,
                                                         num_key_value_heads=1, head_dim=64, intermediate_size=256,
                                                         vocab_size=64))
    source = _fill(QwenInt4ForCausalLM(config, packing="canonical", group_size=64), 17)
    path = save_quantized_checkpoint(source, tmp_path / "awq.safetensors", canonical_awq_metadata(group_size=64))
    target = QwenInt4ForCausalLM(config, packing="canonical", group_size=64)
    fused = fuse_projections(target)
    report = load_quantized_checkpoint(target, path)
    expected_keys = [k for k in source.state_dict() if is_quantized_key(k) or k.endswith(
        ("input_layernorm.weight", "post_attention_layernorm.weight", "v_proj.bias"))]
    assert report.loaded_keys == len(expected_keys) == 2 * (7 * 3 + 3)
    _assert_same_state(source, target, expected_keys)
    for layer, buffers in zip(source.model.layers, fused):
        attn = layer.self_attn
        qkv = torch.cat([attn.q_proj.qweight, attn.k_proj.qweight, attn.v_proj.qweight])
        assert torch.equal(buffers["qkv"]["qweight"].reshape(qkv.shape), qkv)
        mlp = layer.mlp
        assert torch.equal(buffers["gate_up"]["scales"],
                           torch.cat([mlp.gate_proj.scales, mlp.up_proj.scales]))


# --- base-model state ---------------------------------------------------------

def test_non_quantized_state_is_taken_from_the_base_model():
    config = SimpleNamespace(num_hidden_layers=2, **dict(QWEN2_1_5B, hidden_size=128, num_attention_heads=2,
                                                         num_key_value_heads=1, head_dim=64, intermediate_size=256,
                                                         vocab_size=64))
    base = _fill(QwenInt4ForCausalLM(config, packing="canonical", group_size=64), 31)
    target = QwenInt4ForCausalLM(config, packing="canonical", group_size=64)
    state = extract_non_quantized_state(base, target)
    assert not any(is_quantized_key(k) for k in state)
    assert {"model.embed_tokens.weight", "model.norm.weight", "lm_head.weight",
            "model.layers.1.self_attn.k_proj.bias", "model.layers.0.post_attention_layernorm.weight"} <= set(state)
    assert all(v.device.type == "cpu" for v in state.values())
    load_non_quantized_state(target, state)
    _assert_same_state(base, target, list(state))
    assert not torch.equal(base.model.layers[0].mlp.up_proj.qweight, target.model.layers[0].mlp.up_proj.qweight)
    # a base model without a required tensor is rejected
    class NoNorm(nn.Module):
        def __init__(self):
            super().__init__()
            self.model = nn.Module()
            self.model.embed_tokens = nn.Embedding(64, 128)
    with pytest.raises(RuntimeError, match="missing required non-quantized tensors"):
        extract_non_quantized_state(NoNorm(), target)
    with pytest.raises(RuntimeError, match="unexpected HF base keys"):
        load_non_quantized_state(target, {"model.extra.weight": torch.zeros(1)})


# --- frozen v6 manifest ------------------------------------------------------

def _v6_checkpoint(tmp_path: Path, metadata: dict[str, str]) -> tuple[Path, CanonicalAWQV6Contract]:
    tmp_path.mkdir(parents=True, exist_ok=True)
    checkpoint = tmp_path / "model.safetensors"
    save_file({"placeholder": torch.zeros(1)}, str(checkpoint), metadata=metadata)
    manifest = json.loads(V6_MANIFEST.read_text())
    manifest["artifact"]["sha256"] = sha256_file(checkpoint)
    manifest["artifact"]["size_bytes"] = checkpoint.stat().st_size
    manifest_path = tmp_path / "manifest.json"
    manifest_path.write_text(json.dumps(manifest))
    return checkpoint, load_canonical_awq_v6_contract(manifest_path)


def test_frozen_v6_manifest_loads():
    contract = load_canonical_awq_v6_contract(V6_MANIFEST)
    assert contract.group_size == 64
    assert contract.checkpoint_size_bytes == 706537936
    assert contract.checkpoint_sha256 == "131a020962efc4e236b17fbd7da02f4aa9914e4c88a07b647e8cfe47dcaecab6"
    assert contract.model_id == "Qwen/Qwen2-1.5B"


@pytest.mark.parametrize("field,value,message", [
    ("selection.selected_variant", "v7", "selection"),
    ("status", "draft", "frozen"),
    ("quantization_contract.group_size", 128, "W4G64"),
    ("quantization_contract.zero_point", "none", "zero points"),
    ("artifact.sha256", "ABC", "lowercase SHA-256"),
    ("artifact.size_bytes", 0, "positive integer"),
    ("artifact.remote_path", "model.safetensors", "absolute"),
    ("upstream.model_id", "", "non-empty string"),
    ("upstream", [], "must be an object"),
])
def test_v6_manifest_rejects_drift(tmp_path: Path, field: str, value, message: str):
    manifest = json.loads(V6_MANIFEST.read_text())
    node = manifest
    *parents, leaf = field.split(".")
    for part in parents:
        node = node[part]
    node[leaf] = value
    path = tmp_path / "manifest.json"
    path.write_text(json.dumps(manifest))
    with pytest.raises(ValueError, match=message):
        load_canonical_awq_v6_contract(path)


def test_v6_manifest_rejects_invalid_json(tmp_path: Path):
    path = tmp_path / "manifest.json"
    path.write_text("{")
    with pytest.raises(ValueError, match="invalid manifest JSON"):
        load_canonical_awq_v6_contract(path)


def test_v6_checkpoint_bytes_and_metadata_fail_closed(tmp_path: Path):
    checkpoint, contract = _v6_checkpoint(tmp_path / "good", canonical_awq_metadata(group_size=64))
    assert validate_canonical_awq_v6_checkpoint(checkpoint, contract)["zero_point"] == \
        "canonical_signed_packed_per_group"
    bad = canonical_awq_metadata(group_size=64)
    bad["group_size"] = "128"
    bad_checkpoint, bad_contract = _v6_checkpoint(tmp_path / "bad", bad)
    with pytest.raises(ValueError, match="metadata"):
        validate_canonical_awq_v6_checkpoint(bad_checkpoint, bad_contract)
    with pytest.raises(ValueError, match="size"):
        validate_canonical_awq_v6_checkpoint(
            checkpoint, replace(contract, checkpoint_size_bytes=contract.checkpoint_size_bytes + 1))
    with pytest.raises(ValueError, match="SHA-256"):
        validate_canonical_awq_v6_checkpoint(
            checkpoint, replace(contract, checkpoint_sha256="0" * 64))
    with pytest.raises(FileNotFoundError):
        validate_canonical_awq_v6_checkpoint(tmp_path / "absent.safetensors", contract)


def test_v6_loader_checks_the_model_and_loads(tmp_path: Path):
    source = _fill(ToyQuantModel(), 18)
    path = save_quantized_checkpoint(source, tmp_path / "v6" / "model.safetensors",
                                     canonical_awq_metadata(group_size=64))
    manifest = json.loads(V6_MANIFEST.read_text())
    manifest["artifact"].update(sha256=sha256_file(path), size_bytes=path.stat().st_size)
    (tmp_path / "manifest.json").write_text(json.dumps(manifest))
    contract = load_canonical_awq_v6_contract(tmp_path / "manifest.json")
    with pytest.raises(RuntimeError, match="W4G64"):
        load_canonical_awq_v6_checkpoint(ToyQuantModel(group_size=128), path, contract)
    legacy = ToyQuantModel()
    legacy.proj.packing = PackingFormat.LEGACY_SIGNED_ADD
    with pytest.raises(RuntimeError, match="W4G64"):
        load_canonical_awq_v6_checkpoint(legacy, path, contract)
    target = ToyQuantModel()
    assert load_canonical_awq_v6_checkpoint(target, path, contract).loaded_keys == 4
    _assert_same_state(source, target, ["proj.qweight", "proj.scales", "proj.zeros", "input_layernorm.weight"])


@pytest.mark.gpu
def test_load_straight_to_the_gpu_matches_a_host_load(tmp_path: Path):
    """A file read straight into device buffers (of a model already fused for
    decode) gives the same model, and the same logits, as a host load moved
    to the GPU afterwards."""
    config = SimpleNamespace(num_hidden_layers=2, **QWEN2_1_5B)
    source = _fill(QwenInt4ForCausalLM(config, packing="canonical", group_size=64), 19)
    with torch.no_grad():
        for module in source.modules():
            if isinstance(module, QuantLinear):
                module.scales.mul_(0.01)  # keep activations in range over two layers
    path = save_quantized_checkpoint(source, tmp_path / "awq.safetensors", canonical_awq_metadata(group_size=64))
    host = QwenInt4ForCausalLM(config, packing="canonical", group_size=64)
    load_quantized_checkpoint(host, path)
    host.model.embed_tokens.weight.data.copy_(source.model.embed_tokens.weight)
    host = host.cuda()
    device = QwenInt4ForCausalLM(config, packing="canonical", group_size=64).cuda()
    device.model.embed_tokens.weight.data.copy_(source.model.embed_tokens.weight)
    fuse_projections(device)
    report = load_quantized_checkpoint(device, path)
    assert report.loaded_keys == 2 * (7 * 3 + 3)
    _assert_same_state(host, device, [k for k in host.state_dict() if is_quantized_key(k)])
    prompt = torch.randint(0, config.vocab_size, (1, 16), generator=torch.Generator().manual_seed(3)).cuda()
    with torch.inference_mode():
        assert torch.equal(host(prompt), device(prompt))


@pytest.mark.gpu
def test_exported_awq_checkpoint_round_trips_through_the_fused_decoder(tmp_path: Path):
    """A model quantized on the GPU (asymmetric codes, transformed norms and
    v_proj bias), exported, and loaded into a fresh model whose projections
    were fused for decode, generates exactly what the source model generates:
    same prompt logits, same greedy tokens through the graph-replayed step."""
    from qwen_int4_hip.generation import StaticGreedyDecoder
    from qwen_int4_hip.quantization import quantize_asymmetric_rtn

    config = SimpleNamespace(num_hidden_layers=2, **QWEN2_1_5B)
    gen = torch.Generator(device="cuda").manual_seed(23)
    source = QwenInt4ForCausalLM(config, packing="canonical", group_size=64).cuda()
    with torch.no_grad():
        source.model.embed_tokens.weight.copy_(torch.randn(source.model.embed_tokens.weight.shape, generator=gen,
                                                           device="cuda") * 0.02)
        for name, module in source.named_modules():
            if isinstance(module, QuantLinear):
                w = torch.randn((module.out_features, module.in_features), generator=gen, device="cuda") * 0.02
                q, s, z = quantize_asymmetric_rtn(w, group_size=64)
                module.qweight.copy_(q)
                module.scales.copy_(s)
                module.zeros.copy_(z)
                if module.bias is not None:
                    module.bias.copy_(torch.randn(module.out_features, generator=gen, device="cuda") * 0.02)
        for name, p in source.named_parameters():
            if name.endswith("layernorm.weight"):
                p.copy_(torch.rand(p.shape, generator=gen, device="cuda") + 0.5)
    path = save_quantized_checkpoint(source, tmp_path / "awq" / "model.safetensors", canonical_awq_metadata(group_size=64))
    target = QwenInt4ForCausalLM(config, packing="canonical", group_size=64).cuda()
    fuse_projections(target)
    # the reference's load order (src/qwen_int4/cli.py:92-95): base-model tensors, then the checkpoint
    load_non_quantized_state(target, extract_non_quantized_state(source, target))
    assert load_quantized_checkpoint(target, path).loaded_keys == 2 * (7 * 3 + 3)
    prompt = torch.randint(0, config.vocab_size, (1, 24), generator=torch.Generator().manual_seed(1)).cuda()
    a = StaticGreedyDecoder(source, 1, 48)
    b = StaticGreedyDecoder(target, 1, 48)
    with torch.inference_mode():
        la, lb = a.prefill(prompt), b.prefill(prompt)
        assert torch.equal(la, lb)
        for _ in range(8):
            assert torch.equal(a.step(), b.step())
            assert torch.equal(a.token, b.token)
