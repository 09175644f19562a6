"""The Qwen2 model against golden outputs of the reference's own model.

``tests/golden/make_model_golden.py`` ran the reference package
(src/qwen_int4/model.py:17-245, generation.py:10-115; torch backend, CANONICAL
packing, group 64) on a seeded head_dim-128 toy model and stored its weights,
prompt logits, the logits of 8 cached greedy steps and the greedy tokens.
These tests load those files only.

Gates (scripts/validate_phase_f_correctness_matrix.py:109-110 uses cosine
>= 0.9997 plus exact tokens; the model-level bar here is cosine >= 0.9999):
  * prompt logits and every step's logits at cosine >= 0.9999;
  * greedy tokens identical (every golden choice leads its runner-up by
    >= 0.02, i.e. >= 10 bf16 ulps at these logit magnitudes).

CPU: the model's glue around the oracle's restatement of the reference's
torch backend in every linear.  GPU: the HIP module path (growing
cache, left padding through the attention mask) and the serving path that the
end-to-end benchmark times (``FusedPrefill`` + graph-replayed
``FusedDecodeStep`` through ``StaticGreedyDecoder``).
"""

from __future__ import annotations

import copy
import json
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from safetensors.torch import load_file

from oracle import oracle as O
from qwen_int4_hip import QuantLinear
from qwen_int4_hip.generation import CachedGenerationState, StaticGreedyDecoder, greedy_generate_cached
from qwen_int4_hip.model import QwenInt4ForCausalLM

GOLDEN = Path(__file__).resolve().parent / "golden"
INDEX = json.loads((GOLDEN / "model_golden.json").read_text())
CONFIG = SimpleNamespace(**INDEX["config"])
STEPS = INDEX["steps"]
KINDS = ("sym", "asym")
CASES = ("single", "pair", "padded")


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.double().flatten(), b.double().flatten()
    return float(a @ b / (a.norm() * b.norm()))


def load_model(kind: str, device: str) -> QwenInt4ForCausalLM:
    model = QwenInt4ForCausalLM(CONFIG, packing="canonical", group_size=64)
    state = load_file(str(GOLDEN / f"model_golden_{kind}_weights.safetensors"))
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert missing == ["lm_head.weight"] and not unexpected  # tied to the embedding
    return model.to(device).eval()


def load_case(kind: str, case: str, device: str) -> dict:
    records = load_file(str(GOLDEN / f"model_golden_{kind}_cases.safetensors"))
    out = {k.split(".", 1)[1]: v.to(device) for k, v in records.items() if k.startswith(case + ".")}
    if "attention_mask" in out:
        out["attention_mask"] = out["attention_mask"].bool()
    return out


def with_oracle_linears(model):
    ref = copy.deepcopy(model)
    for module in ref.modules():
        if isinstance(module, QuantLinear):
            def forward(x, m=module):
                return O.reference_linear_torch(x, m.qweight, m.scales, m.zeros, m.bias, out_features=m.out_features,
                                                in_features=m.in_features)
            module.forward = forward
    return ref


def check_growing_cache(model, case: dict) -> None:
    """Prompt logits, 8 teacher-forced cached steps and free-running greedy
    tokens against the golden records (generation.py:25-68)."""
    ids, mask = case["input_ids"], case.get("attention_mask")
    want_tokens = case["generated"]
    length = ids.shape[1]
    state = CachedGenerationState.prefill(model, ids, mask)
    assert state.logits.shape == case["prompt_logits"].shape
    valid = (slice(None),) if mask is None else (mask,)
    assert cosine(state.logits[valid], case["prompt_logits"][valid]) >= 0.9999
    for t in range(STEPS):
        assert torch.equal(state.next_greedy_tokens(), want_tokens[:, length + t:length + t + 1])
        logits = state.decode(want_tokens[:, length + t:length + t + 1])
        assert cosine(logits, case["step_logits"][:, t:t + 1]) >= 0.9999, f"step {t}"
    assert torch.equal(state.next_greedy_tokens(), want_tokens[:, -1:])
    got = greedy_generate_cached(model, ids, max_new_tokens=STEPS + 1, attention_mask=mask)
    assert torch.equal(got, want_tokens)


def test_golden_records_are_consistent():
    assert INDEX["config"]["head_dim"] == 128 and INDEX["steps"] == STEPS
    for kind in KINDS:
        for case in CASES:
            rec = load_case(kind, case, "cpu")
            meta = INDEX["models"][kind]["cases"][case]
            b, t = meta["batch"], meta["length"]
            assert rec["input_ids"].shape == (b, t)
            assert rec["prompt_logits"].shape == (b, t, CONFIG.vocab_size)
            assert rec["step_logits"].shape == (b, STEPS, CONFIG.vocab_size)
            assert rec["generated"].shape == (b, t + STEPS + 1)
            assert torch.equal(rec["generated"][:, :t], rec["input_ids"])
            # each recorded greedy token is the argmax of the logits before it
            before = torch.cat((rec["prompt_logits"][:, -1:], rec["step_logits"]), dim=1)
            assert torch.equal(before.float().argmax(dim=-1), rec["generated"][:, t:])
            assert meta["margin"] >= INDEX["min_margin"]


@pytest.mark.parametrize("kind", KINDS)
def test_model_glue_with_oracle_linears_matches_golden(kind):
    """CPU: this package's module tree, RMSNorm, rotary, GQA, masking, fp32
    SwiGLU and tied head around the oracle's linears reproduce the
    reference model."""
    torch.set_num_threads(max(1, min(8, torch.get_num_threads())))
    model = with_oracle_linears(load_model(kind, "cpu"))
    with torch.inference_mode():
        for case in CASES:
            check_growing_cache(model, load_case(kind, case, "cpu"))


gpu = pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")


@pytest.mark.gpu
@gpu
@pytest.mark.parametrize("kind", KINDS)
def test_hip_module_path_matches_golden(kind):
    """The HIP linears in the module path (prompts of 24 and 32 rows run the
    MFMA GEMM, the 1- and 2-row steps the decode GEMV), with the growing
    cache and the left-padded batch."""
    model = load_model(kind, "cuda")
    with torch.inference_mode():
        for case in CASES:
            check_growing_cache(model, load_case(kind, case, "cuda"))


@pytest.mark.gpu
@gpu
@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("case", ["single", "pair"])
def test_fused_serving_path_matches_golden(kind, case):
    """FusedPrefill + graph-replayed FusedDecodeStep (the benchmarked path):
    prompt logits, the logits of every replayed step under teacher forcing,
    and free-running greedy tokens."""
    model = load_model(kind, "cuda")
    rec = load_case(kind, case, "cuda")
    ids, want_tokens = rec["input_ids"], rec["generated"]
    batch, length = ids.shape
    decoder = StaticGreedyDecoder(model, batch, 64, use_graph=True, fused=True)
    with torch.inference_mode():
        logits = decoder.prefill(ids)
        assert cosine(logits, rec["prompt_logits"]) >= 0.9999
        assert torch.equal(decoder.token, want_tokens[:, length:length + 1])
        for t in range(STEPS):
            step = decoder.step(want_tokens[:, length + t:length + t + 1]).clone()
            assert cosine(step, rec["step_logits"][:, t:t + 1]) >= 0.9999, f"step {t}"
            assert torch.equal(decoder.token, want_tokens[:, length + t + 1:length + t + 2]), f"step {t}"
        free = StaticGreedyDecoder(model, batch, 64, use_graph=True, fused=True).generate(ids, STEPS + 1)
    assert torch.equal(free, want_tokens)


def test_generation_state_selects_rejects_and_closes():
    """The cached-generation contract on the CPU (tests/test_kv_cache.py:
    94-133 of the reference): left padding only, request reorder/removal
    keeps the owned caches in step, duplicates are refused, and a closed
    state fails."""
    model = with_oracle_linears(load_model("sym", "cpu"))
    ids = load_case("sym", "pair", "cpu")["input_ids"]
    three = torch.cat((ids, ids[:1]), dim=0)
    with torch.inference_mode():
        with pytest.raises(ValueError, match="left-padded"):
            CachedGenerationState.prefill(model, ids[:1, :3], torch.tensor([[1, 1, 0]], dtype=torch.bool))
        with pytest.raises(ValueError, match="non-empty"):
            CachedGenerationState.prefill(model, ids[:1, :3], torch.zeros((1, 3), dtype=torch.bool))
        with pytest.raises(ValueError, match="non_empty_sequence"):
            CachedGenerationState.prefill(model, ids[:, :0])
        state = CachedGenerationState.prefill(model, three)
        want_rows = [state.logits[2].clone(), state.logits[0].clone()]
        state.select_requests([2, 0])
        assert torch.equal(state.generated_ids, three[[2, 0]])
        assert all(torch.equal(a, b) for a, b in zip(state.logits, want_rows))
        assert state.past_key_values[0][0].shape[0] == 2 and state.attention_mask.shape == (2, ids.shape[1])
        with pytest.raises(ValueError, match="beam-cache"):
            state.select_requests([0, 0])
        with pytest.raises(IndexError):
            state.select_requests([2])
        with pytest.raises(ValueError, match="next_tokens"):
            state.decode(torch.zeros((3, 1), dtype=torch.long))
        step = state.decode(state.next_greedy_tokens())
        assert step.shape == (2, 1, CONFIG.vocab_size) and state.generated_ids.shape == (2, ids.shape[1] + 1)
        # rows 2 and 0 hold the same prompt: they decode identically
        assert torch.equal(step[0], step[1])
        state.close()
        assert state.past_key_values == () and not state.active
        with pytest.raises(RuntimeError, match="closed"):
            state.next_greedy_tokens()
        with pytest.raises(ValueError, match="non-negative"):
            greedy_generate_cached(model, ids, max_new_tokens=-1)
