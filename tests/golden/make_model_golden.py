"""Write golden logits and greedy tokens of the reference's own Qwen2 model.

The model composition around the W4G64 linears (RMSNorm cast order, rotary
embedding, GQA, masking, the fp32 SwiGLU, the tied bf16 head, cached
generation) is only pinned by running the reference itself, so this script
imports the reference package from /root/reference/src (src/qwen_int4/
model.py:17-245, generation.py:10-115) IN THIS CONTAINER ONLY, on the CPU,
with its torch backend (backends.py:73-98), CANONICAL packing and group 64.
The outputs are data: seeded weights (safetensors) plus prompts, logits and
tokens (safetensors + JSON) under tests/golden/.  Nothing of the reference
travels with them; tests load only these files.

Model: a Qwen2-shaped toy with head_dim 128 and GQA 3:1 (hidden 384 = 3 query
heads x 128, as the reference's attention requires, 1 key/value head, SwiGLU
512, 2 layers, vocab 512, RMSNorm eps 1e-6, rope theta 1e6).  Linears are
N(0, 0.02) weights quantized by the reference's own RTN functions: symmetric (codes [-7, 7], zero bytes 0) in
model "sym" and asymmetric (codes [0, 15] with per-group zero points) in
model "asym".  Norm weights are 1 + N(0, 0.1) in bf16 so that the weight
multiply is pinned; embeddings and biases N(0, 0.02).

Cases per model:
  * "single": one unpadded 24-token prompt; prompt logits, then 8 cached
    greedy steps (tokens and each step's logits);
  * "pair": two unpadded 16-token prompts (batch 2), same records;
  * "padded": a left-padded batch of two (valid lengths 11 and 16) through
    the attention-mask path, same records.
Prompts are drawn from a seeded generator; a prompt is kept only when every
greedy choice beats the runner-up by at least MIN_MARGIN (logit units), so
that a correct implementation must reproduce the tokens exactly.

Run from the repository root:  python tests/golden/make_model_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path
from types import SimpleNamespace

import torch
from safetensors.torch import save_file

REFERENCE_SRC = Path("/root/reference/src")
HERE = Path(__file__).resolve().parent
SEED = 20260831
STEPS = 8
MIN_MARGIN = 0.02

CONFIG = dict(hidden_size=384, num_attention_heads=3, num_key_value_heads=1, head_dim=128,
              intermediate_size=512, num_hidden_layers=2, vocab_size=512, rms_norm_eps=1e-6,
              rope_theta=1_000_000.0)


def build_reference_model(ref, asymmetric: bool, seed: int):
    from qwen_int4.linear import QuantLinear
    from qwen_int4.quantization import PackingFormat, quantize_asymmetric_rtn, quantize_symmetric_rtn

    config = SimpleNamespace(**CONFIG)
    model = ref.QwenInt4ForCausalLM(config, backend="torch", packing=PackingFormat.CANONICAL, group_size=64)
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        emb = model.model.embed_tokens.weight
        emb.copy_((torch.randn(emb.shape, generator=gen) * 0.02).to(emb.dtype))
        for name, module in model.named_modules():
            if isinstance(module, QuantLinear):
                w = torch.randn((module.out_features, module.in_features), generator=gen) * 0.02
                if asymmetric:
                    q, s, z = quantize_asymmetric_rtn(w, group_size=64, packing=PackingFormat.CANONICAL)
                    module.zeros.copy_(z)
                else:
                    q, s = quantize_symmetric_rtn(w, group_size=64, packing=PackingFormat.CANONICAL)
                module.qweight.copy_(q)
                module.scales.copy_(s)
                if module.bias is not None:
                    module.bias.copy_((torch.randn(module.out_features, generator=gen) * 0.02).to(module.bias.dtype))
            elif type(module).__name__ == "RMSNorm":
                module.weight.copy_((1.0 + 0.1 * torch.randn(module.weight.shape, generator=gen)).to(torch.bfloat16))
    return model.eval()


def run_case(ref_generation, model, ids, mask):
    """Prompt logits, then STEPS cached greedy steps (generation.py:25-68)."""
    state = ref_generation.CachedGenerationState.prefill(model, ids, mask)
    prompt_logits = state.logits.clone()
    step_logits, margins = [], []
    tokens = []
    for _ in range(STEPS):
        last = state.logits[:, -1].float()
        top2 = last.topk(2, dim=-1).values
        margins.append(float((top2[:, 0] - top2[:, 1]).min()))
        token = state.next_greedy_tokens()
        tokens.append(token)
        step_logits.append(state.decode(token).clone())
    top2 = state.logits[:, -1].float().topk(2, dim=-1).values
    margins.append(float((top2[:, 0] - top2[:, 1]).min()))
    final = state.next_greedy_tokens()
    # the reference's own one-call greedy loop gives the same tokens
    want = ref_generation.greedy_generate_cached(model, ids, max_new_tokens=STEPS + 1, attention_mask=mask)
    got = torch.cat([ids] + tokens + [final], dim=1)
    assert torch.equal(want, got), "state-driven and one-call greedy generation disagree"
    return {
        "prompt_logits": prompt_logits,
        "step_logits": torch.cat(step_logits, dim=1),
        "generated": got,
        "margin": min(margins),
    }


def main() -> None:
    sys.path.insert(0, str(REFERENCE_SRC))
    import qwen_int4 as ref
    from qwen_int4 import generation as ref_generation

    torch.manual_seed(SEED)
    torch.set_num_threads(8)
    index = {"config": CONFIG, "steps": STEPS, "min_margin": MIN_MARGIN, "models": {}}
    for kind, asymmetric, seed in (("sym", False, SEED), ("asym", True, SEED + 1)):
        model = build_reference_model(ref, asymmetric, seed)
        state = {k: v.contiguous() for k, v in model.state_dict().items() if k != "lm_head.weight"}
        save_file(state, str(HERE / f"model_golden_{kind}_weights.safetensors"))
        records, meta = {}, {}
        prompt_gen = torch.Generator().manual_seed(seed + 100)
        cases = (("single", 1, 24, None), ("pair", 2, 16, None), ("padded", 2, 16, (5, 0)))
        with torch.inference_mode():
            for name, batch, length, pads in cases:
                for attempt in range(200):
                    ids = torch.randint(0, CONFIG["vocab_size"], (batch, length), generator=prompt_gen)
                    mask = None
                    if pads is not None:
                        mask = torch.ones((batch, length), dtype=torch.bool)
                        for row, pad in enumerate(pads):
                            mask[row, :pad] = False
                            ids[row, :pad] = 0
                    result = run_case(ref_generation, model, ids, mask)
                    if result["margin"] >= MIN_MARGIN:
                        break
                else:
                    raise RuntimeError(f"no prompt with margin {MIN_MARGIN} for {kind}/{name}")
                records[f"{name}.input_ids"] = ids
                if mask is not None:
                    records[f"{name}.attention_mask"] = mask.to(torch.uint8)
                records[f"{name}.prompt_logits"] = result["prompt_logits"]
                records[f"{name}.step_logits"] = result["step_logits"]
                records[f"{name}.generated"] = result["generated"]
                meta[name] = {"batch": batch, "length": length, "pads": list(pads) if pads else None,
                              "attempts": attempt + 1, "margin": result["margin"]}
                print(kind, name, meta[name], flush=True)
        save_file({k: v.contiguous() for k, v in records.items()}, str(HERE / f"model_golden_{kind}_cases.safetensors"))
        index["models"][kind] = {"asymmetric": asymmetric, "seed": seed, "cases": meta}
    (HERE / "model_golden.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
