"""Qwen2 decoder whose 196 linears are HIP W4G64 ``QuantLinear`` modules.

Restates src/qwen_int4/model.py:17-245 -- same module tree, parameter and
buffer names (so the reference's state dicts load unchanged), the same
RMSNorm cast order (:40-44), RoPE (:22-31, :76-77), grouped-query attention
(:90-91), masking rules (:94-120), fp32 SwiGLU feeding an fp32 down
projection (:133-136) and tied bf16 LM head (:217-218).

Attention scores are computed in fp32 (q k^T, softmax, p v) from the bf16
q/k/v -- the reference calls scaled_dot_product_attention on bf16 tensors;
fp32 is at least as accurate, and it keeps bf16 batched products with
transposed operands out of the path.

Two cache forms:
  * ``forward(..., past_key_values, use_cache)``: the reference's growing
    per-layer (key, value) tuples;
  * ``decode_static(...)``: a preallocated cache written at a device-side
    position, so one decode step has fixed shapes and can be captured once as
    a HIP graph and replayed per token (``generation.StaticGreedyDecoder``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .linear import QuantLinear
from .quantization import PackingFormat

PastKeyValue = tuple[torch.Tensor, torch.Tensor]
PastKeyValues = tuple[PastKeyValue, ...]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, theta: float) -> None:
        super().__init__()
        exponent = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
        self.register_buffer("inv_freq", 1.0 / (theta ** exponent), persistent=False)

    def forward(self, position_ids: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        angles = position_ids.to(torch.float32).unsqueeze(-1) * self.inv_freq
        angles = torch.cat((angles, angles), dim=-1)
        return angles.cos().to(dtype), angles.sin().to(dtype)


class RMSNorm(nn.Module):
    def __init__(self, hidden_size: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size, dtype=torch.bfloat16), requires_grad=False)
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x32 = x.to(torch.float32)
        normalized = x32 * torch.rsqrt(x32.square().mean(dim=-1, keepdim=True) + self.eps)
        return (normalized.to(x.dtype) * self.weight).to(x.dtype)


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, allowed: torch.Tensor, scale: float) -> torch.Tensor:
    """softmax(q k^T * scale, masked) v in fp32; q [B, H, S, D], k/v [B, H, T, D],
    allowed [*, *, S, T] (True = may attend).  A query with no allowed key
    (a padding position) gets a zero output instead of NaN."""
    scores = torch.matmul(q.to(torch.float32), k.to(torch.float32).transpose(-1, -2).contiguous()) * scale
    scores = scores.masked_fill(~allowed, float("-inf"))
    probs = torch.softmax(scores, dim=-1)
    probs = torch.where(allowed.any(dim=-1, keepdim=True), probs, torch.zeros_like(probs))
    return torch.matmul(probs, v.to(torch.float32).contiguous()).to(q.dtype)


class QwenAttention(nn.Module):
    def __init__(self, config, *, backend: str, packing: PackingFormat, group_size: int) -> None:
        super().__init__()
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.num_kv_heads = config.num_key_value_heads
        self.head_dim = getattr(config, "head_dim", self.hidden_size // self.num_heads)
        self.num_kv_groups = self.num_heads // self.num_kv_heads
        common = {"group_size": group_size, "backend": backend, "packing": packing}
        self.q_proj = QuantLinear(self.hidden_size, self.num_heads * self.head_dim, bias=True, **common)
        self.k_proj = QuantLinear(self.hidden_size, self.num_kv_heads * self.head_dim, bias=True, **common)
        self.v_proj = QuantLinear(self.hidden_size, self.num_kv_heads * self.head_dim, bias=True, **common)
        self.o_proj = QuantLinear(self.num_heads * self.head_dim, self.hidden_size, bias=False, **common)

    def _project(self, hidden_states, cos, sin):
        batch, sequence, _ = hidden_states.shape
        q = self.q_proj(hidden_states).view(batch, sequence, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(hidden_states).view(batch, sequence, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(hidden_states).view(batch, sequence, self.num_kv_heads, self.head_dim).transpose(1, 2)
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
        return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin, v

    def _output(self, attended, batch, sequence):
        return self.o_proj(attended.transpose(1, 2).contiguous().view(batch, sequence, self.num_heads * self.head_dim))

    def forward(self, hidden_states, cos, sin, attention_mask, past_key_value=None, use_cache=False):
        batch, sequence, _ = hidden_states.shape
        q, k, v = self._project(hidden_states, cos, sin)
        past_length = 0
        if past_key_value is not None:
            past_k, past_v = past_key_value
            expected = (batch, self.num_kv_heads, past_k.shape[2], self.head_dim)
            if past_k.shape != expected or past_v.shape != expected:
                raise ValueError("past key/value cache shape does not match this attention layer")
            if past_k.device != k.device or past_v.device != v.device:
                raise ValueError("past key/value cache must be on the attention device")
            past_length = past_k.shape[2]
            k = torch.cat((past_k, k), dim=2)
            v = torch.cat((past_v, v), dim=2)
        next_cache = (k, v) if use_cache else None
        total = past_length + sequence
        key_pos = torch.arange(total, device=hidden_states.device)
        query_pos = past_length + torch.arange(sequence, device=hidden_states.device)
        allowed = (key_pos.view(1, -1) <= query_pos.view(-1, 1)).view(1, 1, sequence, total)
        if attention_mask is not None:
            if attention_mask.shape != (batch, total):
                raise ValueError("attention_mask must cover cached and current tokens")
            allowed = allowed & attention_mask.to(torch.bool).view(batch, 1, 1, total)
        k = k.repeat_interleave(self.num_kv_groups, dim=1)
        v = v.repeat_interleave(self.num_kv_groups, dim=1)
        return self._output(attend(q, k, v, allowed, self.head_dim ** -0.5), batch, sequence), next_cache

    def forward_static(self, hidden_states, cos, sin, k_cache, v_cache, position, allowed):
        """One token per sequence: write its key/value at ``position`` (a
        device tensor) into the preallocated caches [B, kv_heads, T, D], then
        attend over the keys ``allowed`` marks."""
        batch = hidden_states.shape[0]
        q, k, v = self._project(hidden_states, cos, sin)
        k_cache.index_copy_(2, position, k)
        v_cache.index_copy_(2, position, v)
        # query head h reads key/value head h // groups: with one query token
        # the groups of a key/value head form the rows of one product
        q = q.reshape(batch, self.num_kv_heads, self.num_kv_groups, self.head_dim)
        out = attend(q, k_cache, v_cache, allowed, self.head_dim ** -0.5)
        return self._output(out.reshape(batch, self.num_heads, 1, self.head_dim), batch, 1)


class QwenMLP(nn.Module):
    def __init__(self, config, *, backend: str, packing: PackingFormat, group_size: int) -> None:
        super().__init__()
        common = {"group_size": group_size, "backend": backend, "packing": packing}
        self.gate_proj = QuantLinear(config.hidden_size, config.intermediate_size, **common)
        self.up_proj = QuantLinear(config.hidden_size, config.intermediate_size, **common)
        self.down_proj = QuantLinear(config.intermediate_size, config.hidden_size, **common)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # fp32 SwiGLU; the down projection takes fp32 activations (HIP fp32 path)
        hidden = F.silu(self.gate_proj(x).to(torch.float32)) * self.up_proj(x).to(torch.float32)
        return self.down_proj(hidden).to(x.dtype)


class DecoderLayer(nn.Module):
    def __init__(self, config, *, backend: str, packing: PackingFormat, group_size: int) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.self_attn = QwenAttention(config, backend=backend, packing=packing, group_size=group_size)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = QwenMLP(config, backend=backend, packing=packing, group_size=group_size)

    def forward(self, x, cos, sin, attention_mask, past_key_value=None, use_cache=False):
        attended, next_cache = self.self_attn(self.input_layernorm(x), cos, sin, attention_mask, past_key_value,
                                              use_cache)
        x = x + attended
        return x + self.mlp(self.post_attention_layernorm(x)), next_cache

    def forward_static(self, x, cos, sin, k_cache, v_cache, position, allowed):
        x = x + self.self_attn.forward_static(self.input_layernorm(x), cos, sin, k_cache, v_cache, position, allowed)
        return x + self.mlp(self.post_attention_layernorm(x))


class QwenModel(nn.Module):
    def __init__(self, config, *, backend: str, packing: PackingFormat, group_size: int) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, dtype=torch.bfloat16)
        self.layers = nn.ModuleList(
            DecoderLayer(config, backend=backend, packing=packing, group_size=group_size)
            for _ in range(config.num_hidden_layers)
        )
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        head_dim = getattr(config, "head_dim", config.hidden_size // config.num_attention_heads)
        self.rotary_emb = RotaryEmbedding(head_dim, getattr(config, "rope_theta", 1_000_000.0))

    def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache=False):
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        batch, sequence = input_ids.shape
        if past_key_values is not None and len(past_key_values) != len(self.layers):
            raise ValueError("past_key_values must contain one entry per decoder layer")
        past_length = 0 if past_key_values is None else past_key_values[0][0].shape[2]
        hidden = self.embed_tokens(input_ids)
        if attention_mask is None:
            attention_mask = torch.ones((batch, past_length + sequence), dtype=torch.bool, device=input_ids.device)
        elif attention_mask.shape != (batch, past_length + sequence):
            raise ValueError("attention_mask must cover cached and current tokens")
        # positions count valid tokens only (left padding): model.py:187-189
        position_ids = (attention_mask.to(torch.long).cumsum(dim=-1) - 1).clamp_min(0)[:, -sequence:]
        cos, sin = self.rotary_emb(position_ids, hidden.dtype)
        caches = []
        for index, layer in enumerate(self.layers):
            past = None if past_key_values is None else past_key_values[index]
            hidden, cache = layer(hidden, cos, sin, attention_mask, past, use_cache)
            if use_cache:
                caches.append(cache)
        hidden = self.norm(hidden)
        return (hidden, tuple(caches)) if use_cache else hidden


class QwenInt4ForCausalLM(nn.Module):
    # The reference's defaults (LEGACY packing, group 128, model.py:207-209);
    # the HIP backend rejects them at the first forward, so a W4G64 model is
    # built with packing="canonical", group_size=64, as the reference's own
    # scripts do.
    def __init__(self, config, *, backend: str = "hip", packing: PackingFormat | str = PackingFormat.LEGACY_SIGNED_ADD,
                 group_size: int = 128) -> None:
        super().__init__()
        packing = PackingFormat(packing)
        self.config = config
        self.model = QwenModel(config, backend=backend, packing=packing, group_size=group_size)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False, dtype=torch.bfloat16)
        self.lm_head.weight = self.model.embed_tokens.weight

    def set_backend(self, backend: str) -> None:
        for module in self.modules():
            if isinstance(module, QuantLinear):
                module.set_backend(backend)

    def set_packing(self, packing: PackingFormat | str) -> None:
        packing = PackingFormat(packing)
        for module in self.modules():
            if isinstance(module, QuantLinear):
                module.packing = packing

    def logits(self, hidden: torch.Tensor) -> torch.Tensor:
        # plain 2D product against the tied embedding (a library GEMM/GEMV)
        flat = hidden.reshape(-1, hidden.shape[-1])
        return F.linear(flat, self.lm_head.weight).view(*hidden.shape[:-1], -1)

    def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache=False):
        output = self.model(input_ids, attention_mask=attention_mask, past_key_values=past_key_values,
                            use_cache=use_cache)
        if not use_cache:
            return self.logits(output)
        hidden, caches = output
        return self.logits(hidden), caches

    def new_static_cache(self, batch: int, max_length: int, device=None) -> list[tuple[torch.Tensor, torch.Tensor]]:
        """Preallocated per-layer (key, value) caches [B, kv_heads, max_length, head_dim]."""
        attn = self.model.layers[0].self_attn
        shape = (batch, attn.num_kv_heads, max_length, attn.head_dim)
        device = device or self.lm_head.weight.device
        return [(torch.zeros(shape, dtype=torch.bfloat16, device=device),
                 torch.zeros(shape, dtype=torch.bfloat16, device=device)) for _ in self.model.layers]

    def decode_static(self, token_ids: torch.Tensor, position: torch.Tensor, caches) -> torch.Tensor:
        """Logits [B, 1, V] of one token per sequence at ``position`` (a 1-element
        long device tensor; all sequences unpadded and at the same position),
        reading and extending the static caches.  Fixed shapes: capturable."""
        hidden = self.model.embed_tokens(token_ids)
        cos, sin = self.model.rotary_emb(position.view(1, 1).expand(token_ids.shape[0], 1), hidden.dtype)
        max_length = caches[0][0].shape[2]
        allowed = (torch.arange(max_length, device=token_ids.device) <= position).view(1, 1, 1, max_length)
        for layer, (k_cache, v_cache) in zip(self.model.layers, caches):
            hidden = layer.forward_static(hidden, cos, sin, k_cache, v_cache, position, allowed)
        return self.logits(self.model.norm(hidden))
