"""Fused single-token decode step of the Qwen2 decoder on the HIP kernels.

Restates one cached-token pass of QwenModel / DecoderLayer
(src/qwen_int4/model.py:61-154, :169-199) as seven launches per layer:

    add_rmsnorm          residual add of the previous MLP output (cast to bf16
                         first, model.py:136) + input RMSNorm
    W4G64 q|k|v          one GEMV over the three projections' rows, with bias
    decode_attention     rotary on q and the new k, cache write, GQA attention
    W4G64 o_proj
    add_rmsnorm          residual add of the attention output + RMSNorm
    W4G64 gate|up        one GEMV over both projections' rows
    W4G64 down (swiglu)  silu(gate) * up in fp32, formed in the down
                         projection's activation staging; fp32 out

The fused projections are views: ``fuse_projections`` concatenates the
q/k/v (and gate/up) buffers of each layer once and points the modules'
buffers at slices of the result, so the state dict, the module tree and the
eager path are unchanged and no weight is stored twice.  All intermediate
tensors are preallocated, so a step has fixed shapes and addresses and can be
captured as one HIP graph.
"""

from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .linear import QuantLinear


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _fuse(modules: list[QuantLinear]) -> dict:
    """Concatenate the packed buffers of linears that share their input along
    the output dimension and re-point each module's buffers at its slice."""
    first = modules[0]
    in_features, groups = first.in_features, first.num_groups
    if any(m.in_features != in_features or m.group_size != 64 for m in modules):
        raise ValueError("fused projections need the same in_features and group size 64")
    if any((m.out_features * groups) % 2 for m in modules):
        raise ValueError("fused projections need byte-aligned zero points (out_features * groups even)")
    with_bias = [m.bias is not None for m in modules]
    if any(with_bias) and not all(with_bias):
        raise ValueError("fused projections must all have a bias or none")
    out_features = sum(m.out_features for m in modules)
    qweight = torch.cat([m.qweight.reshape(-1) for m in modules])
    scales = torch.cat([m.scales.reshape(-1, groups) for m in modules])
    zeros = torch.cat([m.zeros.reshape(-1)[: m.out_features * groups // 2] for m in modules])
    bias = torch.cat([m.bias.reshape(-1) for m in modules]) if all(with_bias) else None
    q0 = s0 = z0 = 0
    for m in modules:
        n = m.out_features
        m.qweight = qweight[q0:q0 + n * in_features // 2].view(-1, 1)
        m.scales = scales[s0:s0 + n]
        m.zeros = zeros[z0:z0 + n * groups // 2].view(-1, 1)
        if bias is not None:
            m.bias = nn.Parameter(bias[s0:s0 + n], requires_grad=False)
        q0 += n * in_features // 2
        s0 += n
        z0 += n * groups // 2
    return {"qweight": qweight, "scales": scales, "zeros": zeros, "bias": bias, "out_features": out_features,
            "in_features": in_features}


def fuse_projections(model) -> list[dict]:
    """Fuse q/k/v and gate/up of every layer (idempotent); returns per-layer
    {"qkv": ..., "gate_up": ...} buffer sets."""
    fused = []
    # ordinary (not inference-mode) tensors, so that load_state_dict can still
    # write through the views
    with torch.inference_mode(False), torch.no_grad():
        for layer in model.model.layers:
            if not hasattr(layer, "_fused_projections"):
                attn, mlp = layer.self_attn, layer.mlp
                layer._fused_projections = {
                    "qkv": _fuse([attn.q_proj, attn.k_proj, attn.v_proj]),
                    "gate_up": _fuse([mlp.gate_proj, mlp.up_proj]),
                }
            fused.append(layer._fused_projections)
    return fused


class FusedDecodeStep:
    """Preallocated buffers and launch sequence of one decode step for
    ``batch`` sequences at a common position, over static caches
    [batch, kv_heads, max_length, head_dim] (``model.new_static_cache``)."""

    def __init__(self, model, batch: int, max_length: int) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("the fused decode step requires a ROCm GPU")
        self.lib = _lib.load()
        self.model = model
        self.batch = batch
        self.max_length = max_length
        attn = model.model.layers[0].self_attn
        self.heads, self.kv_heads, self.head_dim = attn.num_heads, attn.num_kv_heads, attn.head_dim
        if self.head_dim != 128 or self.heads % self.kv_heads or self.heads // self.kv_heads > 8:
            raise ValueError("the fused decode step needs head_dim 128 and at most 8 query heads per key/value "
                             f"head (got head_dim {self.head_dim}, {self.heads}/{self.kv_heads} heads); "
                             "use StaticGreedyDecoder(..., fused=False)")
        self.hidden = model.config.hidden_size
        self.inter = model.config.intermediate_size
        self.eps = float(model.model.norm.eps)
        self.scale = self.head_dim ** -0.5
        self.fused = fuse_projections(model)
        device = model.lm_head.weight.device
        self.device = device
        bf16 = torch.bfloat16

        def buf(cols, dtype=bf16):
            return torch.empty((batch, cols), dtype=dtype, device=device)

        self.x = buf(self.hidden)          # residual stream
        self.normed = buf(self.hidden)
        self.qkv = buf((self.heads + 2 * self.kv_heads) * self.head_dim)
        self.attended = buf(self.heads * self.head_dim)
        self.o = buf(self.hidden)
        self.gate_up = buf(2 * self.inter)
        self.down = buf(self.hidden, torch.float32)
        shapes = [(self.qkv.shape[1], self.hidden, _lib.DTYPE_BF16),
                  (self.hidden, self.heads * self.head_dim, _lib.DTYPE_BF16),
                  (2 * self.inter, self.hidden, _lib.DTYPE_BF16),
                  (self.hidden, self.inter, _lib.DTYPE_BF16_SWIGLU)]
        ws = max(self.lib.w4g64_linear_workspace_bytes(batch, n, k, code) for n, k, code in shapes)
        self.workspace = torch.zeros(max(ws, 1), dtype=torch.uint8, device=device)
        aws = self.lib.qwen2_decode_attention_workspace_bytes(batch, self.kv_heads, max_length)
        self.attn_workspace = torch.zeros(max(aws, 1), dtype=torch.uint8, device=device)

    def _linear(self, x, code, weights, y, stream) -> None:
        bias = weights["bias"]
        _lib.check(self.lib.w4g64_linear(
            _ptr(x), code, _ptr(weights["qweight"]), _ptr(weights["scales"]), _ptr(weights["zeros"]), _ptr(bias),
            _lib.DTYPE_NONE if bias is None else _lib.DTYPE_BF16, _ptr(y), self.batch, y.shape[1], x.shape[1],
            _ptr(self.workspace), self.workspace.numel(), stream))

    def _norm(self, delta, delta_code, weight, stream) -> None:
        _lib.check(self.lib.qwen2_add_rmsnorm(_ptr(self.x), _ptr(delta), delta_code, _ptr(weight),
                                              ctypes.c_float(self.eps), _ptr(self.x), _ptr(self.normed),
                                              self.batch, self.hidden, stream))

    def __call__(self, token_ids: torch.Tensor, position: torch.Tensor, caches) -> torch.Tensor:
        """Logits [batch, 1, vocab] of ``token_ids`` [batch, 1] at ``position``
        (a 1-element int64 device tensor), extending ``caches``."""
        model = self.model
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        torch.index_select(model.model.embed_tokens.weight, 0, token_ids.reshape(-1), out=self.x)
        cos, sin = model.model.rotary_emb(position.view(1, 1).expand(self.batch, 1), torch.bfloat16)
        cos = cos.reshape(self.batch, self.head_dim).contiguous()
        sin = sin.reshape(self.batch, self.head_dim).contiguous()
        delta, delta_code = None, _lib.DTYPE_NONE
        for layer, fused, (k_cache, v_cache) in zip(model.model.layers, self.fused, caches):
            self._norm(delta, delta_code, layer.input_layernorm.weight, stream)
            self._linear(self.normed, _lib.DTYPE_BF16, fused["qkv"], self.qkv, stream)
            _lib.check(self.lib.qwen2_decode_attention(
                _ptr(self.qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(position),
                _ptr(self.attended), self.batch, self.heads, self.kv_heads, self.head_dim, k_cache.shape[2],
                ctypes.c_float(self.scale), _ptr(self.attn_workspace), self.attn_workspace.numel(), stream))
            o_proj = layer.self_attn.o_proj
            self._linear(self.attended, _lib.DTYPE_BF16,
                         {"qweight": o_proj.qweight, "scales": o_proj.scales, "zeros": o_proj.zeros, "bias": None},
                         self.o, stream)
            self._norm(self.o, _lib.DTYPE_BF16, layer.post_attention_layernorm.weight, stream)
            self._linear(self.normed, _lib.DTYPE_BF16, fused["gate_up"], self.gate_up, stream)
            down = layer.mlp.down_proj
            _lib.check(self.lib.w4g64_linear_swiglu(
                _ptr(self.gate_up), _ptr(down.qweight), _ptr(down.scales), _ptr(down.zeros), None, _lib.DTYPE_NONE,
                _ptr(self.down), self.batch, self.hidden, self.inter, _ptr(self.workspace), self.workspace.numel(),
                stream))
            delta, delta_code = self.down, _lib.DTYPE_F32
        self._norm(delta, delta_code, model.model.norm.weight, stream)
        return F.linear(self.normed, model.lm_head.weight).view(self.batch, 1, -1)
