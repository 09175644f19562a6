"""Fused single-token decode step of the Qwen2 decoder on the HIP kernels.

Restates one cached-token pass of QwenModel / DecoderLayer
(src/qwen_int4/model.py:61-154, :169-199) as seven launches per layer (five
at batch 1, where each add_rmsnorm but the first is formed in the staging of
the linear that follows it, ``w4g64_linear_rmsnorm``, and the residual
stream alternates between two buffers):

    add_rmsnorm          residual add of the previous MLP output (cast to bf16
                         first, model.py:136) + input RMSNorm
    W4G64 q|k|v          one GEMV over the three projections' rows, with bias
    decode_attention     rotary on q and the new k, cache write, GQA attention
                         over 64-position chunks, merged by the last chunk
    W4G64 o_proj         (batch 1, caches up to 1024 positions: the attention
                         leaves every chunk's partial result and the o_proj
                         GEMV merges them in its staging,
                         ``w4g64_linear_attention_merge``)
    add_rmsnorm          residual add of the attention output + RMSNorm
    W4G64 gate|up        one GEMV over both projections' rows; its epilogue
                         pairs gate row i with up row I + i and stores
                         silu(gate) * up (fp32, model.py:133-135) as three
                         exact bf16 planes (batches of 1..16)
    W4G64 down           the planes as its activation (three parts along K);
                         fp32 out (larger batches: the down projection forms
                         the product itself from the bf16 gate|up output)

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


def check_static_caches(caches, *, layers: int, batch: int, kv_heads: int, head_dim: int, min_length: int,
                        device) -> int:
    """Validate per-layer (key, value) static caches before any kernel writes
    them: each [batch, kv_heads, L, head_dim], bf16, contiguous, on
    ``device``, one common L >= ``min_length``.  Returns L.  The shape and
    device messages are those of the reference's attention (model.py:80-86)."""
    if len(caches) != layers:
        raise ValueError("past_key_values must contain one entry per decoder layer")
    length = None
    for pair in caches:
        if not isinstance(pair, (tuple, list)) or len(pair) != 2:
            raise ValueError("past key/value cache shape does not match this attention layer")
        for t in pair:
            if not isinstance(t, torch.Tensor) or t.ndim != 4 or tuple(t.shape[:2]) != (batch, kv_heads) \
                    or t.shape[3] != head_dim or (length is not None and t.shape[2] != length):
                raise ValueError("past key/value cache shape does not match this attention layer")
            length = t.shape[2]
            if t.device != torch.device(device):
                raise ValueError("past key/value cache must be on the attention device")
            if t.dtype != torch.bfloat16:
                raise ValueError("static key/value caches must have dtype torch.bfloat16")
            if not t.is_contiguous():
                raise ValueError("static key/value caches must be contiguous")
    if length < min_length:
        raise ValueError(f"static key/value caches hold {length} positions; {min_length} are needed")
    return length


def check_token_ids(token_ids, *, batch: int, length: int | None, device, name: str = "input_ids") -> None:
    """[batch, length] (``length`` None: any positive) int64 ids on ``device``."""
    if not isinstance(token_ids, torch.Tensor) or token_ids.ndim != 2 or token_ids.shape[0] != batch \
            or token_ids.shape[1] == 0 or (length is not None and token_ids.shape[1] != length):
        want = f"[{batch}, {length if length is not None else 'sequence'}]"
        raise ValueError(f"{name} must have shape {want}")
    if token_ids.dtype != torch.int64 or token_ids.device != torch.device(device):
        raise ValueError(f"{name} must be an int64 tensor on {device}")


def check_token_range(token_ids: torch.Tensor, vocab: int) -> None:
    """Every id in [0, vocab), as the reference's embedding requires (it
    raises torch's IndexError).  One device reduction read on the host: for
    ids that come from a caller, outside any graph.  The fused decode step
    itself never reads device memory on the host (it runs under graph
    replay): an id outside the vocabulary gives that row a NaN embedding."""
    if bool(((token_ids < 0) | (token_ids >= vocab)).any()):
        raise IndexError("index out of range in self")


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
    [batch, kv_heads, max_length, head_dim] (``model.new_static_cache``).
    ``merge_attention_in_o_proj=False`` keeps the attention's own merge where
    the o_proj GEMV would take it (the results are the same bit for bit)."""

    def __init__(self, model, batch: int, max_length: int, merge_attention_in_o_proj: bool = True) -> None:
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
        self.cos = buf(self.head_dim)      # rotary factors of the step's position
        self.sin = buf(self.head_dim)
        self.inv_freq = model.model.rotary_emb.inv_freq.to(device=device, dtype=torch.float32).contiguous()
        # batch 1: the norms fuse into the next linear, whose workgroups all
        # read the residual while one writes the updated one -- a second buffer
        self.fused_norm = batch == 1
        self.x_alt = buf(self.hidden) if self.fused_norm else None
        self.normed = buf(self.hidden)
        self.qkv = buf((self.heads + 2 * self.kv_heads) * self.head_dim)
        self.attended = buf(self.heads * self.head_dim)
        self.o = buf(self.hidden)
        # 1..16 rows: the gate|up epilogue writes silu(gate) * up as planes
        self.paired = batch <= 16
        if self.paired:
            self.planes = torch.empty((3, batch, self.inter), dtype=bf16, device=device)
        else:
            self.gate_up = buf(2 * self.inter)
        self.down = buf(self.hidden, torch.float32)
        # the planes down projection leaves its split-K partial sums to the
        # next residual add (the fused norm linear adds at most 8)
        self.down_parts = 0
        if self.paired:
            parts = self.lib.w4g64_linear_partial_count(batch, self.hidden, self.inter, _lib.DTYPE_BF16_PLANES)
            if 1 <= parts <= (8 if self.fused_norm else 255):
                self.down_parts = parts
                self.down_partials = torch.empty((parts, batch, self.hidden), dtype=torch.float32, device=device)
        shapes = [(self.qkv.shape[1], self.hidden, _lib.DTYPE_BF16),
                  (self.hidden, self.heads * self.head_dim, _lib.DTYPE_BF16),
                  (2 * self.inter, self.hidden, _lib.DTYPE_BF16_GATE_UP if self.paired else _lib.DTYPE_BF16),
                  (self.hidden, self.inter, _lib.DTYPE_BF16_PLANES if self.paired else _lib.DTYPE_BF16_SWIGLU)]
        ws = max(self.lib.w4g64_linear_workspace_bytes(batch, n, k, code) for n, k, code in shapes)
        self.workspace = torch.zeros(max(ws, 1), dtype=torch.uint8, device=device)
        aws = self.lib.qwen2_decode_attention_workspace_bytes(batch, self.kv_heads, max_length)
        self.attn_workspace = torch.zeros(max(aws, 1), dtype=torch.uint8, device=device)
        # batch 1, caches up to 1024 positions, up to 12 heads: the attention
        # leaves its per-chunk partial results and the o_proj linear merges
        # them in its staging (the same output; one cross-workgroup merge
        # fewer per layer)
        width = self.heads * self.head_dim
        self.merge_in_o_proj = (merge_attention_in_o_proj and batch == 1 and max_length <= 1024
                                and width % 256 == 0 and width <= 1536)
        head = model.lm_head.weight
        self.vocab = head.shape[0]
        # the HIP LM head (with fused greedy argmax) covers up to 16 rows
        hws = self.lib.qwen2_lm_head_workspace_bytes(batch, self.vocab, self.hidden)
        self.hip_head = hws > 0 and head.dtype == bf16 and head.is_contiguous()
        self.head_workspace = torch.zeros(max(hws, 1), dtype=torch.uint8, device=device)

    def _linear(self, x, code, weights, y, stream) -> None:
        bias = weights["bias"]
        _lib.check(self.lib.w4g64_linear(
            _ptr(x), code, _ptr(weights["qweight"]), _ptr(weights["scales"]), _ptr(weights["zeros"]), _ptr(bias),
            _lib.DTYPE_NONE if bias is None else _lib.DTYPE_BF16, _ptr(y), self.batch, y.shape[1], x.shape[1],
            _ptr(self.workspace), self.workspace.numel(), stream))

    def _norm_at(self, residual, delta, delta_code, weight, stream) -> None:
        """residual <- residual + delta (in place), self.normed <- RMSNorm of it."""
        _lib.check(self.lib.qwen2_add_rmsnorm(_ptr(residual), _ptr(delta), delta_code, _ptr(weight),
                                              ctypes.c_float(self.eps), _ptr(residual), _ptr(self.normed),
                                              self.batch, self.hidden, stream))

    def _norm_linear(self, residual, delta, delta_code, norm_weight, weights, y, planes, out_sum, stream) -> None:
        bias = weights["bias"]
        _lib.check(self.lib.w4g64_linear_rmsnorm(
            _ptr(residual), _ptr(delta), delta_code, _ptr(norm_weight), ctypes.c_float(self.eps), _ptr(out_sum),
            _ptr(weights["qweight"]), _ptr(weights["scales"]), _ptr(weights["zeros"]), _ptr(bias),
            _lib.DTYPE_NONE if bias is None else _lib.DTYPE_BF16, _ptr(y), 1 if planes else 0, self.batch,
            2 * self.inter if planes else y.shape[1], self.hidden, _ptr(self.workspace), self.workspace.numel(),
            stream))

    def __call__(self, token_ids: torch.Tensor, position: torch.Tensor, caches,
                 next_token: torch.Tensor | None = None) -> torch.Tensor:
        """Logits [batch, 1, vocab] of ``token_ids`` [batch, 1] at ``position``
        (a 1-element int64 device tensor), extending ``caches``.  With
        ``next_token`` (int64 [batch, 1], may be ``token_ids`` itself), the
        greedy choice logits.argmax(-1) is written there."""
        model = self.model
        check_token_ids(token_ids, batch=self.batch, length=1, device=self.device, name="token_ids")
        if not isinstance(position, torch.Tensor) or position.numel() != 1 or position.dtype != torch.int64 \
                or position.device != self.device:
            raise ValueError(f"position must be a 1-element int64 tensor on {self.device}")
        check_static_caches(caches, layers=len(model.model.layers), batch=self.batch, kv_heads=self.kv_heads,
                            head_dim=self.head_dim, min_length=1, device=self.device)
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        embed = model.model.embed_tokens.weight
        token_ids = token_ids if token_ids.is_contiguous() else token_ids.contiguous()
        cos, sin = self.cos, self.sin
        # embedding rows, rotary factors and the first layer's input norm (into self.normed)
        _lib.check(self.lib.qwen2_decode_prologue(
            _ptr(token_ids), _ptr(embed), _ptr(position), _ptr(self.inv_freq), _ptr(self.x), _ptr(cos), _ptr(sin),
            _ptr(model.model.layers[0].input_layernorm.weight), ctypes.c_float(self.eps), _ptr(self.normed),
            self.batch, self.hidden, embed.shape[0], self.head_dim, stream))
        delta, delta_code = None, _lib.DTYPE_NONE
        cur, other = self.x, self.x_alt  # residual stream (fused norms: read cur, write other)
        for layer, fused, (k_cache, v_cache) in zip(model.model.layers, self.fused, caches):
            if self.fused_norm and delta is not None:
                self._norm_linear(cur, delta, delta_code, layer.input_layernorm.weight, fused["qkv"], self.qkv,
                                  False, other, stream)
                cur, other = other, cur
            else:
                if delta is not None:  # the first layer's norm came with the prologue
                    self._norm_at(cur, delta, delta_code, layer.input_layernorm.weight, stream)
                self._linear(self.normed, _lib.DTYPE_BF16, fused["qkv"], self.qkv, stream)
            o_proj = layer.self_attn.o_proj
            if self.merge_in_o_proj:
                _lib.check(self.lib.qwen2_decode_attention_partials(
                    _ptr(self.qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(position), self.batch,
                    self.heads, self.kv_heads, self.head_dim, k_cache.shape[2], ctypes.c_float(self.scale),
                    _ptr(self.attn_workspace), self.attn_workspace.numel(), stream))
                _lib.check(self.lib.w4g64_linear_attention_merge(
                    _ptr(self.attn_workspace), self.attn_workspace.numel(), k_cache.shape[2], self.heads,
                    self.kv_heads, _ptr(o_proj.qweight), _ptr(o_proj.scales), _ptr(o_proj.zeros), None,
                    _lib.DTYPE_NONE, _ptr(self.o), self.batch, self.o.shape[1], stream))
            else:
                _lib.check(self.lib.qwen2_decode_attention(
                    _ptr(self.qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(position),
                    _ptr(self.attended), self.batch, self.heads, self.kv_heads, self.head_dim, k_cache.shape[2],
                    ctypes.c_float(self.scale), _ptr(self.attn_workspace), self.attn_workspace.numel(), stream))
                self._linear(self.attended, _lib.DTYPE_BF16,
                             {"qweight": o_proj.qweight, "scales": o_proj.scales, "zeros": o_proj.zeros,
                              "bias": None}, self.o, stream)
            down = layer.mlp.down_proj
            if self.fused_norm:
                self._norm_linear(cur, self.o, _lib.DTYPE_BF16, layer.post_attention_layernorm.weight,
                                  fused["gate_up"], self.planes, True, other, stream)
                cur, other = other, cur
            else:
                self._norm_at(cur, self.o, _lib.DTYPE_BF16, layer.post_attention_layernorm.weight, stream)
            if self.paired and not self.fused_norm:
                gu = fused["gate_up"]
                _lib.check(self.lib.w4g64_linear_gate_up_planes(
                    _ptr(self.normed), _ptr(gu["qweight"]), _ptr(gu["scales"]), _ptr(gu["zeros"]), _ptr(gu["bias"]),
                    _lib.DTYPE_NONE if gu["bias"] is None else _lib.DTYPE_BF16, _ptr(self.planes), self.batch,
                    2 * self.inter, self.hidden, _ptr(self.workspace), self.workspace.numel(), stream))
            if self.paired and self.down_parts:
                _lib.check(self.lib.w4g64_linear_partials(
                    _ptr(self.planes), _lib.DTYPE_BF16_PLANES, _ptr(down.qweight), _ptr(down.scales),
                    _ptr(down.zeros), _ptr(self.down_partials), self.down_partials.numel() * 4, self.batch,
                    self.hidden, self.inter, stream))
            elif self.paired:
                _lib.check(self.lib.w4g64_linear(
                    _ptr(self.planes), _lib.DTYPE_BF16_PLANES, _ptr(down.qweight), _ptr(down.scales),
                    _ptr(down.zeros), None, _lib.DTYPE_NONE, _ptr(self.down), self.batch, self.hidden, self.inter,
                    _ptr(self.workspace), self.workspace.numel(), stream))
            else:
                self._linear(self.normed, _lib.DTYPE_BF16, fused["gate_up"], self.gate_up, stream)
                _lib.check(self.lib.w4g64_linear_swiglu(
                    _ptr(self.gate_up), _ptr(down.qweight), _ptr(down.scales), _ptr(down.zeros), None,
                    _lib.DTYPE_NONE, _ptr(self.down), self.batch, self.hidden, self.inter, _ptr(self.workspace),
                    self.workspace.numel(), stream))
            if self.paired and self.down_parts:
                delta, delta_code = self.down_partials, _lib.dtype_f32_partials(self.down_parts)
            else:
                delta, delta_code = self.down, _lib.DTYPE_F32
        self._norm_at(cur, delta, delta_code, model.model.norm.weight, stream)
        if not self.hip_head:
            logits = F.linear(self.normed, model.lm_head.weight)
            if next_token is not None:
                next_token.copy_(logits.argmax(dim=-1, keepdim=True))
            return logits.view(self.batch, 1, -1)
        logits = torch.empty((self.batch, self.vocab), dtype=torch.bfloat16, device=self.device)
        if next_token is not None and (next_token.dtype != torch.int64 or next_token.numel() != self.batch
                                       or not next_token.is_contiguous()):
            raise ValueError("next_token must be a contiguous int64 tensor of batch elements")
        _lib.check(self.lib.qwen2_lm_head(
            _ptr(self.normed), _ptr(model.lm_head.weight), _ptr(logits), _ptr(next_token), self.batch, self.vocab,
            self.hidden, _ptr(self.head_workspace), self.head_workspace.numel(), stream))
        return logits.view(self.batch, 1, -1)


class FusedPrefill:
    """Prompt pass of ``batch`` unpadded prompts of one length on the HIP
    kernels, filling static caches [batch, kv_heads, max_length, head_dim]:
    per layer add_rmsnorm, the fused q|k|v GEMM (bias), rotary and causal fp32
    attention (torch, as ``QwenAttention.forward``), the o_proj GEMM,
    add_rmsnorm, the fused gate|up GEMM and the SwiGLU down projection (its
    product written as the GEMM's bf16 planes; fp32 out).  Returns the
    logits [batch, length, vocab] of every prompt position, as the model's
    forward does (src/qwen_int4/model.py:169-199, :231-245)."""

    def __init__(self, model) -> None:
        if not torch.cuda.is_available():
            raise RuntimeError("the fused prefill requires a ROCm GPU")
        self.lib = _lib.load()
        self.model = model
        self.fused = fuse_projections(model)
        attn = model.model.layers[0].self_attn
        self.heads, self.kv_heads, self.head_dim = attn.num_heads, attn.num_kv_heads, attn.head_dim
        self.hidden = model.config.hidden_size
        self.inter = model.config.intermediate_size
        self.eps = float(model.model.norm.eps)
        self._workspace = None

    def _ws(self, nbytes: int) -> torch.Tensor:
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.model.lm_head.weight.device)
        return self._workspace

    def __call__(self, input_ids: torch.Tensor, caches) -> torch.Tensor:
        model, lib = self.model, self.lib
        device = model.lm_head.weight.device
        if not isinstance(input_ids, torch.Tensor) or input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        batch, length = input_ids.shape
        check_token_ids(input_ids, batch=batch, length=None, device=device)
        check_static_caches(caches, layers=len(model.model.layers), batch=batch, kv_heads=self.kv_heads,
                            head_dim=self.head_dim, min_length=length, device=device)
        rows = batch * length
        stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        bf16 = torch.bfloat16
        shapes = [(self.heads * self.head_dim + 2 * self.kv_heads * self.head_dim, self.hidden, _lib.DTYPE_BF16),
                  (self.hidden, self.heads * self.head_dim, _lib.DTYPE_BF16),
                  (2 * self.inter, self.hidden, _lib.DTYPE_BF16),
                  (self.hidden, self.inter, _lib.DTYPE_BF16_SWIGLU)]
        ws = self._ws(max(lib.w4g64_linear_workspace_bytes(rows, n, k, c) for n, k, c in shapes))
        x = torch.index_select(model.model.embed_tokens.weight, 0, input_ids.reshape(-1))  # [rows, H]
        normed = torch.empty_like(x)
        qkv = torch.empty((rows, shapes[0][0]), dtype=bf16, device=device)
        o = torch.empty_like(x)
        gate_up = torch.empty((rows, 2 * self.inter), dtype=bf16, device=device)
        down = torch.empty((rows, self.hidden), dtype=torch.float32, device=device)
        positions = torch.arange(length, device=device).view(1, -1).expand(batch, length)
        cos, sin = model.model.rotary_emb(positions, bf16)
        cos, sin = cos.reshape(rows, -1).contiguous(), sin.reshape(rows, -1).contiguous()
        h, kvh, d = self.heads, self.kv_heads, self.head_dim
        attended = torch.empty((rows, h * d), dtype=bf16, device=device)
        qrot = torch.empty(lib.qwen2_prefill_attention_workspace_bytes(batch, h, length) // 2, dtype=bf16,
                           device=device)

        def linear(inp, code, w, out):
            bias = w["bias"]
            _lib.check(lib.w4g64_linear(
                _ptr(inp), code, _ptr(w["qweight"]), _ptr(w["scales"]), _ptr(w["zeros"]), _ptr(bias),
                _lib.DTYPE_NONE if bias is None else _lib.DTYPE_BF16, _ptr(out), rows, out.shape[1], inp.shape[1],
                _ptr(ws), ws.numel(), stream))

        def norm(delta, code, weight):
            _lib.check(lib.qwen2_add_rmsnorm(_ptr(x), _ptr(delta), code, _ptr(weight), ctypes.c_float(self.eps),
                                             _ptr(x), _ptr(normed), rows, self.hidden, stream))

        delta, delta_code = None, _lib.DTYPE_NONE
        with torch.inference_mode():
            for layer, fused, (k_cache, v_cache) in zip(model.model.layers, self.fused, caches):
                norm(delta, delta_code, layer.input_layernorm.weight)
                linear(normed, _lib.DTYPE_BF16, fused["qkv"], qkv)
                # rotary, cache update and causal attention in one call
                _lib.check(lib.qwen2_prefill_attention(
                    _ptr(qkv), _ptr(cos), _ptr(sin), _ptr(k_cache), _ptr(v_cache), _ptr(attended), batch, length,
                    h, kvh, d, k_cache.shape[2], ctypes.c_float(d ** -0.5), _ptr(qrot), qrot.numel() * 2, stream))
                op = layer.self_attn.o_proj
                linear(attended, _lib.DTYPE_BF16, {"qweight": op.qweight, "scales": op.scales, "zeros": op.zeros,
                                                   "bias": None}, o)
                norm(o, _lib.DTYPE_BF16, layer.post_attention_layernorm.weight)
                linear(normed, _lib.DTYPE_BF16, fused["gate_up"], gate_up)
                dp = layer.mlp.down_proj
                _lib.check(lib.w4g64_linear_swiglu(
                    _ptr(gate_up), _ptr(dp.qweight), _ptr(dp.scales), _ptr(dp.zeros), None, _lib.DTYPE_NONE,
                    _ptr(down), rows, self.hidden, self.inter, _ptr(ws), ws.numel(), stream))
                delta, delta_code = down, _lib.DTYPE_F32
            norm(delta, delta_code, model.model.norm.weight)
            return F.linear(normed, model.lm_head.weight).view(batch, length, -1)
