"""Fused decode-step kernels (include/qwen2_decode.h) against the torch
restatement of src/qwen_int4/model.py they replace, and the fused decode step
of the whole decoder against the module-level decode path.

Tolerances: the residual sum and the rotated cache rows repeat the
reference's bf16 roundings exactly (bit-exact); RMSNorm differs from torch
only in the order of the fp32 sum of squares (>= 99% of outputs bit-identical,
the rest one bf16 ulp); attention differs in fp32 summation order (normwise
max error <= 1e-2 of the largest output, cosine >= 0.99999); model logits
cosine >= 0.9999 (the model-level gate).
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import pytest
import torch

from qwen_int4_hip import _lib
from qwen_int4_hip.model import QwenInt4ForCausalLM, RMSNorm, RotaryEmbedding, attend, rotate_half

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


@pytest.mark.parametrize("rows,hidden", [(1, 1536), (3, 1536), (2, 896), (1, 8192), (4, 104), (2, 2056)])
@pytest.mark.parametrize("delta_dtype", [None, torch.bfloat16, torch.float32])
def test_add_rmsnorm_matches_torch(rows, hidden, delta_dtype):
    lib = _lib.load()
    g = _gen(rows * 7 + hidden)
    x = (torch.randn((rows, hidden), generator=g, device="cuda") * 3).to(torch.bfloat16)
    delta = None if delta_dtype is None else (torch.randn((rows, hidden), generator=g, device="cuda") * 2).to(delta_dtype)
    norm = RMSNorm(hidden, 1e-6).cuda()
    with torch.no_grad():
        norm.weight.copy_((torch.rand(hidden, generator=g, device="cuda") + 0.5).to(torch.bfloat16))
    want_sum = x if delta is None else x + delta.to(torch.bfloat16)
    want = norm(want_sum)
    out_sum = torch.empty_like(x)
    out = torch.empty_like(x)
    code = {None: 0, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}[delta_dtype]
    _lib.check(lib.qwen2_add_rmsnorm(_p(x), _p(delta), code, _p(norm.weight), ctypes.c_float(1e-6), _p(out_sum),
                                     _p(out), rows, hidden, _stream()))
    torch.cuda.synchronize()
    assert torch.equal(out_sum, want_sum)
    same = (out == want).float().mean().item()
    rel = ((out.float() - want.float()).abs() / want.float().abs().clamp_min(1e-30)).max().item()
    assert same >= 0.99 and rel <= 2.0 ** -7, (same, rel)
    # in place on the residual stream (out_sum aliases x)
    x2 = x.clone()
    _lib.check(lib.qwen2_add_rmsnorm(_p(x2), _p(delta), code, _p(norm.weight), ctypes.c_float(1e-6), _p(x2),
                                     _p(out), rows, hidden, _stream()))
    torch.cuda.synchronize()
    assert torch.equal(x2, want_sum)


@pytest.mark.parametrize("delta_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("form,n,k", [("linear", 2048, 1536), ("linear", 200, 640), ("planes", 8960, 1536),
                                      ("planes", 72, 192), ("planes", 256, 256), ("planes", 2064, 640),
                                      ("planes", 17920, 1536), ("planes", 512, 2048)])
def test_linear_rmsnorm_matches_norm_then_linear(delta_dtype, form, n, k):
    """w4g64_linear_rmsnorm (one row) = qwen2_add_rmsnorm followed by the
    plain linear (or the gate|up planes entry): the residual sum bit-exact
    (torch's bf16 add), the activation to the norm's own bar (the fp32 sum of
    squares runs in another order), so the outputs agree to the bf16 rounding
    that can flip (normwise 1e-2; most outputs identical)."""
    lib = _lib.load()
    g = _gen(n + k + (1 if delta_dtype == torch.float32 else 0))
    x = (torch.randn((1, k), generator=g, device="cuda") * 3).to(torch.bfloat16)
    delta = (torch.randn((1, k), generator=g, device="cuda") * 2).to(delta_dtype)
    norm = RMSNorm(k, 1e-6).cuda()
    with torch.no_grad():
        norm.weight.copy_((torch.rand(k, generator=g, device="cuda") + 0.5).to(torch.bfloat16))
    qw, sc, z = _weights(n, k, 23, asymmetric=True)
    bias = (torch.randn(n, generator=g, device="cuda") * 0.3).to(torch.bfloat16) if form == "linear" else None
    dcode = _lib.DTYPE_BF16 if delta_dtype == torch.bfloat16 else _lib.DTYPE_F32
    planes = form == "planes"
    y = (torch.empty((3, 1, n // 2), dtype=torch.bfloat16, device="cuda") if planes
         else torch.empty((1, n), dtype=torch.bfloat16, device="cuda"))
    out_sum = torch.empty_like(x)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    _lib.check(lib.w4g64_linear_rmsnorm(_p(x), _p(delta), dcode, _p(norm.weight), ctypes.c_float(1e-6), _p(out_sum),
                                        _p(qw), _p(sc), _p(z), _p(bias), _lib.DTYPE_BF16 if bias is not None else 0,
                                        _p(y), 1 if planes else 0, 1, n, k, _p(ws), ws.numel(), _stream()))
    # the separate kernels
    ref_sum, normed = torch.empty_like(x), torch.empty_like(x)
    _lib.check(lib.qwen2_add_rmsnorm(_p(x), _p(delta), dcode, _p(norm.weight), ctypes.c_float(1e-6), _p(ref_sum),
                                     _p(normed), 1, k, _stream()))
    want = torch.empty_like(y)
    if planes:
        _lib.check(lib.w4g64_linear_gate_up_planes(_p(normed), _p(qw), _p(sc), _p(z), None, 0, _p(want), 1, n, k,
                                                   _p(ws), ws.numel(), _stream()))
    else:
        _lib.check(lib.w4g64_linear(_p(normed), _lib.DTYPE_BF16, _p(qw), _p(sc), _p(z), _p(bias), _lib.DTYPE_BF16,
                                    _p(want), 1, n, k, _p(ws), ws.numel(), _stream()))
    torch.cuda.synchronize()
    assert torch.equal(out_sum, x + delta.to(torch.bfloat16)) and torch.equal(out_sum, ref_sum)
    got = y.float().sum(0) if planes else y.float()
    ref = want.float().sum(0) if planes else want.float()
    assert bool(torch.isfinite(got).all())
    assert _normwise(got, ref) <= 1e-2
    assert (got == ref).float().mean().item() >= 0.9


def _torch_attention(qkv, cos, sin, k_cache, v_cache, pos, heads, kv_heads):
    """The module path of one cached token: rotary in bf16, cache write,
    fp32 attention over positions 0..pos (qwen_int4_hip.model, which restates
    model.py:61-122)."""
    batch = qkv.shape[0]
    d = 128
    q = qkv[:, : heads * d].view(batch, heads, 1, d)
    k = qkv[:, heads * d:(heads + kv_heads) * d].view(batch, kv_heads, 1, d)
    v = qkv[:, (heads + kv_heads) * d:].view(batch, kv_heads, 1, d)
    c, s = cos.view(batch, 1, 1, d), sin.view(batch, 1, 1, d)
    q = q * c + rotate_half(q) * s
    k = k * c + rotate_half(k) * s
    k_cache = k_cache.clone()
    v_cache = v_cache.clone()
    k_cache[:, :, pos] = k[:, :, 0]
    v_cache[:, :, pos] = v[:, :, 0]
    group = heads // kv_heads
    allowed = (torch.arange(k_cache.shape[2], device="cuda") <= pos).view(1, 1, 1, -1)
    out = attend(q.reshape(batch, kv_heads, group, d), k_cache, v_cache, allowed, d ** -0.5)
    return out.reshape(batch, heads * d), k_cache, v_cache


@pytest.mark.parametrize("batch,heads,kv_heads,max_length,positions", [
    (1, 12, 2, 640, (0, 1, 63, 64, 65, 200, 511, 639)),
    (3, 12, 2, 130, (0, 64, 127, 129)),
    (2, 8, 1, 64, (0, 31, 63)),
    (1, 4, 4, 700, (5, 699)),
    (1, 12, 2, 2048, (1000, 2047)),  # 32 chunks merged
    (1, 12, 2, 2200, (0, 64, 2199)),  # a partial last chunk; early positions leave most chunks empty
])
def test_decode_attention_matches_torch(batch, heads, kv_heads, max_length, positions):
    lib = _lib.load()
    g = _gen(batch * 1000 + heads * 10 + kv_heads)
    d = 128
    rot = RotaryEmbedding(d, 1_000_000.0).cuda()
    k_cache = (torch.randn((batch, kv_heads, max_length, d), generator=g, device="cuda")).to(torch.bfloat16)
    v_cache = (torch.randn((batch, kv_heads, max_length, d), generator=g, device="cuda")).to(torch.bfloat16)
    ws = torch.zeros(lib.qwen2_decode_attention_workspace_bytes(batch, kv_heads, max_length), dtype=torch.uint8,
                     device="cuda")
    for pos in positions:
        qkv = (torch.randn((batch, (heads + 2 * kv_heads) * d), generator=g, device="cuda") * 2).to(torch.bfloat16)
        position = torch.tensor([pos], dtype=torch.long, device="cuda")
        cos, sin = rot(position.view(1, 1).expand(batch, 1), torch.bfloat16)
        cos, sin = cos.reshape(batch, d).contiguous(), sin.reshape(batch, d).contiguous()
        want, want_k, want_v = _torch_attention(qkv, cos, sin, k_cache, v_cache, pos, heads, kv_heads)
        out = torch.empty((batch, heads * d), dtype=torch.bfloat16, device="cuda")
        for _ in range(2):  # a second call on the same workspace: counters were left at zero
            _lib.check(lib.qwen2_decode_attention(
                _p(qkv), _p(cos), _p(sin), _p(k_cache), _p(v_cache), _p(position), _p(out), batch, heads, kv_heads,
                d, max_length, ctypes.c_float(d ** -0.5), _p(ws), ws.numel(), _stream()))
            torch.cuda.synchronize()
            assert torch.equal(k_cache, want_k) and torch.equal(v_cache, want_v)
            err = (out.float() - want.float()).abs().max().item()
            cos_sim = torch.nn.functional.cosine_similarity(out.double().flatten(), want.double().flatten(), dim=0)
            assert err <= 1e-2 * want.float().abs().max().item(), (pos, err)
            assert cos_sim.item() >= 0.99999, (pos, cos_sim.item())


@pytest.mark.parametrize("heads,kv_heads,max_length,positions,n,with_bias", [
    (12, 2, 640, (0, 1, 63, 64, 65, 511, 639), 1536, False),
    (12, 2, 1024, (0, 700, 1023), 1536, True),  # 16 chunks: the most the merge form takes
    (8, 1, 100, (3, 99), 200, False),            # 8 query heads per key/value head, a partial last chunk
    (2, 2, 64, (0, 63), 96, False),              # one query head per key/value head, one chunk
    (4, 2, 200, (130,), 1536, True),
])
def test_attention_merged_in_o_proj_equals_attention_then_o_proj(heads, kv_heads, max_length, positions, n,
                                                                 with_bias):
    """qwen2_decode_attention_partials + w4g64_linear_attention_merge against
    qwen2_decode_attention + w4g64_linear on the same inputs: the same cache
    writes and, bit for bit, the same o_proj output (the merge in the GEMV's
    staging repeats the attention's own merge operation for operation).  The
    unmerged path's workspace starts as NaN, so chunks past the position must
    be written (as empty partials), not assumed."""
    lib = _lib.load()
    g = _gen(heads * 100 + kv_heads + max_length)
    d = 128
    k = heads * d
    rot = RotaryEmbedding(d, 1_000_000.0).cuda()
    k_cache = torch.randn((1, kv_heads, max_length, d), generator=g, device="cuda").to(torch.bfloat16)
    v_cache = torch.randn((1, kv_heads, max_length, d), generator=g, device="cuda").to(torch.bfloat16)
    k_part, v_part = k_cache.clone(), v_cache.clone()
    qw, sc, z = _weights(n, k, heads + n, asymmetric=True)
    bias = (torch.randn(n, generator=g, device="cuda") * 0.1).to(torch.bfloat16) if with_bias else None
    bias_code = _lib.DTYPE_BF16 if with_bias else _lib.DTYPE_NONE
    wbytes = lib.qwen2_decode_attention_workspace_bytes(1, kv_heads, max_length)
    ws = torch.zeros(wbytes, dtype=torch.uint8, device="cuda")
    ws_part = torch.full((wbytes,), 0xFF, dtype=torch.uint8, device="cuda")  # NaN partials
    lws = torch.zeros(max(lib.w4g64_linear_workspace_bytes(1, n, k, _lib.DTYPE_BF16), 1), dtype=torch.uint8,
                      device="cuda")
    attended = torch.empty((1, k), dtype=torch.bfloat16, device="cuda")
    want = torch.empty((1, n), dtype=torch.bfloat16, device="cuda")
    got = torch.empty((1, n), dtype=torch.bfloat16, device="cuda")
    for pos in positions:
        qkv = (torch.randn((1, (heads + 2 * kv_heads) * d), generator=g, device="cuda") * 2).to(torch.bfloat16)
        position = torch.tensor([pos], dtype=torch.long, device="cuda")
        cos, sin = rot(position.view(1, 1), torch.bfloat16)
        cos, sin = cos.reshape(1, d).contiguous(), sin.reshape(1, d).contiguous()
        _lib.check(lib.qwen2_decode_attention(
            _p(qkv), _p(cos), _p(sin), _p(k_cache), _p(v_cache), _p(position), _p(attended), 1, heads, kv_heads, d,
            max_length, ctypes.c_float(d ** -0.5), _p(ws), ws.numel(), _stream()))
        _lib.check(lib.w4g64_linear(_p(attended), _lib.DTYPE_BF16, _p(qw), _p(sc), _p(z), _p(bias), bias_code,
                                    _p(want), 1, n, k, _p(lws), lws.numel(), _stream()))
        _lib.check(lib.qwen2_decode_attention_partials(
            _p(qkv), _p(cos), _p(sin), _p(k_part), _p(v_part), _p(position), 1, heads, kv_heads, d, max_length,
            ctypes.c_float(d ** -0.5), _p(ws_part), ws_part.numel(), _stream()))
        _lib.check(lib.w4g64_linear_attention_merge(_p(ws_part), ws_part.numel(), max_length, heads, kv_heads,
                                                    _p(qw), _p(sc), _p(z), _p(bias), bias_code, _p(got), 1, n,
                                                    _stream()))
        torch.cuda.synchronize()
        assert torch.equal(k_part, k_cache) and torch.equal(v_part, v_cache), pos
        assert torch.isfinite(want.float()).all(), pos
        assert torch.equal(got, want), (pos, (got.float() - want.float()).abs().max().item())


def test_fused_decode_step_merged_in_o_proj_is_bit_identical():
    """The batch-1 decode step with the attention merged in the o_proj GEMV
    against the same step with the attention's own merge: identical logits,
    greedy tokens and caches over 70 steps (across a 64-position chunk
    boundary)."""
    from qwen_int4_hip.decode import FusedDecodeStep
    from qwen_int4_hip.generation import StaticGreedyDecoder

    model = _build(SMALL128, 21)
    prompt = torch.randint(0, SMALL128.vocab_size, (1, 13), generator=torch.Generator().manual_seed(7)).cuda()
    merged = StaticGreedyDecoder(model, 1, 96, use_graph=False, fused=True)
    plain = StaticGreedyDecoder(model, 1, 96, use_graph=False, fused=True)
    plain.fused = FusedDecodeStep(model, 1, 96, merge_attention_in_o_proj=False)
    assert merged.fused.merge_in_o_proj and not plain.fused.merge_in_o_proj
    merged.prefill(prompt)
    plain.prefill(prompt)
    for step in range(70):
        token = plain.token.clone()
        want = plain.step(token).clone()
        got = merged.step(token).clone()
        assert torch.equal(got, want), step
        assert torch.equal(merged.token, plain.token), step
    for (k0, v0), (k1, v1) in zip(plain.caches, merged.caches):
        assert torch.equal(k0, k1) and torch.equal(v0, v1)


@pytest.mark.parametrize("batch,hidden,vocab", [(1, 1536, 151936), (3, 256, 512)])
def test_decode_prologue_matches_embedding_and_rotary(batch, hidden, vocab):
    """qwen2_decode_prologue = the embedding lookup and RotaryEmbedding.forward
    of one position (model.py:22-31, :182, :190), bit for bit, at positions up
    to a 17408-position cache, and the first layer's RMSNorm to its bar; an id
    outside [0, vocab) gives a NaN row."""
    lib = _lib.load()
    g = _gen(batch * 31 + hidden)
    embed = (torch.randn((vocab, hidden), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    rot = RotaryEmbedding(128, 1_000_000.0).cuda()
    x = torch.empty((batch, hidden), dtype=torch.bfloat16, device="cuda")
    normed = torch.empty_like(x)
    norm = RMSNorm(hidden, 1e-6).cuda()
    with torch.no_grad():
        norm.weight.copy_((torch.rand(hidden, generator=g, device="cuda") + 0.5).to(torch.bfloat16))
    cos = torch.empty((batch, 128), dtype=torch.bfloat16, device="cuda")
    sin = torch.empty_like(cos)
    for pos in (0, 1, 63, 511, 640, 4095, 17407):
        ids = torch.randint(0, vocab, (batch,), generator=g, device="cuda", dtype=torch.int64)
        position = torch.tensor([pos], dtype=torch.int64, device="cuda")
        _lib.check(lib.qwen2_decode_prologue(_p(ids), _p(embed), _p(position), _p(rot.inv_freq), _p(x), _p(cos),
                                             _p(sin), _p(norm.weight), ctypes.c_float(1e-6), _p(normed), batch,
                                             hidden, vocab, 128, _stream()))
        want_cos, want_sin = rot(position.view(1, 1).expand(batch, 1), torch.bfloat16)
        want_x = embed[ids]
        want_n = norm(want_x)
        torch.cuda.synchronize()
        assert torch.equal(x, want_x), pos
        assert torch.equal(cos, want_cos.reshape(batch, 128)), pos
        assert torch.equal(sin, want_sin.reshape(batch, 128)), pos
        # the norm to RMSNorm's bar (the fp32 sum of squares runs in another order)
        rel = ((normed.float() - want_n.float()).abs() / want_n.float().abs().clamp_min(1e-30)).max().item()
        assert (normed == want_n).float().mean().item() >= 0.99 and rel <= 2.0 ** -7, (pos, rel)
    # without the norm: x, cos and sin only
    _lib.check(lib.qwen2_decode_prologue(_p(ids), _p(embed), _p(position), _p(rot.inv_freq), _p(x), _p(cos), _p(sin),
                                         None, ctypes.c_float(1e-6), None, batch, hidden, vocab, 128, _stream()))
    torch.cuda.synchronize()
    assert torch.equal(x, embed[ids])
    bad = torch.full((batch,), vocab, dtype=torch.int64, device="cuda")
    _lib.check(lib.qwen2_decode_prologue(_p(bad), _p(embed), _p(position), _p(rot.inv_freq), _p(x), _p(cos), _p(sin),
                                         None, ctypes.c_float(1e-6), None, batch, hidden, vocab, 128, _stream()))
    torch.cuda.synchronize()
    assert bool(torch.isnan(x.float()).all())


@pytest.mark.parametrize("batch,heads,kv_heads,length,max_length", [
    (1, 12, 2, 512, 640),  # the prefill of the model's workload
    (2, 8, 1, 100, 128),   # a partial last block; group 8
    (3, 4, 4, 65, 70),     # one query row past a block boundary; no grouping
    (1, 12, 2, 1, 8),      # a single position
])
def test_prefill_attention_matches_torch(batch, heads, kv_heads, length, max_length):
    """Rotary, cache update and causal attention over a prompt against the
    module path's torch restatement (rotary in bf16, fp32 attention)."""
    lib = _lib.load()
    g = _gen(batch * 100 + length)
    d = 128
    rows = batch * length
    qkv = (torch.randn((rows, (heads + 2 * kv_heads) * d), generator=g, device="cuda") * 2).to(torch.bfloat16)
    k_cache = torch.randn((batch, kv_heads, max_length, d), generator=g, device="cuda").to(torch.bfloat16)
    v_cache = torch.randn((batch, kv_heads, max_length, d), generator=g, device="cuda").to(torch.bfloat16)
    positions = torch.arange(length, device="cuda").view(1, -1).expand(batch, length)
    cos, sin = RotaryEmbedding(d, 1_000_000.0).cuda()(positions, torch.bfloat16)
    q = qkv[:, : heads * d].view(batch, length, heads, d).transpose(1, 2)
    k = qkv[:, heads * d:(heads + kv_heads) * d].view(batch, length, kv_heads, d).transpose(1, 2)
    v = qkv[:, (heads + kv_heads) * d:].view(batch, length, kv_heads, d).transpose(1, 2)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    q = q * c + rotate_half(q) * s
    k = k * c + rotate_half(k) * s
    want_k, want_v = k_cache.clone(), v_cache.clone()
    want_k[:, :, :length] = k
    want_v[:, :, :length] = v
    allowed = torch.ones((length, length), dtype=torch.bool, device="cuda").tril().view(1, 1, length, length)
    group = heads // kv_heads
    want = attend(q, k.repeat_interleave(group, dim=1), v.repeat_interleave(group, dim=1), allowed, d ** -0.5)
    want = want.transpose(1, 2).reshape(rows, heads * d)
    out = torch.empty((rows, heads * d), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(lib.qwen2_prefill_attention_workspace_bytes(batch, heads, length), dtype=torch.uint8,
                     device="cuda")
    _lib.check(lib.qwen2_prefill_attention(
        _p(qkv), _p(cos.reshape(rows, d).contiguous()), _p(sin.reshape(rows, d).contiguous()), _p(k_cache),
        _p(v_cache), _p(out), batch, length, heads, kv_heads, d, max_length, ctypes.c_float(d ** -0.5), _p(ws),
        ws.numel(), _stream()))
    torch.cuda.synchronize()
    assert torch.equal(k_cache, want_k) and torch.equal(v_cache, want_v)  # rows past the prompt untouched
    err = (out.float() - want.float()).abs().max().item()
    cos_sim = torch.nn.functional.cosine_similarity(out.double().flatten(), want.double().flatten(), dim=0)
    assert err <= 1e-2 * want.float().abs().max().item(), err
    assert cos_sim.item() >= 0.99999, cos_sim.item()


@pytest.mark.parametrize("rows,inter", [(1, 8960), (4, 8960), (16, 100)])
def test_silu_mul_matches_torch(rows, inter):
    lib = _lib.load()
    g = _gen(rows + inter)
    gate_up = (torch.randn((rows, 2 * inter), generator=g, device="cuda") * 4).to(torch.bfloat16)
    want = torch.nn.functional.silu(gate_up[:, :inter].float()) * gate_up[:, inter:].float()
    out = torch.empty((rows, inter), dtype=torch.float32, device="cuda")
    _lib.check(lib.qwen2_silu_mul(_p(gate_up), _p(out), rows, inter, _stream()))
    torch.cuda.synchronize()
    assert torch.allclose(out, want, rtol=2e-6, atol=1e-30)
    assert (out == want).float().mean().item() >= 0.99


def _weights(n, k, seed, asymmetric=False):
    from oracle import oracle as O

    q, sc, z = (O.asymmetric_weights(n, k, seed) if asymmetric else O.symmetric_weights(n, k, seed))
    return tuple(torch.from_numpy(t).cuda() for t in (q, sc, z))


def _normwise(got, want):
    return ((got.float() - want.float()).abs().max() / want.float().abs().max()).item()


@pytest.mark.parametrize("rows", [1, 4, 9, 16])
@pytest.mark.parametrize("n,k", [(1536, 8960), (100, 128), (256, 1536)])
def test_linear_swiglu_matches_silu_then_reference_linear(rows, n, k):
    """w4g64_linear_swiglu = fp32 silu(gate) * up (torch) followed by the
    reference torch backend's fp32 linear (the oracle); the fp32 activations
    run exactly (three bf16 parts), so the output agrees to fp32 summation
    order (normwise 1e-5)."""
    from oracle import oracle as O

    lib = _lib.load()
    g = _gen(rows * 17 + n + k)
    gate_up = (torch.randn((rows, 2 * k), generator=g, device="cuda") * 3).to(torch.bfloat16)
    h = torch.nn.functional.silu(gate_up[:, :k].float()) * gate_up[:, k:].float()
    qw, sc, z = _weights(n, k, 9)
    want = O.reference_linear_torch(h, qw, sc, z, None, out_features=n, in_features=k)
    ws = torch.zeros(max(1, lib.w4g64_linear_workspace_bytes(rows, n, k, _lib.DTYPE_BF16_SWIGLU)),
                     dtype=torch.uint8, device="cuda")
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    _lib.check(lib.w4g64_linear_swiglu(_p(gate_up), _p(qw), _p(sc), _p(z), None, 0, _p(y), rows, n, k, _p(ws),
                                       ws.numel(), _stream()))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all()) and _normwise(y, want) <= 1e-5


def _split3(h):
    """Exact three-way bf16 split of fp32 h by truncation: planes [3, ...]
    with hi + mid + lo == h (the decomposition the GEMV kernels stage)."""
    mask = torch.tensor(-65536, dtype=torch.int32, device=h.device)  # 0xFFFF0000
    hi = (h.contiguous().view(torch.int32) & mask).view(torch.float32)
    r1 = h - hi
    mid = (r1.view(torch.int32) & mask).view(torch.float32)
    lo = r1 - mid
    top = lambda t: (t.view(torch.int32) >> 16).to(torch.int16).view(torch.bfloat16)
    return torch.stack([top(hi), top(mid), top(lo)])


@pytest.mark.parametrize("rows", [1, 4, 9, 16])
@pytest.mark.parametrize("n,k", [(1536, 8960), (100, 128), (256, 1536)])
def test_linear_planes_form_matches_reference_linear(rows, n, k):
    """w4g64_linear with the bf16-planes activation form = the reference torch
    backend's fp32 linear of the planes' sum (the oracle); the planes are the
    exact split, so the output agrees to fp32 summation order (normwise 1e-5)."""
    from oracle import oracle as O

    lib = _lib.load()
    g = _gen(rows * 23 + n + k)
    h = torch.randn((rows, k), generator=g, device="cuda") * 2
    planes = _split3(h)
    assert torch.equal(planes.float().sum(0), h)
    qw, sc, z = _weights(n, k, 13, asymmetric=True)
    want = O.reference_linear_torch(h, qw, sc, z, None, out_features=n, in_features=k)
    ws = torch.zeros(max(1, lib.w4g64_linear_workspace_bytes(rows, n, k, _lib.DTYPE_BF16_PLANES)),
                     dtype=torch.uint8, device="cuda")
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    _lib.check(lib.w4g64_linear(_p(planes), _lib.DTYPE_BF16_PLANES, _p(qw), _p(sc), _p(z), None, 0, _p(y), rows, n,
                                k, _p(ws), ws.numel(), _stream()))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all()) and _normwise(y, want) <= 1e-5


def _partials_and_reduced(lib, x, code, qw, sc, z, rows, n, k):
    """w4g64_linear_partials' partial sums and w4g64_linear's reduced output."""
    parts = lib.w4g64_linear_partial_count(rows, n, k, code)
    assert parts >= 1
    partials = torch.empty((parts, rows, n), dtype=torch.float32, device="cuda")
    _lib.check(lib.w4g64_linear_partials(_p(x), code, _p(qw), _p(sc), _p(z), _p(partials), partials.numel() * 4,
                                         rows, n, k, _stream()))
    ws = torch.zeros(max(1, lib.w4g64_linear_workspace_bytes(rows, n, k, code)), dtype=torch.uint8, device="cuda")
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    _lib.check(lib.w4g64_linear(_p(x), code, _p(qw), _p(sc), _p(z), None, 0, _p(y), rows, n, k, _p(ws), ws.numel(),
                                _stream()))
    torch.cuda.synchronize()
    return partials, y


def _sum_in_order(partials):
    total = torch.zeros_like(partials[0])
    for part in partials:
        total = total + part
    return total + 0.0


@pytest.mark.parametrize("code", [_lib.DTYPE_BF16_PLANES, _lib.DTYPE_F32])
@pytest.mark.parametrize("rows", [1, 2, 5, 16])
@pytest.mark.parametrize("n,k", [(1536, 8960), (100, 128)])
def test_linear_partials_sum_to_the_reduced_linear(code, rows, n, k):
    """w4g64_linear_partials leaves the split-K partial sums to the caller:
    their sum in order from part 0 is w4g64_linear's fp32 output bit for bit
    (the reduction kernel adds them in that order)."""
    lib = _lib.load()
    g = _gen(rows * 29 + n + k + code)
    h = torch.randn((rows, k), generator=g, device="cuda") * 2
    x = _split3(h) if code == _lib.DTYPE_BF16_PLANES else h
    qw, sc, z = _weights(n, k, 31, asymmetric=True)
    partials, y = _partials_and_reduced(lib, x, code, qw, sc, z, rows, n, k)
    assert torch.equal(_sum_in_order(partials), y)
    if n == 1536 and k == 8960 and code == _lib.DTYPE_BF16_PLANES:
        assert partials.shape[0] > 1  # the decode down projection splits K


@pytest.mark.parametrize("rows", [1, 3])
def test_add_rmsnorm_adds_partial_sums_like_the_reduced_delta(rows):
    """qwen2_add_rmsnorm with delta W4G64_DTYPE_F32_PARTIALS(count) = with the
    reduced fp32 delta, bit for bit (sum and norm)."""
    lib = _lib.load()
    hidden, k = 1536, 8960
    g = _gen(rows + 41)
    x = (torch.randn((rows, hidden), generator=g, device="cuda") * 3).to(torch.bfloat16)
    planes = _split3(torch.randn((rows, k), generator=g, device="cuda") * 2)
    qw, sc, z = _weights(hidden, k, 37, asymmetric=False)
    partials, y = _partials_and_reduced(lib, planes, _lib.DTYPE_BF16_PLANES, qw, sc, z, rows, hidden, k)
    weight = (torch.rand(hidden, generator=g, device="cuda") + 0.5).to(torch.bfloat16)
    outs = []
    for delta, code in ((y, _lib.DTYPE_F32), (partials, _lib.dtype_f32_partials(partials.shape[0]))):
        out_sum, out = torch.empty_like(x), torch.empty_like(x)
        _lib.check(lib.qwen2_add_rmsnorm(_p(x), _p(delta), code, _p(weight), ctypes.c_float(1e-6), _p(out_sum),
                                         _p(out), rows, hidden, _stream()))
        outs.append((out_sum, out))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("form,n", [("linear", 2048), ("planes", 17920)])
def test_linear_rmsnorm_adds_partial_sums_like_the_reduced_delta(form, n):
    """w4g64_linear_rmsnorm with the down projection's partial sums as delta =
    with their reduced fp32 output: residual sum and linear output bit for bit."""
    lib = _lib.load()
    hidden, inter = 1536, 8960
    g = _gen(n + 43)
    x = (torch.randn((1, hidden), generator=g, device="cuda") * 3).to(torch.bfloat16)
    planes = _split3(torch.randn((1, inter), generator=g, device="cuda") * 2)
    dq, ds, dz = _weights(hidden, inter, 47, asymmetric=True)
    partials, y = _partials_and_reduced(lib, planes, _lib.DTYPE_BF16_PLANES, dq, ds, dz, 1, hidden, inter)
    assert 1 < partials.shape[0] <= 8
    qw, sc, z = _weights(n, hidden, 53, asymmetric=True)
    weight = (torch.rand(hidden, generator=g, device="cuda") + 0.5).to(torch.bfloat16)
    pl = form == "planes"
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    outs = []
    for delta, code in ((y, _lib.DTYPE_F32), (partials, _lib.dtype_f32_partials(partials.shape[0]))):
        out_sum = torch.empty_like(x)
        out = (torch.empty((3, 1, n // 2), dtype=torch.bfloat16, device="cuda") if pl
               else torch.empty((1, n), dtype=torch.bfloat16, device="cuda"))
        _lib.check(lib.w4g64_linear_rmsnorm(_p(x), _p(delta), code, _p(weight), ctypes.c_float(1e-6), _p(out_sum),
                                            _p(qw), _p(sc), _p(z), None, 0, _p(out), 1 if pl else 0, 1, n, hidden,
                                            _p(ws), ws.numel(), _stream()))
        outs.append((out_sum, out))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("rows", [1, 4, 9, 16])
@pytest.mark.parametrize("inter,k", [(8960, 1536), (100, 128), (72, 192)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gate_up_planes_matches_reference_swiglu_product(rows, inter, k, with_bias):
    """w4g64_linear_gate_up_planes over a stacked [gate; up] weight writes
    h = silu(bf16(gate)) * bf16(up) (model.py:133-135) as the exact bf16
    split of its fp32 value: the planes reassemble to h exactly, and h agrees
    with the oracle's projections (bf16 outputs, as the reference's) followed
    by torch's silu and product -- to the bf16 rounding of gate and up that
    a different fp32 summation order can flip (normwise 1e-2, the GEMM bar)."""
    from oracle import oracle as O

    lib = _lib.load()
    g = _gen(rows * 31 + inter + k)
    x = (torch.randn((rows, k), generator=g, device="cuda")).to(torch.bfloat16)
    gw = _weights(inter, k, 17)
    uw = _weights(inter, k, 19, asymmetric=True)
    qw, sc, z = (torch.cat([a.reshape(-1), b.reshape(-1)]) for a, b in zip(gw, uw))
    sc = sc.view(2 * inter, k // 64)
    bias = (torch.randn(2 * inter, generator=g, device="cuda") * 0.5).to(torch.bfloat16) if with_bias else None
    ws = torch.zeros(max(1, lib.w4g64_linear_workspace_bytes(rows, 2 * inter, k, _lib.DTYPE_BF16_GATE_UP)),
                     dtype=torch.uint8, device="cuda")
    planes = torch.empty((3, rows, inter), dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.w4g64_linear_gate_up_planes(_p(x), _p(qw), _p(sc), _p(z), _p(bias),
                                               _lib.DTYPE_BF16 if with_bias else _lib.DTYPE_NONE, _p(planes), rows,
                                               2 * inter, k, _p(ws), ws.numel(), _stream()))
    torch.cuda.synchronize()
    h = planes.float().sum(0)
    assert torch.equal(_split3(h), planes)
    gate = O.reference_linear_torch(x, *gw, None if bias is None else bias[:inter], out_features=inter, in_features=k)
    up = O.reference_linear_torch(x, *uw, None if bias is None else bias[inter:], out_features=inter, in_features=k)
    want = torch.nn.functional.silu(gate.float()) * up.float()
    assert bool(torch.isfinite(h).all()) and _normwise(h, want) <= 1e-2


@pytest.mark.parametrize("rows", [17, 64, 512])
@pytest.mark.parametrize("n,k", [(1536, 8960), (100, 128)])
def test_linear_swiglu_gemm_rows(rows, n, k):
    """Prefill rows: the product is written as the GEMM's bf16 hi|lo planes and
    multiplied by bf16-rounded dequantized weights -- the GEMM bar, normwise
    1e-2."""
    from oracle import oracle as O

    lib = _lib.load()
    g = _gen(rows * 13 + n + k)
    gate_up = (torch.randn((rows, 2 * k), generator=g, device="cuda") * 3).to(torch.bfloat16)
    h = torch.nn.functional.silu(gate_up[:, :k].float()) * gate_up[:, k:].float()
    qw, sc, z = _weights(n, k, 11, asymmetric=True)
    want = O.reference_linear_torch(h, qw, sc, z, None, out_features=n, in_features=k)
    ws = torch.zeros(lib.w4g64_linear_workspace_bytes(rows, n, k, _lib.DTYPE_BF16_SWIGLU), dtype=torch.uint8,
                     device="cuda")
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    _lib.check(lib.w4g64_linear_swiglu(_p(gate_up), _p(qw), _p(sc), _p(z), None, 0, _p(y), rows, n, k, _p(ws),
                                       ws.numel(), _stream()))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all()) and _normwise(y, want) <= 1e-2


def _lm_head(x, weight, with_argmax=True):
    lib = _lib.load()
    rows, hidden = x.shape
    vocab = weight.shape[0]
    logits = torch.full((rows, vocab), float("nan"), dtype=torch.bfloat16, device="cuda")
    argmax = torch.full((rows,), -1, dtype=torch.int64, device="cuda") if with_argmax else None
    nbytes = lib.qwen2_lm_head_workspace_bytes(rows, vocab, hidden)
    assert nbytes > 0
    workspace = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    _lib.check(lib.qwen2_lm_head(_p(x), _p(weight), _p(logits), _p(argmax), rows, vocab, hidden, _p(workspace),
                                 nbytes, _stream()))
    torch.cuda.synchronize()
    return logits, argmax


def _first_argmax(logits):
    """torch.argmax's rule on bf16 rows, written out: the first index of the
    largest value, NaN largest (torch documents the first occurrence)."""
    values = logits.float()
    nan = torch.isnan(values)
    top = torch.where(nan.any(dim=1, keepdim=True), nan, values == values.max(dim=1, keepdim=True).values)
    return top.float().argmax(dim=1)  # first True


@pytest.mark.parametrize("rows,vocab,hidden", [(1, 151936, 1536), (2, 151936, 1536), (16, 4099, 1536),
                                               (5, 1000, 896), (3, 257, 128), (1, 33, 4096), (7, 2048, 3584)])
def test_lm_head_matches_fp64_and_argmax_is_torchs(rows, vocab, hidden):
    g = _gen(rows * 1000 + hidden)
    x = (torch.randn((rows, hidden), generator=g, device="cuda")).to(torch.bfloat16)
    weight = (torch.randn((vocab, hidden), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    logits, argmax = _lm_head(x, weight)
    exact = x.double() @ weight.double().T
    # fp32 sums of exact bf16 products, one bf16 rounding: within half a bf16
    # ulp of the exact value plus the fp32 summation error
    bound = exact.abs() * 2.0 ** -8 + 1e-5 * (x.double().abs() @ weight.double().abs().T)
    assert bool(((logits.double() - exact).abs() <= bound).all())
    assert torch.equal(argmax, logits.argmax(dim=1))
    assert torch.equal(argmax, _first_argmax(logits))
    # without the argmax: same logits, no workspace needed
    again, _ = _lm_head(x, weight, with_argmax=False)
    assert torch.equal(again, logits)


def test_lm_head_argmax_ties_and_nan():
    hidden, vocab = 256, 3000
    g = _gen(77)
    weight = (torch.randn((vocab, hidden), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    # rows 2900, 40 and 1999 equal the largest row: ties resolve to the first
    big = torch.full((hidden,), 0.5, dtype=torch.bfloat16, device="cuda")
    for v in (2900, 40, 1999):
        weight[v] = big
    x = torch.ones((4, hidden), dtype=torch.bfloat16, device="cuda")
    x[1] = -1.0  # all-negative ties: row 0 of the smallest weights wins instead
    x[2, 5] = float("nan")  # every logit NaN: index 0
    x[3] = 0.0  # every logit +0: index 0
    logits, argmax = _lm_head(x, weight)
    assert argmax[0].item() == 40
    assert torch.equal(argmax, _first_argmax(logits))
    assert argmax[2].item() == 0 and argmax[3].item() == 0


def test_lm_head_repeated_calls_share_the_workspace():
    """Back-to-back calls on one stream reuse one workspace."""
    lib = _lib.load()
    g = _gen(5)
    weight = (torch.randn((151936, 1536), generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    nbytes = lib.qwen2_lm_head_workspace_bytes(4, 151936, 1536)
    workspace = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    outs = []
    for seed in range(6):
        x = torch.randn((4, 1536), generator=_gen(seed), device="cuda").to(torch.bfloat16)
        logits = torch.empty((4, 151936), dtype=torch.bfloat16, device="cuda")
        argmax = torch.empty(4, dtype=torch.int64, device="cuda")
        _lib.check(lib.qwen2_lm_head(_p(x), _p(weight), _p(logits), _p(argmax), 4, 151936, 1536, _p(workspace),
                                     nbytes, _stream()))
        outs.append((logits, argmax))
    torch.cuda.synchronize()
    for logits, argmax in outs:
        assert torch.equal(argmax, logits.argmax(dim=1))


SMALL128 = SimpleNamespace(hidden_size=256, num_attention_heads=2, num_key_value_heads=1, head_dim=128,
                           intermediate_size=512, num_hidden_layers=3, vocab_size=512, rms_norm_eps=1e-6,
                           rope_theta=1_000_000.0)


def _build(config, seed):
    from qwen_int4_hip import QuantLinear, quantize_symmetric_rtn

    gen = _gen(seed)
    model = QwenInt4ForCausalLM(config, packing="canonical", group_size=64).cuda()
    with torch.no_grad():
        emb = model.model.embed_tokens.weight
        emb.copy_(torch.randn(emb.shape, generator=gen, device="cuda") * 0.02)
        for module in model.modules():
            if isinstance(module, QuantLinear):
                w = torch.randn((module.out_features, module.in_features), generator=gen, device="cuda") * 0.02
                q, s = quantize_symmetric_rtn(w, group_size=64)
                module.qweight.copy_(q)
                module.scales.copy_(s)
                if module.bias is not None:
                    module.bias.copy_(torch.randn(module.out_features, generator=gen, device="cuda") * 0.02)
    return model.eval()


def _cos(a, b):
    return torch.nn.functional.cosine_similarity(a.double().flatten(), b.double().flatten(), dim=0).item()


def test_fuse_projections_keeps_state_dict_and_eager_outputs():
    from qwen_int4_hip.decode import fuse_projections

    model = _build(SMALL128, 3)
    tokens = torch.randint(0, SMALL128.vocab_size, (1, 9), generator=torch.Generator().manual_seed(0)).cuda()
    with torch.inference_mode():
        before = model(tokens)
        state = {k: v.clone() for k, v in model.state_dict().items()}
        fused = fuse_projections(model)
        after = model(tokens)
    assert torch.equal(before, after)
    assert state.keys() == model.state_dict().keys()
    assert all(torch.equal(state[k], v) for k, v in model.state_dict().items())
    attn = model.model.layers[0].self_attn
    assert attn.k_proj.qweight.data_ptr() == attn.q_proj.qweight.data_ptr() + attn.q_proj.qweight.numel()
    assert fused[0]["qkv"]["out_features"] == 4 * 128 and fused[0]["gate_up"]["out_features"] == 1024
    # loading a state dict writes through the views into the fused buffers
    with torch.no_grad():
        sd = model.state_dict()
        sd["model.layers.0.self_attn.v_proj.scales"] = sd["model.layers.0.self_attn.v_proj.scales"] * 2
        model.load_state_dict(sd)
    assert torch.equal(fused[0]["qkv"]["scales"][384:], sd["model.layers.0.self_attn.v_proj.scales"])


@pytest.mark.parametrize("batch", [1, 2])
def test_fused_decode_step_matches_module_decode(batch):
    from qwen_int4_hip.generation import StaticGreedyDecoder

    model = _build(SMALL128, 11 + batch)
    prompt = torch.randint(0, SMALL128.vocab_size, (batch, 13), generator=torch.Generator().manual_seed(batch)).cuda()
    module = StaticGreedyDecoder(model, batch, 96, use_graph=False, fused=False)
    fused = StaticGreedyDecoder(model, batch, 96, use_graph=False, fused=True)
    graph = StaticGreedyDecoder(model, batch, 96, use_graph=True, fused=True)
    module.prefill(prompt)
    fused.prefill(prompt)
    graph.prefill(prompt)
    for step in range(70):  # crosses the 64-position chunk boundary of the attention kernel
        token = module.token.clone()
        want = module.step(token).clone()
        got = fused.step(token).clone()
        replay = graph.step(token).clone()
        assert torch.equal(got, replay), step  # graph replays run the same kernels on the same inputs
        assert _cos(got, want) >= 0.9999, (step, _cos(got, want))
        # the fused step's greedy choice is argmax of its own logits
        assert torch.equal(fused.token, got[:, -1].argmax(dim=-1, keepdim=True)), step
        assert torch.equal(graph.token, fused.token), step
    for (k0, v0), (k1, v1) in zip(module.caches, fused.caches):
        assert _cos(k0[:, :, :83], k1[:, :, :83]) >= 0.9999 and _cos(v0[:, :, :83], v1[:, :, :83]) >= 0.9999


def test_static_decoder_rejects_out_of_vocabulary_tokens():
    """Caller-supplied ids (a prompt, or the token given to step) outside
    [0, vocab) raise the reference embedding's IndexError before anything
    runs; the decoder's state is left as it was."""
    from qwen_int4_hip.generation import StaticGreedyDecoder

    model = _build(SMALL128, 23)
    dec = StaticGreedyDecoder(model, 1, 32, use_graph=True, fused=True)
    bad_prompt = torch.tensor([[1, SMALL128.vocab_size]], device="cuda")
    with pytest.raises(IndexError, match="index out of range"):
        dec.prefill(bad_prompt)
    dec.prefill(torch.tensor([[1, 2, 3]], device="cuda"))
    before = dec.token.clone()
    for bad in (-1, SMALL128.vocab_size):
        with pytest.raises(IndexError, match="index out of range"):
            dec.step(torch.tensor([[bad]], device="cuda"))
    assert dec.length == 3 and torch.equal(dec.token, before)
    logits = dec.step(torch.tensor([[SMALL128.vocab_size - 1]], device="cuda"))
    assert bool(torch.isfinite(logits.float()).all())


@pytest.mark.parametrize("batch,length", [(1, 40), (2, 17)])
def test_fused_prefill_matches_module_forward(batch, length):
    from qwen_int4_hip.decode import FusedPrefill

    model = _build(SMALL128, 5 + batch)
    prompt = torch.randint(0, SMALL128.vocab_size, (batch, length), generator=torch.Generator().manual_seed(7)).cuda()
    with torch.inference_mode():
        want, cache = model(prompt, use_cache=True)
        caches = model.new_static_cache(batch, 64, "cuda")
        got = FusedPrefill(model)(prompt, caches)
    assert got.shape == want.shape and _cos(got, want) >= 0.9999
    for (k0, v0), (k1, v1) in zip(cache, caches):
        assert _cos(k1[:, :, :length], k0) >= 0.9999 and _cos(v1[:, :, :length], v0) >= 0.9999
        assert not bool(k1[:, :, length:].any())  # positions past the prompt untouched


def test_full_width_fused_decode_against_reference_backend():
    """Qwen2-1.5B widths at 2 layers: the fused prefill and the fused
    graph-replayed decode steps stay within cosine 0.9999 of the model whose
    linears run the reference's torch backend (the oracle's restatement,
    backends.py:73-98)."""
    from test_model import QWEN2_1_5B, with_reference_linears

    from qwen_int4_hip.generation import StaticGreedyDecoder

    config = SimpleNamespace(num_hidden_layers=2, **QWEN2_1_5B)
    model = _build(config, 20260831)
    ref = with_reference_linears(model)
    prompt = torch.randint(0, config.vocab_size, (1, 64), generator=torch.Generator().manual_seed(4)).cuda()
    decoder = StaticGreedyDecoder(model, 1, 96)
    with torch.inference_mode():
        got = decoder.prefill(prompt)
        want, cache = ref(prompt, use_cache=True)
        assert _cos(got, want) >= 0.9999  # the fused prefill
        token = want[:, -1:].argmax(dim=-1)
        for _ in range(4):
            got = decoder.step(token)
            want, cache = ref(token, past_key_values=cache, use_cache=True)
            assert _cos(got, want) >= 0.9999
            token = want[:, -1:].argmax(dim=-1)
