"""CPU-side checks of the C ABI library and the host-side contract.

No GPU compute happens here: the library is loaded and every symbol the
header declares is resolved; the C layer's argument validation (which runs
before any launch) is exercised with null/misaligned pointers; the Python
layer's fail-closed validation mirrors the reference's rejection tests
(tests/test_backends.py:140-270, tests/test_triton_unpack.py:49-56, :75-90,
:122-130) on CPU tensors.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from qwen_int4_hip import _lib
from qwen_int4_hip.backends import SUPPORTED_BACKENDS, validate_canonical_w4g64_inputs
from qwen_int4_hip.linear import QuantLinear
from qwen_int4_hip.quantization import PackingFormat

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("*.h"))

pytestmark = pytest.mark.skipif(not _lib.library_built(), reason="HIP library not built (run __graft_entry__.build())")


def _declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b((?:w4g64|qwen2)_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    assert {h.name for h in HEADERS} == {"w4g64.h", "qwen2_decode.h"}
    declared = _declared_functions()
    assert declared, "no declarations parsed from include/*.h"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/*.h but not exported"
    assert set(declared) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert lib.w4g64_abi_version() == 3


def test_c_layer_rejects_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(64)
    p = ctypes.c_void_p(ctypes.addressof(buf))
    # bad activation dtype
    assert lib.w4g64_linear(p, 9, p, p, p, null, 0, p, 1, 64, 64, null, 0, null) == _lib.STATUS_INVALID_DTYPE
    assert b"dtype" in lib.w4g64_last_error()
    # in_features not a multiple of 64
    assert lib.w4g64_linear(p, 1, p, p, p, null, 0, p, 1, 64, 96, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert b"W4G64" in lib.w4g64_last_error()
    # null pointers
    assert lib.w4g64_linear(null, 1, p, p, p, null, 0, p, 1, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    # bias pointer without a bias dtype
    assert lib.w4g64_linear(p, 1, p, p, p, p, 0, p, 1, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    # misaligned activations
    odd = ctypes.c_void_p(ctypes.addressof(buf) | 1)
    assert lib.w4g64_linear(odd, 1, p, p, p, null, 0, p, 1, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert b"aligned" in lib.w4g64_last_error()
    # unpack element range
    assert lib.w4g64_unpack_canonical_int4(p, 4, p, 9, null) == _lib.STATUS_INVALID_VALUE
    assert b"elements" in lib.w4g64_last_error()
    assert lib.w4g64_unpack_canonical_int4(p, 4, p, 0, null) == _lib.STATUS_OK
    # dequant K not divisible by 64
    assert lib.w4g64_dequantize_canonical(p, p, p, p, 1, 96, null) == _lib.STATUS_INVALID_VALUE
    assert b"divisible" in lib.w4g64_last_error()


def test_decode_step_entry_points_reject_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.c_void_p((ctypes.addressof(buf) + 15) & ~15)
    f = ctypes.c_float
    # add_rmsnorm: hidden bounds, delta dtype, null pointers; zero rows is a no-op
    assert lib.qwen2_add_rmsnorm(p, null, 0, p, f(1e-6), p, p, 1, 0, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_add_rmsnorm(p, null, 0, p, f(1e-6), p, p, 1, 8200, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_add_rmsnorm(p, null, 0, p, f(1e-6), p, p, 1, 100, null) == _lib.STATUS_INVALID_VALUE
    odd2 = ctypes.c_void_p(p.value + 2)
    assert lib.qwen2_add_rmsnorm(odd2, null, 0, p, f(1e-6), p, p, 1, 64, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_add_rmsnorm(p, p, _lib.DTYPE_F16, p, f(1e-6), p, p, 1, 64, null) == _lib.STATUS_INVALID_DTYPE
    assert lib.qwen2_add_rmsnorm(null, null, 0, p, f(1e-6), p, p, 1, 64, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_add_rmsnorm(null, null, 0, null, f(1e-6), null, null, 0, 64, null) == _lib.STATUS_OK
    # decode-step prologue: head_dim, hidden, vocab, null and misaligned pointers; an empty batch is a no-op
    pro = [p] * 7 + [p, f(1e-6), p]  # ids .. sin, norm_weight, eps, normed
    assert lib.qwen2_decode_prologue(*pro, 1, 1536, 100, 64, null) == _lib.STATUS_UNSUPPORTED
    assert lib.qwen2_decode_prologue(*pro, 1, 1530, 100, 128, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_prologue(*pro, 1, 1536, 0, 128, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_prologue(null, *pro[1:], 1, 1536, 100, 128, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_prologue(p, odd2, *pro[2:], 1, 1536, 100, 128, null) == _lib.STATUS_INVALID_VALUE
    half = [p] * 7 + [p, f(1e-6), null]  # a norm weight without an output
    assert lib.qwen2_decode_prologue(*half, 1, 1536, 100, 128, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_prologue(*[null] * 7, null, f(1e-6), null, 0, 1536, 100, 128, null) == _lib.STATUS_OK
    # attention: head_dim, head grouping, workspace, alignment
    ws = lib.qwen2_decode_attention_workspace_bytes(1, 2, 640)
    assert ws == 256 + 1 * 2 * 10 * (16 + 8 * 128) * 4
    assert lib.qwen2_decode_attention_workspace_bytes(0, 2, 640) == 0
    args = [p] * 7
    assert lib.qwen2_decode_attention(*args, 1, 12, 2, 64, 640, f(0.1), p, ws, null) == _lib.STATUS_UNSUPPORTED
    assert lib.qwen2_decode_attention(*args, 1, 12, 5, 128, 640, f(0.1), p, ws, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_attention(*args, 1, 18, 2, 128, 640, f(0.1), p, ws, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_attention(*args, 1, 12, 2, 128, 640, f(0.1), p, ws - 4, null) == _lib.STATUS_WORKSPACE
    assert lib.qwen2_decode_attention(*args, 1, 12, 2, 128, 17409, f(0.1), p, 1 << 30,
                                      null) == _lib.STATUS_INVALID_VALUE
    odd = ctypes.c_void_p(p.value + 2)
    assert lib.qwen2_decode_attention(p, p, p, odd, p, p, p, 1, 12, 2, 128, 640, f(0.1), p, ws,
                                      null) == _lib.STATUS_INVALID_VALUE
    assert b"aligned" in lib.w4g64_last_error()
    # the merge stores four bf16 outputs at once and loads the partial sums 16 bytes at a time
    odd4 = ctypes.c_void_p(p.value + 4)
    assert lib.qwen2_decode_attention(p, p, p, p, p, p, odd4, 1, 12, 2, 128, 640, f(0.1), p, ws,
                                      null) == _lib.STATUS_INVALID_VALUE
    assert b"out must be 8-byte aligned" in lib.w4g64_last_error()
    assert lib.qwen2_decode_attention(*args, 1, 12, 2, 128, 640, f(0.1), odd4, ws, null) == _lib.STATUS_WORKSPACE
    assert b"16-byte aligned" in lib.w4g64_last_error()
    # prefill attention: head_dim, grouping, length vs cache, workspace, alignment
    pws = lib.qwen2_prefill_attention_workspace_bytes(1, 12, 512)
    assert pws == 12 * 512 * 128 * 2
    assert lib.qwen2_prefill_attention_workspace_bytes(1, 12, 0) == 0
    pargs = [p] * 6
    assert lib.qwen2_prefill_attention(*pargs, 1, 512, 12, 2, 64, 640, f(0.1), p, pws, null) == _lib.STATUS_UNSUPPORTED
    assert lib.qwen2_prefill_attention(*pargs, 1, 512, 12, 5, 128, 640, f(0.1), p, pws,
                                       null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_prefill_attention(*pargs, 1, 641, 12, 2, 128, 640, f(0.1), p, 1 << 30,
                                       null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_prefill_attention(*pargs, 1, 512, 12, 2, 128, 640, f(0.1), p, pws - 2,
                                       null) == _lib.STATUS_WORKSPACE
    assert lib.qwen2_prefill_attention(p, p, p, odd, p, p, 1, 512, 12, 2, 128, 640, f(0.1), p, pws,
                                       null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_prefill_attention(*pargs, 0, 512, 12, 2, 128, 640, f(0.1), null, 0, null) == _lib.STATUS_OK
    # silu_mul
    assert lib.qwen2_silu_mul(p, p, 1, 0, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_silu_mul(null, p, 1, 64, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_silu_mul(null, null, 0, 64, null) == _lib.STATUS_OK
    # lm_head: rows <= 16, hidden a multiple of 128 up to 4096, workspace for the argmax
    hws = lib.qwen2_lm_head_workspace_bytes(1, 151936, 1536)
    assert hws == 1 * (151936 // 16) * 8  # one tile of 16 vocab rows per workgroup up to 8 rows
    assert lib.qwen2_lm_head_workspace_bytes(2, 1000, 4096) == 2 * 63 * 8
    assert lib.qwen2_lm_head_workspace_bytes(16, 1000, 1536) == 16 * 32 * 8  # two tiles above 8 rows
    assert lib.qwen2_lm_head_workspace_bytes(16, 1000, 2560) == 16 * 63 * 8  # one where two do not fit
    assert lib.qwen2_lm_head_workspace_bytes(17, 1000, 1536) == 0
    assert lib.qwen2_lm_head_workspace_bytes(1, 1000, 100) == 0
    i64 = ctypes.cast(p, ctypes.c_void_p)
    assert lib.qwen2_lm_head(p, p, p, i64, 17, 1000, 1536, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(p, p, p, i64, 1, 1000, 1000, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(p, p, p, i64, 1, 1000, 4224, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(p, p, p, i64, 1, 0, 1536, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(p, null, p, i64, 1, 1000, 1536, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(odd, p, p, i64, 1, 1000, 1536, p, 1 << 20, null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_lm_head(p, p, p, i64, 1, 151936, 1536, p, hws - 8, null) == _lib.STATUS_WORKSPACE
    assert lib.qwen2_lm_head(p, p, p, i64, 1, 151936, 1536, null, hws, null) == _lib.STATUS_WORKSPACE
    assert lib.qwen2_lm_head(null, null, null, null, 0, 1000, 1536, null, 0, null) == _lib.STATUS_OK


def test_fused_swiglu_linear_rejects_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(buf) + 255) & ~255
    p = ctypes.c_void_p(base)
    f = ctypes.c_float
    # swiglu linear: rows range, alignment, bias agreement
    assert lib.w4g64_linear_swiglu(p, p, p, p, null, 0, p, 0, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert lib.w4g64_linear_swiglu(ctypes.c_void_p(base + 8), p, p, p, null, 0, p, 1, 64, 64, null, 0,
                                   null) == _lib.STATUS_INVALID_VALUE
    assert lib.w4g64_linear_swiglu(p, p, p, p, p, 0, p, 1, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    # the fused forms are valid workspace / kernel-name queries for decode rows only
    assert lib.w4g64_linear_kernel_name(1, 1536, 8960, _lib.DTYPE_BF16_SWIGLU).decode().startswith(
        "gemv_kernel<swiglu_bf16,")
    assert lib.w4g64_linear_kernel_name(12, 1536, 8960, _lib.DTYPE_BF16_SWIGLU).decode().startswith(
        "gemv_kernel<swiglu_bf16,")
    assert lib.w4g64_linear_kernel_name(64, 1536, 8960, _lib.DTYPE_BF16_SWIGLU).startswith(b"gemm_kernel<")
    assert lib.w4g64_linear_workspace_bytes(512, 1536, 8960, _lib.DTYPE_BF16_SWIGLU) == \
        lib.w4g64_linear_workspace_bytes(512, 1536, 8960, _lib.DTYPE_F32)
    assert lib.w4g64_linear_workspace_bytes(1, 64, 64, 4) == 0 and lib.w4g64_linear_kernel_name(1, 64, 64, 4) == b"none"
    assert lib.w4g64_linear_workspace_bytes(1, 1536, 8960, _lib.DTYPE_BF16_SWIGLU) == \
        lib.w4g64_linear_workspace_bytes(1, 1536, 8960, _lib.DTYPE_F32)


def test_gate_up_planes_and_planes_form_reject_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(buf) + 255) & ~255
    p = ctypes.c_void_p(base)
    gate_up = lib.w4g64_linear_gate_up_planes
    # rows 1..16 only; out_features even (gate rows then up rows); x aligned; bias agreement
    assert gate_up(p, p, p, p, null, 0, p, 17, 128, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert gate_up(p, p, p, p, null, 0, p, 0, 128, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert gate_up(p, p, p, p, null, 0, p, 1, 127, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert "even" in lib.w4g64_last_error().decode()
    assert gate_up(ctypes.c_void_p(base + 8), p, p, p, null, 0, p, 1, 128, 64, null, 0, null) == \
        _lib.STATUS_INVALID_VALUE
    assert gate_up(p, p, p, p, p, 0, p, 1, 128, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    # the planes activation form of w4g64_linear: 1..16 rows, fp32-aligned output
    planes = _lib.DTYPE_BF16_PLANES
    assert lib.w4g64_linear(p, planes, p, p, p, null, 0, p, 17, 64, 64, null, 0, null) == _lib.STATUS_INVALID_VALUE
    assert lib.w4g64_linear(p, planes, p, p, p, null, 0, ctypes.c_void_p(base + 2), 1, 64, 64, null, 0,
                            null) == _lib.STATUS_INVALID_VALUE
    # queries: decode rows only.  One row runs the pipelined kernel: the planes
    # are 3 staged rows, two segments of 7 steps of one pair each per wave, so
    # the 1536 x 8960 down projection (70 pairs) splits K 5 ways (fp32
    # partials) and its workspace is the larger need of the two decode
    # kernels (the other splits 6 ways); the paired gate|up needs no split.
    # Two rows run the earlier kernels.
    assert lib.w4g64_linear_kernel_name(1, 1536, 8960, planes) == b"gemv_pipe_kernel<planes_bf16,2,1,4,1,1,7,4>"
    assert lib.w4g64_linear_partial_count(1, 1536, 8960, planes) == 5
    assert lib.w4g64_linear_workspace_bytes(1, 1536, 8960, planes) == 6 * 1536 * 4
    assert lib.w4g64_linear_kernel_name(1, 17920, 1536, _lib.DTYPE_BF16_GATE_UP) == \
        b"gemv_pipe_kernel<bf16_gate_up,4,1,4,1,2,3,3>"
    assert lib.w4g64_linear_workspace_bytes(1, 17920, 1536, _lib.DTYPE_BF16_GATE_UP) == 0
    assert lib.w4g64_linear_kernel_name(2, 1536, 8960, planes) == b"gemv_kernel<planes_bf16,2,9,1>"
    assert lib.w4g64_linear_partial_count(2, 1536, 8960, planes) == 10
    assert lib.w4g64_linear_kernel_name(4, 17920, 1536, _lib.DTYPE_BF16_GATE_UP) == b"gemv_kernel<bf16,4,6,1>"
    assert lib.w4g64_linear_kernel_name(17, 1536, 8960, planes) == b"none"
    assert lib.w4g64_linear_workspace_bytes(17, 17920, 1536, _lib.DTYPE_BF16_GATE_UP) == 0
    # the fused RMSNorm linear: one row, bf16/fp32 delta, out_sum apart from the residual, even planes rows
    rn = lib.w4g64_linear_rmsnorm
    f = ctypes.c_float(1e-6)
    other = ctypes.c_void_p(base + 4096)
    assert rn(p, p, _lib.DTYPE_BF16, p, f, other, p, p, p, null, 0, p, 0, 2, 128, 64, null, 0, null) == \
        _lib.STATUS_INVALID_VALUE
    assert rn(p, p, _lib.DTYPE_F16, p, f, other, p, p, p, null, 0, p, 0, 1, 128, 64, null, 0, null) == \
        _lib.STATUS_INVALID_DTYPE
    assert rn(p, p, _lib.DTYPE_BF16, p, f, ctypes.c_void_p(base + 64), p, p, p, null, 0, p, 0, 1, 128, 64, null, 0,
              null) == _lib.STATUS_INVALID_VALUE
    assert "overlap" in lib.w4g64_last_error().decode()
    assert rn(p, p, _lib.DTYPE_F32, p, f, other, p, p, p, null, 0, p, 1, 1, 127, 64, null, 0, null) == \
        _lib.STATUS_INVALID_VALUE
    assert rn(p, null, _lib.DTYPE_F32, p, f, other, p, p, p, null, 0, p, 0, 1, 128, 64, null, 0, null) == \
        _lib.STATUS_INVALID_VALUE
    # 9..16 rows pair inside the segmented kernel (one segment per wave)
    assert lib.w4g64_linear_kernel_name(16, 17920, 1536, _lib.DTYPE_BF16_GATE_UP).startswith(b"gemv_kernel<bf16,1,")


def test_partial_sum_forms_reject_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(buf) + 255) & ~255
    p = ctypes.c_void_p(base)
    f = ctypes.c_float(1e-6)
    planes = _lib.DTYPE_BF16_PLANES
    # the decode down projection (1 row, planes) splits K; more rows, other
    # activation kinds or GEMM rows do not take the form
    count = lib.w4g64_linear_partial_count(1, 1536, 8960, planes)
    assert 2 <= count <= 8
    assert lib.w4g64_linear_partial_count(1, 1536, 8960, _lib.DTYPE_F32) >= 1
    assert lib.w4g64_linear_partial_count(17, 1536, 8960, planes) == 0
    assert lib.w4g64_linear_partial_count(1, 1536, 8960, _lib.DTYPE_BF16) == 0
    assert lib.w4g64_linear_partial_count(0, 1536, 8960, planes) == 0
    assert lib.w4g64_linear_partial_count(1, 1536, 100, planes) == 0
    need = count * 1536 * 4
    assert lib.w4g64_linear_partials(p, _lib.DTYPE_BF16, p, p, p, p, need, 1, 1536, 8960,
                                     null) == _lib.STATUS_INVALID_DTYPE
    assert lib.w4g64_linear_partials(p, planes, p, p, p, p, 1 << 30, 17, 1536, 8960, null) == _lib.STATUS_UNSUPPORTED
    assert lib.w4g64_linear_partials(p, planes, p, p, p, p, need - 4, 1, 1536, 8960,
                                     null) == _lib.STATUS_INVALID_VALUE
    assert b"partial sums" in lib.w4g64_last_error()
    assert lib.w4g64_linear_partials(ctypes.c_void_p(base + 8), planes, p, p, p, p, need, 1, 1536, 8960,
                                     null) == _lib.STATUS_INVALID_VALUE
    assert lib.w4g64_linear_partials(null, planes, p, p, p, p, need, 1, 1536, 8960, null) == _lib.STATUS_INVALID_VALUE
    # the residual-delta code: 1..255 parts; the fused norm linear adds at most 8
    assert _lib.dtype_f32_partials(6) == 0x106
    with pytest.raises(ValueError):
        _lib.dtype_f32_partials(0)
    assert lib.qwen2_add_rmsnorm(p, p, 0x200, p, f, p, p, 1, 1536, null) == _lib.STATUS_INVALID_DTYPE
    assert lib.w4g64_linear_rmsnorm(p, p, _lib.dtype_f32_partials(9), p, f, ctypes.c_void_p(base + 4096), p, p, p,
                                    null, 0, p, 0, 1, 64, 64, null, 0, null) == _lib.STATUS_UNSUPPORTED
    assert lib.w4g64_linear_rmsnorm(p, p, 0x300, p, f, ctypes.c_void_p(base + 4096), p, p, p, null, 0, p, 0, 1, 64,
                                    64, null, 0, null) == _lib.STATUS_INVALID_DTYPE


def test_attention_merge_forms_reject_before_launch():
    lib = _lib.load()
    null = None
    buf = ctypes.create_string_buffer(1 << 16)
    base = (ctypes.addressof(buf) + 255) & ~255
    p = ctypes.c_void_p(base)
    f = ctypes.c_float(128 ** -0.5)
    big = 1 << 40  # workspace bytes claimed, so that the checks after the size one are reached
    need = lib.qwen2_decode_attention_workspace_bytes(1, 2, 640)

    def merge(ws=p, ws_bytes=big, max_length=640, heads=12, kv=2, rows=1, n=1536):
        return lib.w4g64_linear_attention_merge(ws, ws_bytes, max_length, heads, kv, p, p, p, null, 0, p, rows, n,
                                                null)

    assert merge(rows=2) == _lib.STATUS_INVALID_VALUE and b"one row" in lib.w4g64_last_error()
    assert merge(heads=12, kv=5) == _lib.STATUS_INVALID_VALUE
    assert merge(heads=18, kv=2) == _lib.STATUS_INVALID_VALUE  # 9 query heads per key/value head
    assert merge(max_length=0) == _lib.STATUS_INVALID_VALUE
    assert merge(ws_bytes=need - 4) == _lib.STATUS_WORKSPACE
    assert merge(ws=ctypes.c_void_p(base + 8)) == _lib.STATUS_WORKSPACE
    assert merge(ws=null) == _lib.STATUS_WORKSPACE
    # 17 chunks, 14 heads (1792 features), 3 heads (384: not a multiple of 256)
    for kwargs in ({"max_length": 1025}, {"heads": 14, "kv": 2}, {"heads": 3, "kv": 3}):
        assert merge(**kwargs) == _lib.STATUS_UNSUPPORTED, kwargs
        assert b"qwen2_decode_attention and w4g64_linear" in lib.w4g64_last_error()
    # the unmerged attention: qwen2_decode_attention's checks, without `out`
    assert lib.qwen2_decode_attention_partials(p, p, p, p, p, p, 1, 12, 2, 128, 20000, f, p, big,
                                               null) == _lib.STATUS_INVALID_VALUE
    assert lib.qwen2_decode_attention_partials(p, p, p, p, p, p, 1, 12, 2, 64, 640, f, p, big,
                                               null) == _lib.STATUS_UNSUPPORTED
    assert lib.qwen2_decode_attention_partials(p, p, p, p, p, p, 1, 12, 2, 128, 640, f, null, 0,
                                               null) == _lib.STATUS_WORKSPACE
    assert lib.qwen2_decode_attention_partials(p, p, p, p, p, p, 1, 12, 2, 128, 640, f, p, need - 16,
                                               null) == _lib.STATUS_WORKSPACE


def test_workspace_and_kernel_plan_queries():
    lib = _lib.load()
    # decode shapes that split K across workgroups need a workspace for their
    # fp32 partials [splits][rows][out_features]; 9..16 rows stage the K
    # range's activations in LDS (~60 KB: at most 28 groups at 16 rows), so
    # long K splits across workgroups (140 groups -> 5 splits of 28; 145
    # groups -> 6 of 25); short K needs no workspace
    assert lib.w4g64_linear_workspace_bytes(4, 1536, 8960, _lib.DTYPE_F16) % (4 * 1536 * 4) == 0
    assert lib.w4g64_linear_workspace_bytes(4, 1536, 8960, _lib.DTYPE_F16) >= 2 * 4 * 1536 * 4
    assert lib.w4g64_linear_workspace_bytes(16, 1536, 8960, _lib.DTYPE_F16) == 5 * 16 * 1536 * 4
    assert lib.w4g64_linear_workspace_bytes(16, 1536, 1536, _lib.DTYPE_F16) == 0
    assert lib.w4g64_linear_workspace_bytes(16, 40, 9280, _lib.DTYPE_BF16) == 6 * 16 * 40 * 4
    # prefill: 560 tiles of 128x256 on 512 workgroup slots (256 CUs, the default
    # when no device answers): 512 data-parallel tiles, the other 48 split in 3
    # K ranges with fp32 partials; whole rounds need none
    # and every GEMM stages its activations as fp16 rows (rows x in_features x 2 B)
    # plus one fp32 row factor per tile row
    staged = 2048 * 1536 * 2 + 16 * 128 * 4
    assert lib.w4g64_linear_workspace_bytes(2048, 8960, 1536, _lib.DTYPE_BF16) == 48 * 3 * 128 * 256 * 4 + staged
    assert lib.w4g64_linear_workspace_bytes(2048, 8192, 1536, _lib.DTYPE_BF16) == staged
    # fp32 GEMM activations: two fp16 planes (rows x 2 in_features x 2 B) after the partials
    ws32 = lib.w4g64_linear_workspace_bytes(512, 1536, 8960, _lib.DTYPE_F32)
    assert 512 * 8960 * 4 + 512 * 4 <= ws32 <= (64 << 20) + 512 * 8960 * 4 + 512 * 4 + 512
    assert lib.w4g64_linear_kernel_name(512, 1536, 8960, _lib.DTYPE_F32).startswith(b"gemm_kernel<")
    assert lib.w4g64_linear_workspace_bytes(1, 1536, 100, _lib.DTYPE_F16) == 0
    # fp16 / bf16 decode rows with in_features a multiple of 256: the pipelined
    # GEMV, its launch shape by rows, K and out_features (no workspace unless
    # K is split across workgroups)
    assert lib.w4g64_linear_kernel_name(1, 8960, 1536, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16,4,1,4,1,1,3,3>"
    assert lib.w4g64_linear_kernel_name(1, 1536, 1536, _lib.DTYPE_BF16) == b"gemv_pipe_kernel<bf16,8,1,4,1,1,2,2>"
    assert lib.w4g64_linear_kernel_name(1, 256, 1536, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16,4,1,1,3,1,1,1>"
    assert lib.w4g64_linear_kernel_name(1, 501760, 1536, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16,4,1,4,1,2,3,3>"
    assert lib.w4g64_linear_workspace_bytes(1, 8960, 1536, _lib.DTYPE_F16) == 0
    assert lib.w4g64_linear_kernel_name(1, 1536, 8960, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16,8,1,4,1,1,9,5>"
    assert lib.w4g64_linear_kernel_name(4, 1536, 1536, _lib.DTYPE_BF16) == b"gemv_pipe_kernel<bf16,2,1,2,2,1,3,3>"
    assert lib.w4g64_linear_kernel_name(8, 1536, 8960, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16,1,1,1,7,1,2,2>"
    assert lib.w4g64_linear_kernel_name(16, 1536, 8960, _lib.DTYPE_BF16) == b"gemv_pipe_kernel<bf16_grouped,1,1,2,7,1,2,1>"
    assert lib.w4g64_linear_kernel_name(16, 8960, 1536, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16_grouped,1,1,4,2,1,6,2>"
    assert lib.w4g64_linear_kernel_name(16, 1536, 1536, _lib.DTYPE_F16) == b"gemv_pipe_kernel<f16_grouped,1,1,1,12,1,1,1>"
    # the down projection at 16 rows splits K in 5 (span 14 pairs): fp32 partial sums
    assert lib.w4g64_linear_workspace_bytes(16, 1536, 8960, _lib.DTYPE_F16) >= 5 * 16 * 1536 * 4
    # other K: one row of even-group shapes takes the lean kernel, the rest the
    # segmented kernel (9..16 fp16/bf16 rows: the 16-row kernel)
    assert lib.w4g64_linear_kernel_name(1, 256, 640, _lib.DTYPE_F16) == b"gemv_seg_kernel<f16,4,1,4,1>"
    assert lib.w4g64_linear_kernel_name(1, 64, 192, _lib.DTYPE_F16).startswith(b"gemv_kernel<f16")
    assert lib.w4g64_linear_kernel_name(4, 256, 640, _lib.DTYPE_BF16).startswith(b"gemv_kernel<bf16")
    assert lib.w4g64_linear_kernel_name(16, 40, 9280, _lib.DTYPE_BF16).startswith(b"gemv16_kernel<bf16")
    assert lib.w4g64_linear_kernel_name(16, 1536, 8960, _lib.DTYPE_F32).startswith(b"gemv_kernel<f32")
    assert lib.w4g64_linear_kernel_name(2048, 8960, 1536, _lib.DTYPE_BF16).startswith(b"gemm_kernel<")
    # 8-wave workgroups only for unsplit launches of at most one workgroup per CU (256 CUs)
    assert b"8 waves" in lib.w4g64_linear_kernel_name(512, 8960, 1536, _lib.DTYPE_BF16)  # 140 tiles
    assert b"8 waves" in lib.w4g64_linear_kernel_name(512, 8960, 1536, _lib.DTYPE_F32)
    assert b"8 waves" not in lib.w4g64_linear_kernel_name(2048, 8960, 1536, _lib.DTYPE_BF16)  # 560 tiles
    assert b"8 waves" not in lib.w4g64_linear_kernel_name(128, 8960, 1536, _lib.DTYPE_BF16)  # K split
    assert b"8 waves" not in lib.w4g64_linear_kernel_name(512, 1536, 8960, _lib.DTYPE_BF16)  # K split
    assert lib.w4g64_linear_kernel_name(1, 8960, 1536, 8) == b"none"


def test_status_mapping_uses_reference_exception_types():
    lib = _lib.load()
    lib.w4g64_linear(None, 9, None, None, None, None, 0, None, 1, 64, 64, None, 0, None)
    with pytest.raises(TypeError, match="dtype"):
        _lib.check(_lib.STATUS_INVALID_DTYPE)
    with pytest.raises(ValueError):
        _lib.check(_lib.STATUS_INVALID_VALUE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.STATUS_HIP_ERROR)


# ---- Python layer: fail-closed contract checks (CPU tensors suffice) -------

def _tensors(out_features=6, in_features=128):
    groups = in_features // 64
    return (
        torch.zeros(out_features * in_features // 2, 1, dtype=torch.uint8),
        torch.ones(out_features, groups, dtype=torch.float16),
        torch.zeros((out_features * groups + 1) // 2, 1, dtype=torch.uint8),
    )


def _validate(x, q, s, z, b=None, **over):
    args = dict(out_features=6, in_features=128, group_size=64, packing=PackingFormat.CANONICAL)
    args.update(over)
    return validate_canonical_w4g64_inputs(x, q, s, z, b, **args)


@pytest.mark.parametrize(
    ("override", "error", "message"),
    [
        ({"group_size": 128}, ValueError, "W4G64"),
        ({"packing": PackingFormat.LEGACY_SIGNED_ADD}, ValueError, "canonical INT4 packing"),
        ({"in_features": 64}, ValueError, "activation feature dimension"),
    ],
)
def test_rejects_incompatible_mapping(override, error, message):
    q, s, z = _tensors()
    with pytest.raises(error, match=message):
        _validate(torch.ones(1, 128, dtype=torch.bfloat16), q, s, z, **override)


@pytest.mark.parametrize("target", ["qweight", "scales", "zeros", "bias"])
def test_rejects_inconsistent_tensor_shapes(target):
    q, s, z = _tensors()
    tensors = {"qweight": q, "scales": s, "zeros": z, "bias": torch.zeros(6, dtype=torch.bfloat16)}
    tensors[target] = tensors[target][:-1]
    with pytest.raises(ValueError, match=target):
        _validate(torch.ones(1, 128, dtype=torch.bfloat16), tensors["qweight"], tensors["scales"],
                  tensors["zeros"], tensors["bias"])


@pytest.mark.parametrize(
    ("mutation", "error", "message"),
    [
        ("qweight_dtype", TypeError, "uint8"),
        ("zeros_dtype", TypeError, "uint8"),
        ("scales_dtype", TypeError, "FP16"),
        ("nonfinite_scale", ValueError, "finite"),
        ("nonpositive_scale", ValueError, "positive"),
        ("activation_dtype", TypeError, "FP16, BF16, or FP32"),
    ],
)
def test_rejects_malformed_metadata(mutation, error, message):
    q, s, z = _tensors()
    x = torch.ones(1, 128, dtype=torch.bfloat16)
    if mutation == "qweight_dtype":
        q = q.to(torch.int8)
    elif mutation == "zeros_dtype":
        z = z.to(torch.int8)
    elif mutation == "scales_dtype":
        s = s.to(torch.float32)
    elif mutation == "nonfinite_scale":
        s[0, 0] = float("nan")
    elif mutation == "nonpositive_scale":
        s[0, 0] = 0
    elif mutation == "activation_dtype":
        x = x.to(torch.float64)
    with pytest.raises(error, match=message):
        _validate(x, q, s, z)


def test_unknown_backend_is_rejected_and_registry_is_explicit():
    # tests/test_backends.py:140-143
    layer = QuantLinear(8, 4, group_size=4)
    with pytest.raises(ValueError):
        layer.set_backend("environment-variable-magic")
    assert SUPPORTED_BACKENDS == ("torch", "lpu", "triton", "hip")
    assert layer.backend == "hip"  # this package's default (the reference's is "torch")
    assert layer.qweight.shape == (16, 1) and layer.scales.shape == (4, 2) and layer.zeros.shape == (4, 1)
    assert QuantLinear(128, 6, group_size=64, bias=True).bias.dtype == torch.bfloat16


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU failure mode")
def test_hip_backend_fails_loudly_without_gpu():
    layer = QuantLinear(128, 64, group_size=64, packing=PackingFormat.CANONICAL)
    with pytest.raises(RuntimeError, match="HIP backend requires"):
        layer(torch.zeros(1, 128, dtype=torch.float16))


def test_workspace_growth_keeps_replaced_buffers_and_refuses_capture():
    """A captured HIP graph holds the raw address of the workspace it was
    captured with: growing the (device, stream) buffer must keep the old one
    alive, and growing during a capture must be refused."""
    from qwen_int4_hip import kernels

    key = ("cpu-test", 1)
    try:
        first = kernels._grow_workspace(key, 100, "cpu", capturing=False)
        assert first.numel() >= 100 and not bool(first.any())
        assert kernels._grow_workspace(key, 50, "cpu", capturing=True) is first  # fits: no allocation
        retired = len(kernels._retired)
        second = kernels._grow_workspace(key, first.numel() + 1, "cpu", capturing=False)
        assert second.numel() > first.numel() and second is not first
        assert kernels._retired[-1] is first and len(kernels._retired) == retired + 1
        with pytest.raises(RuntimeError, match="capture"):
            kernels._grow_workspace(key, second.numel() + 1, "cpu", capturing=True)
        with pytest.raises(RuntimeError, match="capture"):
            kernels._grow_workspace(("cpu-test", 2), 10, "cpu", capturing=True)
        assert kernels._workspaces[key] is second
    finally:
        kernels._workspaces.pop(key, None)
        kernels._workspaces.pop(("cpu-test", 2), None)


def test_fused_paths_reject_mismatched_caches_and_ids_on_the_host():
    """The fused decode step and prefill validate the caches they write, and
    the token ids, before any launch (the reference's attention rejects
    mismatched caches, src/qwen_int4/model.py:80-86)."""
    from qwen_int4_hip.decode import check_static_caches, check_token_ids

    def caches(n=2, shape=(1, 2, 16, 128), dtype=torch.bfloat16):
        return [(torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)) for _ in range(n)]

    ok = dict(layers=2, batch=1, kv_heads=2, head_dim=128, min_length=4, device="cpu")
    assert check_static_caches(caches(), **ok) == 16
    with pytest.raises(ValueError, match="one entry per decoder layer"):
        check_static_caches(caches(3), **ok)
    for bad in [(2, 2, 16, 128), (1, 1, 16, 128), (1, 2, 16, 64), (1, 2, 16)]:
        with pytest.raises(ValueError, match="cache shape does not match"):
            check_static_caches(caches(shape=bad), **ok)
    mixed = caches()
    mixed[1] = (mixed[1][0], torch.zeros((1, 2, 8, 128), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="cache shape does not match"):
        check_static_caches(mixed, **ok)
    with pytest.raises(ValueError, match="bfloat16"):
        check_static_caches(caches(dtype=torch.float16), **ok)
    strided = [(k.transpose(2, 3).contiguous().transpose(2, 3), v) for k, v in caches()]
    with pytest.raises(ValueError, match="contiguous"):
        check_static_caches(strided, **ok)
    with pytest.raises(ValueError, match="positions"):
        check_static_caches(caches(), **dict(ok, min_length=17))
    with pytest.raises(ValueError, match="attention device"):
        check_static_caches(caches(), **dict(ok, device="meta"))
    check_token_ids(torch.zeros((2, 5), dtype=torch.int64), batch=2, length=None, device="cpu")
    with pytest.raises(ValueError, match="shape"):
        check_token_ids(torch.zeros((1, 5), dtype=torch.int64), batch=2, length=None, device="cpu")
    with pytest.raises(ValueError, match="shape"):
        check_token_ids(torch.zeros((2, 2), dtype=torch.int64), batch=2, length=1, device="cpu", name="token_ids")
    with pytest.raises(ValueError, match="int64"):
        check_token_ids(torch.zeros((2, 1), dtype=torch.int32), batch=2, length=1, device="cpu")
