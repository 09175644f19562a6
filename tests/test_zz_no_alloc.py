"""The allocation-free linear (w4g64_linear_static_scratch) against the
workspace one (w4g64_linear), through the C ABI.

It shares w4g64_linear's kernels and plans, so outputs must be bit-identical:
two calls in a row (the second on a smaller problem, so stale scratch from
the first would show), a split-K shape whose partial sums live in the
scratch, and a HIP graph of the allocation-free call replayed several times.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU"),
]

from qwen_int4_hip import _lib  # noqa: E402

DEV = "cuda"


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _problem(n, k, rows, seed, dtype):
    q, s, z = O.symmetric_weights(n, k, seed)
    x = O.activations(rows, k, seed=seed + 1, dtype=dtype)
    xt = (torch.from_numpy(x.view(np.int16)).view(torch.bfloat16) if dtype == "bf16" else torch.from_numpy(x)).to(DEV)
    return xt, torch.from_numpy(q).to(DEV), torch.from_numpy(s).to(DEV), torch.from_numpy(z).to(DEV)


def _code(x):
    return {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}[x.dtype]


def _with_workspace(lib, x, q, s, z, n, stream):
    rows, k = x.shape
    y = torch.empty((rows, n), dtype=x.dtype, device=DEV)
    need = lib.w4g64_linear_workspace_bytes(rows, n, k, _code(x))
    ws = torch.zeros(max(need, 16), dtype=torch.uint8, device=DEV)
    _lib.check(lib.w4g64_linear(_ptr(x), _code(x), _ptr(q), _ptr(s), _ptr(z), None, _lib.DTYPE_NONE, _ptr(y), rows,
                                n, k, _ptr(ws), ws.numel(), stream))
    return y


def _static(lib, x, q, s, z, n, stream, y=None):
    rows, k = x.shape
    y = torch.empty((rows, n), dtype=x.dtype, device=DEV) if y is None else y
    _lib.check(lib.w4g64_linear_static_scratch(_ptr(x), _code(x), _ptr(q), _ptr(s), _ptr(z), None, _lib.DTYPE_NONE,
                                               _ptr(y), rows, n, k, stream))
    return y


def test_static_scratch_matches_the_workspace_linear():
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.w4g64_static_scratch_bytes() == 4 << 20
    # split-K decode shape (down 1536x8960 at 4 rows: partials in the
    # scratch), then a smaller problem on the same scratch
    cases = [(1536, 8960, 4, "fp16"), (1536, 1536, 1, "fp16"), (2048, 1536, 16, "bf16"), (256, 1536, 3, "fp32")]
    for n, k, rows, dtype in cases:
        print(f"static scratch case n={n} k={k} rows={rows} {dtype}", flush=True)
        x, q, s, z = _problem(n, k, rows, O.BASE_SEED + n + rows, dtype)
        want = _with_workspace(lib, x, q, s, z, n, stream)
        for _ in range(2):
            got = _static(lib, x, q, s, z, n, stream)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16) if got.dtype != torch.float32 else got.view(torch.int32),
                               want.view(torch.int16) if want.dtype != torch.float32 else want.view(torch.int32))


def test_static_scratch_rejects_problems_beyond_its_size():
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    x, q, s, z = _problem(1536, 8960, 2048, O.BASE_SEED, "bf16")
    y = torch.empty((2048, 1536), dtype=torch.bfloat16, device=DEV)
    status = lib.w4g64_linear_static_scratch(_ptr(x), _lib.DTYPE_BF16, _ptr(q), _ptr(s), _ptr(z), None,
                                             _lib.DTYPE_NONE, _ptr(y), 2048, 1536, 8960, stream)
    if lib.w4g64_linear_workspace_bytes(2048, 1536, 8960, _lib.DTYPE_BF16) > lib.w4g64_static_scratch_bytes():
        assert status == _lib.STATUS_UNSUPPORTED and b"scratch" in lib.w4g64_last_error()
    else:
        assert status == _lib.STATUS_OK


def test_static_scratch_under_graph_capture():
    """The caller it exists for: a captured HIP graph of the allocation-free
    call (split-K partials in the scratch), replayed with eager calls of the
    same entry point in between; every replay equals the eager result."""
    lib = _lib.load()
    x, q, s, z = _problem(1536, 8960, 4, O.BASE_SEED + 77, "fp16")
    want = _with_workspace(lib, x, q, s, z, 1536, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    side = torch.cuda.Stream()
    out = torch.empty_like(want)
    with torch.cuda.stream(side):
        _static(lib, x, q, s, z, 1536, ctypes.c_void_p(side.cuda_stream), out)  # set-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        _static(lib, x, q, s, z, 1536, ctypes.c_void_p(side.cuda_stream), out)
    small = _problem(1536, 1536, 2, O.BASE_SEED + 78, "fp16")
    small_want = _with_workspace(lib, *small, 1536, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for replay in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {replay}"
        eager = _static(lib, *small, 1536, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        assert torch.equal(eager.view(torch.int16), small_want.view(torch.int16))
