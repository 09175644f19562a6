#!/usr/bin/env python3
"""W4G64 linear benchmark on one MI355X: decode GEMV HBM GB/s and prefill GEMM
TFLOP/s, each as a fraction of the MI355X peak.

Decode workload (the `value` line): one step = the seven Qwen2-1.5B linear
shapes (q/k/v/o, gate/up/down) at activation rows 1, 4 and 16, fp16
activations N(0, 1), symmetric RTN W4G64 weights quantized from N(0, 0.02)
-- 21 linear calls.  Weights are replicated into distinct device copies
(~800 MB in total) and every call of a step reads a different copy, so the
256 MB Infinity Cache and the L2s cannot serve a repeat: the figure is HBM
throughput.  Each step is captured once as a HIP graph; the timed region
replays K step graphs back to back between two device synchronizations.
value = algorithmic bytes of the step / step time.

The roofline object is for the kernels that do the decode work (all 21
calls): each call's average launch duration is measured live the way the
step runs -- a HIP graph of 32 back-to-back launches of that call (rotating
over the weight copies), replayed between HIP events recorded on the replay
stream -- and agrees with the per-kernel durations rocprofv3 --kernel-trace
reports for graph replays; achieved = algorithmic bytes / summed average
durations.  (Launched one at a time with start/stop events of their own,
the same kernels measure ~0.6 us longer each.)

Algorithmic bytes per call (M rows, N out, K in):
    N*K/2 + 2*N*K/64 + N*K/128 + 2*M*K + 2*M*N
(packed codes, fp16 scales, packed zeros, fp16 activations, fp16 outputs).

The prefill GEMM (gate/up 8960x1536 and down 1536x8960 at rows 128/512/2048,
bf16) is reported in the "gemm" object with its own roofline (MFMA bound).

End to end ("e2e" object): the Qwen2-1.5B architecture with random-init
weights over the HIP linears, batch 1, a 512-token random prompt, then 128
greedy tokens with a static KV cache, each decode step one HIP graph replay:
prefill and decode tokens/s.

Weights and activations are generated on the GPU with the package's own
quantizer (the mirror of src/qwen_int4/quantization.py).  Protocol (the
reference harness's: scripts/autotune_phase_e_triton_v6.py:41-56, :96-113;
scripts/benchmark_phase_f_model.py:33-50): parity first -- every decode output
and the rows-2048 GEMM outputs of this run are checked against the CPU
restatement of the reference's torch backend (normwise relative error <=
1e-2) before anything is timed, on every run; then warm-up, the timed steps,
and medians and 95th percentiles over >= 100 samples per decode shape, per
decode step, per GEMM shape, and p50/p95 for the end-to-end prefill and
decode tokens.  The cpu_baseline leg times the same CPU restatement on the
host cores over a bounded sample of the decode steps, and the single
q_proj 1536x1536 call at M = 1 on its own.

HBM traffic (roofline "traffic"): `--profile-pass` runs, untimed, a
calibration kernel of exactly known traffic (the unpack kernel: reads P bytes,
writes 2P bytes), three decode steps on rotating weight copies and the M=2048
GEMMs, each group after a 1 GiB write that evicts the caches, for two
`rocprofv3 --pmc` runs (FETCH_SIZE, then WRITE_SIZE);
`--summarize-pmc FETCH_CSV WRITE_CSV` scales each counter by the calibration
kernel's reading and writes the per-launch traffic to profiles/pmc_traffic.json,
which later bench runs report.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
PACKAGE_ROOT = REPO_ROOT / "qwen2-int4-systems_amd"
for _path in (REPO_ROOT, PACKAGE_ROOT):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

METRIC = "W4G64 GEMV HBM GB/s (M=1) + GEMM TFLOP/s (M=2048), % of MI355X peak"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
DECODE_ROWS = (1, 4, 16)
PREFILL_ROWS = (128, 512, 2048)
PREFILL_SHAPES = ("gate_proj", "down_proj")
COPIES = 32  # distinct weight copies per shape (32 x 25.2 MB = 806 MB)
BASE_SEED = 20260831  # the reference's seed convention (tests/test_triton_unpack.py:42)
QWEN2_SHAPES = {  # (out_features, in_features), configs/qwen2-1.5b/config.json
    "q_proj": (1536, 1536),
    "k_proj": (256, 1536),
    "v_proj": (256, 1536),
    "o_proj": (1536, 1536),
    "gate_proj": (8960, 1536),
    "up_proj": (8960, 1536),
    "down_proj": (1536, 8960),
}
PMC_TRAFFIC_FILE = REPO_ROOT / "profiles" / "pmc_traffic.json"
CALIBRATION_PACKED_BYTES = 128 << 20  # unpack kernel: reads this, writes twice this
SCRUB_BYTES = 1 << 30  # written before each measured group: evicts the L2s and the 256 MB Infinity Cache


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def algorithmic_bytes(m: int, n: int, k: int, act_bytes: int = 2) -> int:
    return n * k // 2 + 2 * n * (k // 64) + n * (k // 64) // 2 + act_bytes * m * k + act_bytes * m * n


class Hip:
    """The few HIP runtime calls the harness needs (events, sync)."""

    def __init__(self) -> None:
        self.lib = ctypes.CDLL("libamdhip64.so")
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.lib.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.lib.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.lib.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]

    def event(self) -> ctypes.c_void_p:
        ev = ctypes.c_void_p()
        if self.lib.hipEventCreate(ctypes.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev

    def record(self, event, stream) -> None:
        if self.lib.hipEventRecord(event, stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, start, stop) -> float:
        self.lib.hipEventSynchronize(stop)
        ms = ctypes.c_float()
        if self.lib.hipEventElapsedTime(ctypes.byref(ms), start, stop) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(ms.value)


# ---------------------------------------------------------------------------
# Synthetic workload (generated on the GPU with the package's quantizer)
# ---------------------------------------------------------------------------

def gen_weights(n: int, k: int, seed: int, torch):
    """Symmetric RTN W4G64 of W ~ N(0, 0.02) (configs 0-2); zeros all 0, as
    scripts/quantize_model.py:127 builds them."""
    from qwen_int4_hip import quantize_symmetric_rtn

    gen = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    qweight, scales = quantize_symmetric_rtn(w, group_size=64)
    zeros = torch.zeros(((n * (k // 64) + 1) // 2, 1), dtype=torch.uint8, device="cuda")
    return qweight, scales, zeros


def gen_activations(rows: int, k: int, seed: int, dtype, torch):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn((rows, k), generator=gen, device="cuda", dtype=torch.float32).to(dtype)


def decode_cases(torch, copies_per_shape: int):
    """The decode step's 21 calls: base weights, device copies, activations."""
    base, copies = {}, {}
    for name, (n, k) in QWEN2_SHAPES.items():
        base[name] = gen_weights(n, k, BASE_SEED + n + k, torch)
        copies[name] = [tuple(t.clone() for t in base[name]) for _ in range(copies_per_shape)]
    cases = []
    for r_index, rows in enumerate(DECODE_ROWS):
        for s_index, (name, (n, k)) in enumerate(QWEN2_SHAPES.items()):
            x = gen_activations(rows, k, BASE_SEED + 1000 * rows + s_index, torch.float16, torch)
            cases.append({"name": name, "rows": rows, "n": n, "k": k, "x": x, "w": base[name],
                          "copies": copies[name], "copy0": r_index, "bytes": algorithmic_bytes(rows, n, k)})
    return base, copies, cases


def timed_call(lib, x, w, y, workspace, stream, events):
    from qwen_int4_hip import _lib

    q, s, z = w
    rows, k = x.shape
    n = y.shape[1]
    code = {"torch.float16": _lib.DTYPE_F16, "torch.bfloat16": _lib.DTYPE_BF16}[str(x.dtype)]
    _lib.check(lib.w4g64_linear_timed(
        ctypes.c_void_p(x.data_ptr()), code, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()),
        ctypes.c_void_p(z.data_ptr()), None, _lib.DTYPE_NONE, ctypes.c_void_p(y.data_ptr()), rows, n, k,
        None if workspace is None else ctypes.c_void_p(workspace.data_ptr()),
        0 if workspace is None else workspace.numel(), stream, events[0], events[1]))


def kernel_durations(cases, reps, hip, torch):
    """Per-case kernel durations (ms) from start/stop events recorded by the
    kernel launch itself; calls rotate over the weight copies."""
    from qwen_int4_hip import _lib
    from qwen_int4_hip.kernels import _workspace

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    pairs = [(hip.event(), hip.event()) for _ in range(len(cases) * reps)]
    outputs = []
    i = 0
    for rep in range(reps):
        for case in cases:
            x, copies, n = case["x"], case["copies"], case["n"]
            w = copies[(case["copy0"] + rep * 3) % len(copies)]
            y = torch.empty((x.shape[0], n), dtype=x.dtype, device="cuda")
            ws_bytes = lib.w4g64_linear_workspace_bytes(x.shape[0], n, x.shape[1],
                                                        _lib.DTYPE_F16 if x.dtype == torch.float16 else _lib.DTYPE_BF16)
            ws = _workspace(torch.device("cuda"), ws_bytes)
            timed_call(lib, x, w, y, ws, stream, pairs[i])
            outputs.append(y)
            i += 1
    torch.cuda.synchronize()
    durations = [[] for _ in cases]
    i = 0
    for rep in range(reps):
        for c in range(len(cases)):
            durations[c].append(hip.elapsed_ms(*pairs[i]))
            i += 1
    for a, b in pairs:
        hip.lib.hipEventDestroy(a)
        hip.lib.hipEventDestroy(b)
    return durations


def graph_kernel_durations(cases, reps, hip, torch, launches: int = 32):
    """Per-case average launch duration (ms), measured the way the decode step
    runs: one HIP graph per case holding `launches` back-to-back calls
    (rotating over the weight copies), replayed `reps` times between HIP
    events recorded on the replay stream; each sample is one replay's
    elapsed time / `launches`."""
    from qwen_int4_hip.kernels import linear_canonical_w4g64_hip

    side = torch.cuda.Stream()
    stream = ctypes.c_void_p(side.cuda_stream)
    durations = []
    with torch.cuda.stream(side):
        for case in cases:
            x, copies = case["x"], case["copies"]
            ws = [copies[(case["copy0"] + 3 * i) % len(copies)] for i in range(launches)]
            linear_canonical_w4g64_hip(x, *ws[0])  # workspace and kernel set-up outside capture
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for w in ws:
                    linear_canonical_w4g64_hip(x, *w)
            g.replay()
            events = [(hip.event(), hip.event()) for _ in range(reps)]
            for a, b in events:
                hip.record(a, stream)
                g.replay()
                hip.record(b, stream)
            torch.cuda.synchronize()
            durations.append([hip.elapsed_ms(a, b) / launches for a, b in events])
            for a, b in events:
                hip.lib.hipEventDestroy(a)
                hip.lib.hipEventDestroy(b)
            del g
    return durations


def replay_samples(run, reps: int, hip, torch):
    """Durations (ms) of `reps` calls of run(i), each between two HIP events
    recorded on the current stream (where graph replays launch)."""
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    events = [(hip.event(), hip.event()) for _ in range(reps)]
    for i, (a, b) in enumerate(events):
        hip.record(a, stream)
        run(i)
        hip.record(b, stream)
    torch.cuda.synchronize()
    out = [hip.elapsed_ms(a, b) for a, b in events]
    for a, b in events:
        hip.lib.hipEventDestroy(a)
        hip.lib.hipEventDestroy(b)
    return out


def dense_library_gemm_ms(cases, torch, reps: int = 12):
    """Median time (ms) of torch.matmul on each case's bf16 activations with a
    dense bf16 [K, N] weight of the same shape: the vendor GEMM library's rate
    on the same problem without dequantization (a calibration of what the
    shapes allow, not a parity reference)."""
    out = []
    for c in cases:
        x = c["x"]
        w = torch.randn((c["k"], c["n"]), device="cuda", dtype=torch.float32).to(x.dtype).contiguous()
        for _ in range(3):
            torch.matmul(x, w)
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for a, b in events:
            a.record()
            torch.matmul(x, w)
            b.record()
        torch.cuda.synchronize()
        out.append(statistics.median(a.elapsed_time(b) for a, b in events))
    return out


# ---------------------------------------------------------------------------
# Floors and the reference's own operator profiles
# ---------------------------------------------------------------------------

STREAM_FLOOR_BYTES = (7_434_240, 1_327_104, 212_992)  # gate/down M=1, q/o M=1, k/v M=1 (rounded to 4 KiB)


def _cold_pool_slices(torch, nbytes: int, pool_bytes: int = 640 << 20):
    """One device buffer of >= pool_bytes split into slices of nbytes (4 KiB
    aligned): graph launches that rotate over them read HBM, not the 256 MB
    Infinity Cache."""
    step = (nbytes + 4095) // 4096 * 4096
    count = max(32, -(-pool_bytes // step))
    pool = torch.empty(count * step, dtype=torch.uint8, device="cuda")
    pool.fill_(1)
    return pool, [pool[i * step: i * step + nbytes] for i in range(count)]


def stream_floor(torch, hip, reps: int = 50, launches: int = 32) -> list:
    """The bare-stream floor of a decode launch, measured the way the decode
    calls are: a HIP graph of `launches` back-to-back launches of the stream
    probe (w4g64_stream_probe: one 16-byte nontemporal load per lane over
    exactly the call's bytes, nothing else), rotating over a 640 MB pool,
    replayed between HIP events on the replay stream."""
    from qwen_int4_hip import _lib

    lib = _lib.load()
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    side = torch.cuda.Stream()
    sp = ctypes.c_void_p(side.cuda_stream)
    out = []
    for nbytes in STREAM_FLOOR_BYTES:
        pool, slices = _cold_pool_slices(torch, nbytes)
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            def probe(i):
                _lib.check(lib.w4g64_stream_probe(ctypes.c_void_p(slices[i % len(slices)].data_ptr()), nbytes,
                                                  ctypes.c_void_p(sink.data_ptr()), sp))
            probe(0)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for i in range(launches):
                    probe(7 * i)
            g.replay()
            events = [(hip.event(), hip.event()) for _ in range(reps)]
            for a, b in events:
                hip.record(a, sp)
                g.replay()
                hip.record(b, sp)
            torch.cuda.synchronize()
            d = [hip.elapsed_ms(a, b) * 1e3 / launches for a, b in events]
            for a, b in events:
                hip.lib.hipEventDestroy(a)
                hip.lib.hipEventDestroy(b)
            del g
        out.append({"bytes": nbytes, "us_p50": round(statistics.median(d), 3), "us_p95": round(percentile(d, 95), 3),
                    "GBps": round(nbytes / statistics.median(d) / 1e3, 1)})
        del pool, slices
        torch.cuda.empty_cache()
    return out


# The reference's operator autotune profiles (configs/phase-e-triton-autotune-v1.json:17-21) and the
# median kernel times its Triton kernel reached there (results/phase_e_triton_autotune_v1.json:18-56,
# RTX 4090, CUDA events; other hardware, shown for context only).
REFERENCE_PROFILES = (
    ("v_projection_fp16", 1, 256, 1536, "fp16", 0.01, 0.0625, 79.904),
    ("q_projection_bf16", 8, 1536, 1536, "bf16", 0.02, 0.25, 80.896),
    ("mlp_down_projection_fp16", 4, 1536, 8960, "fp16", 0.01, 0.0625, 325.568),
)


def awq_weights_gpu(n: int, k: int, seed: int, torch):
    """Asymmetric AWQ-style W4G64 drawn on the GPU (config 3): codes u in
    [0, 15] and per-group zero points in [4, 11] stored as signed u - 8,
    log-normal scales (mu = ln 0.003, sigma = 0.5) -- the distributions of an
    AWQ export, whose input-channel scales are already folded into the
    codes and scales (the kernels' work does not depend on the values)."""
    from qwen_int4_hip import pack_int4

    gen = torch.Generator(device="cuda").manual_seed(seed)
    codes = torch.randint(0, 16, (n, k), generator=gen, device="cuda", dtype=torch.int16) - 8
    zeros_u = torch.randint(4, 12, (n * (k // 64),), generator=gen, device="cuda", dtype=torch.int16) - 8
    scales = torch.exp(torch.randn((n, k // 64), generator=gen, device="cuda") * 0.5 + float(math.log(0.003)))
    return (pack_int4(codes.to(torch.int8)).reshape(n, k // 2), scales.to(torch.float16),
            pack_int4(zeros_u.to(torch.int8)).reshape(-1, 1))


def outlier_activations(rows: int, k: int, seed: int, dtype, torch):
    """x ~ N(0, 1) with 1 % of the channels scaled by 20 (config 3)."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((rows, k), generator=gen, device="cuda", dtype=torch.float32)
    channels = torch.randperm(k, generator=gen, device="cuda")[: max(1, k // 100)]
    x[:, channels] *= 20.0
    return x.to(dtype)


def _awq_cases(torch, specs, copies_bytes: int = 640 << 20):
    """Cases with cold weight copies for graph_kernel_durations: specs are
    (name, rows, n, k, dtype, seed)."""
    cases = []
    for name, rows, n, k, dtype, seed in specs:
        w = awq_weights_gpu(n, k, seed, torch)
        wbytes = sum(t.numel() * t.element_size() for t in w)
        ncopies = max(2, min(256, -(-copies_bytes // wbytes)))
        ncopies += ncopies % 3 == 0  # the replay visits copies with stride 3
        copies = [w] + [tuple(t.clone() for t in w) for _ in range(ncopies - 1)]
        x = outlier_activations(rows, k, seed + 1, dtype, torch)
        cases.append({"name": name, "rows": rows, "n": n, "k": k, "x": x, "w": w, "copies": copies, "copy0": 0,
                      "bytes": algorithmic_bytes(rows, n, k)})
    return cases


def _oracle_check(case, torch, rtol=None, atol=None) -> float:
    """Normwise relative error of the case's HIP output against the CPU
    restatement of the reference's torch backend (and the reference's own
    rtol/atol where given)."""
    from oracle import oracle as O
    from qwen_int4_hip import linear_canonical_w4g64_hip

    got = linear_canonical_w4g64_hip(case["x"], *case["w"]).float().cpu()
    x, q, s, z = case["x"].cpu(), *(t.cpu() for t in case["w"])
    ref = O.reference_linear_torch(x, q, s, z, None, out_features=case["n"], in_features=case["k"], return_f32=True)
    rel = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
    ok = bool(torch.isfinite(got).all()) and rel <= 1e-2
    if rtol is not None:
        ok = ok and bool(torch.allclose(got, ref, rtol=rtol, atol=atol))
    if not ok:
        raise SystemExit(f"parity failed for {case['name']} rows={case['rows']}: normwise relative error {rel:.3e}")
    return rel


def reference_profiles(torch, hip) -> list:
    """The reference's three operator profiles on AWQ-style weights, cold,
    graph-replayed as the decode calls are; median and p95 per launch."""
    out = []
    specs = [(name, m, n, k, torch.float16 if dt == "fp16" else torch.bfloat16, BASE_SEED + 31 * i)
             for i, (name, m, n, k, dt, *_rest) in enumerate(REFERENCE_PROFILES)]
    cases = _awq_cases(torch, specs)
    durations = graph_kernel_durations(cases, 100, hip, torch)
    from qwen_int4_hip import linear_kernel_name

    for case, d, prof in zip(cases, durations, REFERENCE_PROFILES):
        rel = _oracle_check(case, torch, rtol=prof[5], atol=prof[6])
        us = [v * 1e3 for v in d]
        p50 = statistics.median(us)
        gbs = case["bytes"] / p50 / 1e3
        out.append({"profile": prof[0], "shape_mnk": [case["rows"], case["n"], case["k"]], "dtype": prof[4],
                    "kernel": linear_kernel_name(case["rows"], case["n"], case["k"], case["x"].dtype),
                    "us_p50": round(p50, 3), "us_p95": round(percentile(us, 95), 3), "samples": len(us),
                    "GBps": round(gbs, 1), "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                                       "peak": HBM_PEAK_GBS, "frac": round(gbs / HBM_PEAK_GBS, 4)},
                    "parity_normwise_rel_err": rel, "parity_rtol_atol": [prof[5], prof[6]],
                    "reference_rtx4090_triton_median_us": prof[7]})
        log(f"  profile {prof[0]:26s} {case['rows']}x{case['n']}x{case['k']} {prof[4]}: p50 {p50:6.2f} us "
            f"(p95 {percentile(us, 95):6.2f}), {gbs:7.1f} GB/s; reference Triton on RTX 4090: {prof[7]:.1f} us")
    del cases
    torch.cuda.empty_cache()
    return out


def awq_config3(torch, hip, gemm_reps: int = 100) -> dict:
    """Config 3: asymmetric AWQ-style weights on the seven shapes at M = 1
    (cold, graph-replayed; GB/s) and M = 2048 (event-timed launches; TFLOP/s),
    fp16 activations with 1 % outlier channels x20; every M = 1 output and
    the q_proj M = 2048 output checked against the CPU oracle first."""
    from qwen_int4_hip import linear_kernel_name

    specs1 = [(name, 1, n, k, torch.float16, BASE_SEED + 101 + i) for i, (name, (n, k)) in enumerate(QWEN2_SHAPES.items())]
    cases1 = _awq_cases(torch, specs1)
    worst = max(_oracle_check(c, torch) for c in cases1)
    d1 = graph_kernel_durations(cases1, 100, hip, torch)
    rows1, tot_b, tot_us = [], 0, 0.0
    for c, d in zip(cases1, d1):
        us = statistics.fmean(d) * 1e3
        tot_b += c["bytes"]
        tot_us += us
        rows1.append({"name": c["name"], "n": c["n"], "k": c["k"], "kernel": linear_kernel_name(1, c["n"], c["k"], torch.float16),
                      "us_mean": round(us, 3), "us_p50": round(statistics.median(d) * 1e3, 3),
                      "us_p95": round(percentile(d, 95) * 1e3, 3), "GBps": round(c["bytes"] / us / 1e3, 1)})
    del cases1
    torch.cuda.empty_cache()
    specs2 = [(name, 2048, n, k, torch.float16, BASE_SEED + 201 + i) for i, (name, (n, k)) in enumerate(QWEN2_SHAPES.items())]
    cases2 = []
    for name, rows, n, k, dtype, seed in specs2:
        w = awq_weights_gpu(n, k, seed, torch)
        cases2.append({"name": name, "rows": rows, "n": n, "k": k, "x": outlier_activations(rows, k, seed + 1, dtype, torch),
                       "w": w, "copies": [w] + [tuple(t.clone() for t in w) for _ in range(3)], "copy0": 0})
    worst = max(worst, _oracle_check(cases2[0], torch))
    d2 = kernel_durations(cases2, gemm_reps, hip, torch)
    rows2, tot_f, tot_ms = [], 0.0, 0.0
    for c, d in zip(cases2, d2):
        ms = statistics.fmean(d)
        flops = 2.0 * c["rows"] * c["n"] * c["k"]
        tot_f += flops
        tot_ms += ms
        rows2.append({"name": c["name"], "n": c["n"], "k": c["k"], "kernel": linear_kernel_name(2048, c["n"], c["k"], torch.float16),
                      "us_mean": round(ms * 1e3, 2), "us_p50": round(statistics.median(d) * 1e3, 2),
                      "us_p95": round(percentile(d, 95) * 1e3, 2), "TFLOPs": round(flops / ms / 1e9, 1)})
    del cases2
    torch.cuda.empty_cache()
    m1 = tot_b / tot_us / 1e3
    m2048 = tot_f / tot_ms / 1e9
    log(f"config 3 (AWQ asymmetric, outliers): M=1 {m1:.1f} GB/s over 7 shapes ({tot_us:.1f} us); "
        f"M=2048 {m2048:.1f} TFLOP/s over 7 shapes ({tot_ms * 1e3:.1f} us)")
    return {"workload": "config 3: asymmetric AWQ-style W4G64 (codes 0..15, zero points 4..11, log-normal scales), "
                        "seven Qwen2-1.5B shapes, fp16 activations with 1% outlier channels x20",
            "parity_worst_normwise_rel_err": worst,
            "m1": {"GBps": round(m1, 1), "roofline": {"bound": "hbm", "achieved": round(m1, 1), "peak": HBM_PEAK_GBS,
                                                     "frac": round(m1 / HBM_PEAK_GBS, 4)}, "per_shape": rows1},
            "m2048": {"TFLOPs": round(m2048, 1),
                      "roofline": {"bound": "mfma", "achieved": round(m2048, 1), "peak": MFMA_PEAK_TFLOPS,
                                   "frac": round(m2048 / MFMA_PEAK_TFLOPS, 4)}, "per_shape": rows2}}


# ---------------------------------------------------------------------------
# CPU baseline (and the parity check against it)
# ---------------------------------------------------------------------------

def host_threads() -> int:
    """CPUs this process may run on (os.cpu_count() counts the whole machine,
    which on a shared host can exceed the process's CPU set)."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_model_name() -> str:
    name = platform.processor() or "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return name


def cpu_parity(decode, gemm, torch):
    """The cpu_baseline leg's parity check, run before any timed region: every
    decode output and the rows-2048 GEMM outputs of this run against the
    CPU restatement of the reference's torch backend (backends.py:73-98),
    normwise relative error <= 1e-2 -- the reference harness checks parity
    before it times (scripts/autotune_phase_e_triton_v6.py:96-101)."""
    from oracle import oracle as O

    torch.set_num_threads(host_threads())
    worst = 0.0
    for case in list(decode) + list(gemm):
        x, q, s, z = case["x"].cpu(), *(t.cpu() for t in case["w"])
        ref = O.reference_linear_torch(x, q, s, z, None, out_features=case["n"], in_features=case["k"],
                                       return_f32=True)
        got = case["out"].float().cpu()
        rel = float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        if not bool(torch.isfinite(got).all()) or rel > 1e-2:
            raise SystemExit(f"parity failed for {case['name']} rows={case['rows']}: normwise relative error "
                             f"{rel:.3e}")
        worst = max(worst, rel)
    log(f"parity vs CPU reference: worst normwise relative error {worst:.2e} over {len(decode) + len(gemm)} calls")
    return {"calls": len(decode) + len(gemm), "worst_normwise_rel_err": worst, "bar": 1e-2}


def _cpu_samples(fn, warmup: int, reps: int, budget_s: float):
    """perf_counter_ns samples (s) of fn: warm-up, then up to `reps` calls
    within `budget_s` (scripts/autotune_phase_e_triton_v6.py:41-56 times
    warm-up 20 + 100 iterations; the CPU leg is bounded by time instead)."""
    for _ in range(warmup):
        fn()
    times = []
    start = time.perf_counter()
    while len(times) < reps and (time.perf_counter() - start) < budget_s:
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    return times


def cpu_baseline(decode, torch, budget_s: float = 12.0):
    """The reference's torch backend restated on CPU (the oracle's port),
    timed on the host cores: the decode step (all 21 calls) over a bounded
    sample, and the single q_proj 1536x1536 call at M = 1 of the CPU
    configuration on its own."""
    from oracle import oracle as O

    threads = host_threads()
    torch.set_num_threads(threads)
    tensors = [(c["x"].cpu(), *(t.cpu() for t in c["w"]), c["n"], c["k"]) for c in decode]
    step_bytes = sum(case["bytes"] for case in decode)

    def one_step():
        for x, q, s, z, n, k in tensors:
            O.reference_linear_torch(x, q, s, z, None, out_features=n, in_features=k)

    times = _cpu_samples(one_step, 1, 30, budget_s)
    step_s = statistics.median(times)
    # the CPU configuration: symmetric RTN q_proj 1536x1536, M = 1, fp16 activations
    q_case = next(c for c in decode if c["name"] == "q_proj" and c["rows"] == 1)
    qx, qq, qs, qz = q_case["x"].cpu(), *(t.cpu() for t in q_case["w"])
    q_times = _cpu_samples(lambda: O.reference_linear_torch(qx, qq, qs, qz, None, out_features=1536,
                                                            in_features=1536), 5, 100, 5.0)
    q_s = statistics.median(q_times)
    return {
        "value": step_bytes / step_s / 1e9,
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{len(times)} decode steps (21 calls each: 7 shapes x rows 1/4/16, fp16) of the torch CPU "
                   f"restatement of the reference's torch backend; median {step_s * 1e3:.1f} ms/step; "
                   f"host {cpu_model_name()}, os.cpu_count()={os.cpu_count()}, threads = CPUs in this process's "
                   f"affinity set"),
        "step_ms_p50": round(step_s * 1e3, 3),
        "step_ms_p95": round(percentile(times, 95) * 1e3, 3),
        "q_proj_m1": {
            "workload": "q_proj 1536x1536, M=1, symmetric RTN W4G64, fp16 activations, CPU torch backend",
            "calls": len(q_times), "us_p50": round(q_s * 1e6, 1), "us_p95": round(percentile(q_times, 95) * 1e6, 1),
            "GBps": round(q_case["bytes"] / q_s / 1e9, 3),
        },
    }


def percentile(values, p: float) -> float:
    """Nearest-rank percentile."""
    ordered = sorted(values)
    if not ordered:
        return float("nan")
    rank = max(1, int(-(-len(ordered) * p // 100)))
    return ordered[min(rank, len(ordered)) - 1]


# ---------------------------------------------------------------------------
# rocprofv3 --pmc support
# ---------------------------------------------------------------------------

def profile_pass() -> int:
    """Untimed dispatch sequence for rocprofv3 --pmc (see the module docstring)."""
    import torch

    from qwen_int4_hip import hip_available, linear_canonical_w4g64_hip, unpack_canonical_signed_int4_hip

    if not hip_available():
        raise SystemExit("bench.py needs a ROCm GPU and the built HIP library")
    scrub = torch.empty(SCRUB_BYTES, dtype=torch.uint8, device="cuda")
    packed = torch.randint(0, 256, (CALIBRATION_PACKED_BYTES,), dtype=torch.uint8, device="cuda")
    _, copies, cases = decode_cases(torch, 8)
    scrub.fill_(1)
    unpack_canonical_signed_int4_hip(packed)
    for step in range(3):
        scrub.fill_(2 + step)
        for c in cases:
            linear_canonical_w4g64_hip(c["x"], *c["copies"][(3 * step + c["copy0"]) % 8])
    for name in PREFILL_SHAPES:
        n, k = QWEN2_SHAPES[name]
        x = gen_activations(2048, k, BASE_SEED + 7 * 2048 + n, torch.bfloat16, torch)
        for rep in range(2):
            scrub.fill_(7 + rep)
            linear_canonical_w4g64_hip(x, *copies[name][rep])
    torch.cuda.synchronize()
    log(f"profile pass done: 1 calibration dispatch, {3 * len(cases)} decode calls, "
        f"{2 * len(PREFILL_SHAPES)} GEMM calls")
    return 0


def _pmc_dispatches(csv_path: str, counter: str):
    """[(dispatch id, kernel name, counter value in KiB)] in dispatch order."""
    import csv

    per = {}
    with open(csv_path, newline="") as fh:
        for row in csv.DictReader(fh):
            if row["Counter_Name"] != counter:
                continue
            key = int(row["Dispatch_Id"])
            name, total = per.get(key, (row["Kernel_Name"], 0.0))
            per[key] = (name, total + float(row["Counter_Value"]))
    return [(k, v[0], v[1]) for k, v in sorted(per.items())]


def summarize_pmc(fetch_csv: str, write_csv: str, out_path: str) -> int:
    fetch = _pmc_dispatches(fetch_csv, "FETCH_SIZE")
    write = _pmc_dispatches(write_csv, "WRITE_SIZE")

    def split(rows):
        cal = [v for _, name, v in rows if "unpack_kernel" in name]
        dec = [v for _, name, v in rows if "gemv" in name]
        red = [v for _, name, v in rows if "split_reduce" in name]  # second dispatch of a split-K decode call
        gem = [v for _, name, v in rows if "gemm" in name]
        if len(cal) != 1 or len(dec) % 21 or not dec:
            raise SystemExit(f"unexpected dispatch sequence: {len(cal)} calibration, {len(dec)} decode dispatches")
        return cal[0], dec + red, gem

    f_cal, f_dec, f_gem = split(fetch)
    w_cal, w_dec, w_gem = split(write)
    f_scale = (CALIBRATION_PACKED_BYTES / 1024) / f_cal   # true KiB per counted KiB
    w_scale = (2 * CALIBRATION_PACKED_BYTES / 1024) / w_cal
    steps = sum(1 for _, name, _ in fetch if "gemv" in name) // 21
    step_bytes = sum(algorithmic_bytes(r, n, k) for r in DECODE_ROWS for (n, k) in QWEN2_SHAPES.values())
    fetch_step = sum(f_dec) * f_scale * 1024 / steps
    write_step = sum(w_dec) * w_scale * 1024 / steps
    summary = {
        "calibration": {"kernel": "unpack_kernel", "reads_bytes": CALIBRATION_PACKED_BYTES,
                        "writes_bytes": 2 * CALIBRATION_PACKED_BYTES, "FETCH_SIZE_KiB": f_cal, "WRITE_SIZE_KiB": w_cal,
                        "fetch_scale": f_scale, "write_scale": w_scale},
        "decode": {"kernel": "decode GEMV kernels and their split-K reductions (all 21 calls of a step)", "steps": steps, "launches_per_step": 21,
                   "algorithmic_bytes_per_launch": step_bytes / 21,
                   "fetch_bytes_per_launch": fetch_step / 21, "write_bytes_per_launch": write_step / 21,
                   "traffic_bytes_per_launch": (fetch_step + write_step) / 21,
                   "traffic_over_algorithmic": (fetch_step + write_step) / step_bytes},
    }
    if f_gem and len(f_gem) == len(w_gem):
        # a split GEMM call is two dispatches (GEMM + reduction): totals per call
        calls = len(PREFILL_SHAPES) * 2
        per_call = sum(a * f_scale + b * w_scale for a, b in zip(f_gem, w_gem)) * 1024 / calls
        summary["gemm_2048"] = {"kernel": "gemm_kernel<f16 a x int b,128x256> (+ activation staging, split-K reduction)", "calls": calls,
                                "algorithmic_bytes_per_call": algorithmic_bytes(2048, 8960, 1536),
                                "traffic_bytes_per_call": per_call}
    Path(out_path).parent.mkdir(parents=True, exist_ok=True)
    Path(out_path).write_text(json.dumps(summary, indent=2) + "\n")
    print(json.dumps(summary, indent=2))
    return 0


MFMA_PASS_COUNTERS = "GRBM_GUI_ACTIVE SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES"
XCDS = 8  # GRBM_GUI_ACTIVE is summed over the XCDs: cycles / XCDS / duration = shader clock


def mfma_pass() -> int:
    """Untimed dispatch sequence for rocprofv3 --pmc MFMA_PASS_COUNTERS: the
    rows-2048 prefill GEMMs (4 calls per shape), then the same problems as
    dense bf16 torch.matmul (4 calls per shape)."""
    import torch

    from qwen_int4_hip import hip_available, linear_canonical_w4g64_hip

    if not hip_available():
        raise SystemExit("bench.py needs a ROCm GPU and the built HIP library")
    problems = []
    for name in PREFILL_SHAPES:
        n, k = QWEN2_SHAPES[name]
        x = gen_activations(2048, k, BASE_SEED + 7 * 2048 + n, torch.bfloat16, torch)
        problems.append((name, x, gen_weights(n, k, BASE_SEED + n + k, torch), n, k))
    for _, x, w, _, _ in problems:
        for _ in range(4):
            linear_canonical_w4g64_hip(x, *w)
    for _, x, _, n, k in problems:
        dense = torch.randn((k, n), device="cuda", dtype=torch.float32).to(torch.bfloat16).contiguous()
        for _ in range(4):
            torch.matmul(x, dense)
    torch.cuda.synchronize()
    log(f"mfma pass done: {4 * len(problems)} W4G64 GEMM calls, {4 * len(problems)} dense bf16 matmuls")
    return 0


def summarize_mfma(csv_path: str, out_path: str, cus: int = 256) -> int:
    """Per-kernel shader clock and MFMA busy fraction from an --mfma-pass
    counter file: clock = GRBM_GUI_ACTIVE / XCDS / duration; MFMA busy =
    SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x CUs x clock cycles)."""
    import csv

    per = {}
    with open(csv_path, newline="") as fh:
        for row in csv.DictReader(fh):
            key = int(row["Dispatch_Id"])
            d = per.setdefault(key, {"name": row["Kernel_Name"], "grid": row["Grid_Size"],
                                     "ns": int(row["End_Timestamp"]) - int(row["Start_Timestamp"])})
            d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    groups = {}
    for key in sorted(per):
        d = per[key]
        if d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) <= 0:
            continue
        label = "W4G64 gemm_kernel" if "gemm_kernel" in d["name"] else d["name"].split("_MT")[0][:48]
        groups.setdefault((label, d["grid"], d["SQ_VALU_MFMA_BUSY_CYCLES"]), []).append(d)
    rows = []
    for (label, grid, busy), ds in groups.items():
        ds = ds[1:] if len(ds) > 1 else ds  # the first call of each group warms clocks and caches
        ns = statistics.median(d["ns"] for d in ds)
        cycles = statistics.median(d["GRBM_GUI_ACTIVE"] for d in ds) / XCDS
        mfma_insts = busy / 32.0  # one v_mfma_*_32x32x16 bf16 keeps a SIMD busy for 32 cycles
        flops = mfma_insts * 32 * 32 * 16 * 2
        rows.append({"kernel": label, "grid": int(grid), "calls": len(ds), "duration_us": ns / 1e3,
                     "clock_GHz": cycles / ns,
                     "mfma_busy_frac": busy / (4 * cus * cycles), "flops": flops,
                     "TFLOPs": flops / ns / 1e3, "frac_of_2p5PF": flops / ns / 1e3 / MFMA_PEAK_TFLOPS})
    Path(out_path).parent.mkdir(parents=True, exist_ok=True)
    Path(out_path).write_text(json.dumps(rows, indent=2) + "\n")
    print("| kernel | grid (threads) | problem GFLOP | calls | duration (us) | clock (GHz) | MFMA busy | TFLOP/s | "
          "of 2.5 PF |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {r['kernel']} | {r['grid']} | {r['flops'] / 1e9:.2f} | {r['calls']} | {r['duration_us']:.1f} | "
              f"{r['clock_GHz']:.2f} | {r['mfma_busy_frac']:.1%} | {r['TFLOPs']:.0f} | {r['frac_of_2p5PF']:.1%} |")
    return 0


TIMELINE_PHASES = ("entry", "loads issued", "staging landed", "LDS barrier", "MFMA steps done",
                   "reduction barrier", "stores issued", "stores complete")
STREAM_PHASES = ("entry", "load issued", "data landed")
GEMV_PHASES = ("entry", "staging landed", "staged in LDS", "LDS barrier", "MFMA steps done",
               "partial sums combined", "stores issued", "stores complete")
PIPE_PHASES = ("entry", "staging landed, first loads issued", "LDS barrier", "steps done", "stores issued", "-", "-",
               "stores complete")
UNMERGED_ATTENTION_PHASES = ("entry", "chunk staged in LDS", "scores", "softmax statistics", "partials stored",
                             "exit", "-", "stores complete")
MERGE_PHASES = ("entry", "staging landed, first loads issued", "LDS barrier", "steps done", "stores issued",
                "merge statistics in LDS", "merged row formed", "stores complete")
ATTENTION_PHASES = ("entry", "chunk staged in LDS", "scores", "softmax statistics", "partials stored",
                    "arrival counted", "merge statistics (last arrival)", "stores complete")


SUSTAINED_CASES = (  # (rows, out_features, in_features, what the tall shape stacks)
    (1, 17920 * 28, 1536, "gate and up of 28 layers"),
    (1, 1536 * 28, 8960, "down_proj of 28 layers (stacked output rows)"),
    (4, 17920 * 28, 1536, "gate and up of 28 layers"),
    (16, 17920 * 28, 1536, "gate and up of 28 layers"),
    (16, 1536 * 28, 8960, "down_proj of 28 layers (stacked output rows)"),
)


def sustained_rates(torch) -> list:
    """Steady-state rate of the decode GEMV kernels: one launch over a tall
    weight matrix (the listed projection stacked over 28 layers, 200-430 MB),
    so that launch and the per-workgroup latency chain are amortised.  Random
    packed codes, fp16 scales in [0.001, 0.011), zero codes 0 (the kernels'
    work does not depend on the values); fp16 activations; HIP events around
    each of 10 launches after 3 warm-ups, the median reported."""
    from qwen_int4_hip import _lib
    from qwen_int4_hip.kernels import _workspace

    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    gen = torch.Generator(device="cuda").manual_seed(BASE_SEED + 9)
    out = []
    for rows, n, k, what in SUSTAINED_CASES:
        q = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device="cuda", generator=gen)
        sc = (torch.rand((n, k // 64), device="cuda", generator=gen) * 0.01 + 0.001).to(torch.float16)
        z = torch.zeros((n * (k // 64) + 1) // 2, dtype=torch.uint8, device="cuda")
        x = torch.randn((rows, k), device="cuda", generator=gen).to(torch.float16)
        y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
        ws = _workspace(torch.device("cuda"), max(16, lib.w4g64_linear_workspace_bytes(rows, n, k, _lib.DTYPE_F16)))
        name = lib.w4g64_linear_kernel_name(rows, n, k, _lib.DTYPE_F16).decode()
        p_ = lambda t: ctypes.c_void_p(t.data_ptr())

        def call():
            _lib.check(lib.w4g64_linear(p_(x), _lib.DTYPE_F16, p_(q), p_(sc), p_(z), None, _lib.DTYPE_NONE, p_(y), rows,
                                        n, k, p_(ws), ws.numel(), stream))

        for _ in range(3):
            call()
        torch.cuda.synchronize()
        times = []
        for _ in range(10):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            call()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3)
        us = statistics.median(times)
        nbytes = algorithmic_bytes(rows, n, k)
        out.append({"rows": rows, "n": n, "k": k, "stacks": what, "kernel": name, "us_p50": round(us, 2),
                    "MB": round(nbytes / 1e6, 1), "GBps": round(nbytes / us / 1e3, 1),
                    "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)})
        del q, sc, z, x, y
    return out


def sustained_pass() -> int:
    """The steady-state table (sustained_rates) as markdown."""
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench.py --sustained needs a ROCm GPU")
    print("| rows | out x in | stacks | MB | kernel | us (p50) | GB/s | of 8 TB/s |")
    print("|---:|---|---|---:|---|---:|---:|---:|")
    for r in sustained_rates(torch):
        print(f"| {r['rows']} | {r['n']}x{r['k']} | {r['stacks']} | {r['MB']} | {r['kernel']} | {r['us_p50']} | "
              f"{r['GBps']:.0f} | {r['frac']:.1%} |", flush=True)
    return 0


def timeline_pass() -> int:
    """Per-workgroup phase timelines of the one-row decode GEMV (gemv_seg_kernel)
    and of a bare streaming kernel over the same bytes, from the profiling
    build libw4g64_hip_timeline.so: chip-wide s_memrealtime stamps (100 MHz),
    cold caches (a 512 MiB write before each call), eager launches; the last
    of 5 calls is reported, relative to the first workgroup's entry."""
    import torch

    from qwen_int4_hip import _lib, build as hip_build
    from qwen_int4_hip.kernels import _workspace

    if not hip_build.TIMELINE_LIBRARY.exists():
        hip_build.build(timeline=True)  # the profiling build is made on demand
    if not torch.cuda.is_available():
        raise SystemExit("bench.py --timeline needs a ROCm GPU")
    lib = ctypes.CDLL(str(hip_build.TIMELINE_LIBRARY))
    for name, (res, argtypes) in _lib.SIGNATURES.items():
        if hasattr(lib, name):
            getattr(lib, name).restype = res
            getattr(lib, name).argtypes = argtypes
    lib.w4g64_timeline_register.restype = ctypes.c_int
    lib.w4g64_timeline_register.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    lib.w4g64_timeline_stream.restype = ctypes.c_int
    lib.w4g64_timeline_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    max_wgs = 4096
    stamps = torch.zeros(max_wgs * 8, dtype=torch.int64, device="cuda")
    lib.w4g64_timeline_register(ctypes.c_void_p(stamps.data_ptr()), max_wgs)
    scrub = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def report(label, phases, run, scrubbed=True):
        for i in range(5):
            if scrubbed:
                scrub.fill_(i + 1)
            stamps.zero_()
            torch.cuda.synchronize()
            run()
            torch.cuda.synchronize()
        t = stamps.view(max_wgs, 8).cpu()
        used = t[:, 0] != 0
        t = t[used].double()
        t0 = float(t[:, 0].min())
        print(f"\n{label}: {int(used.sum())} workgroups; us after the first workgroup's entry")
        print("| point | workgroups | p10 | p50 | p90 | max |")
        print("|---|---:|---:|---:|---:|---:|")
        cols = list(range(len(phases))) if phases is STREAM_PHASES else list(range(8))
        for c, nm in zip(cols, phases):
            v = t[:, c][t[:, c] != 0]  # points a workgroup did not reach stay 0
            if v.numel() == 0:
                continue
            v = ((v - t0) * 0.01).sort().values  # 100 MHz ticks -> us
            q = lambda f: float(v[min(len(v) - 1, int(f * (len(v) - 1)))])
            print(f"| {nm} | {v.numel()} | {q(.1):.2f} | {q(.5):.2f} | {q(.9):.2f} | {q(1):.2f} |")

    for nbytes in (7_434_240, 1_327_104):
        src = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
        report(f"stream {nbytes / 1e6:.2f} MB (one 16-byte load per lane)", STREAM_PHASES,
               lambda: _lib.check(lib.w4g64_timeline_stream(ctypes.c_void_p(src.data_ptr()), nbytes,
                                                            ctypes.c_void_p(sink.data_ptr()), stream)))
    for name, rows in (("gate_proj", 1), ("q_proj", 1), ("down_proj", 1), ("gate_proj", 4), ("gate_proj", 16),
                       ("down_proj", 16)):
        n, k = QWEN2_SHAPES[name]
        q, s_, z = gen_weights(n, k, BASE_SEED + n + k, torch)
        x = gen_activations(rows, k, BASE_SEED + 3, torch.float16, torch)
        y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
        ws = _workspace(torch.device("cuda"), max(16, lib.w4g64_linear_workspace_bytes(rows, n, k, _lib.DTYPE_F16)))
        kname = lib.w4g64_linear_kernel_name(rows, n, k, _lib.DTYPE_F16).decode()

        def call():
            _lib.check(lib.w4g64_linear(ctypes.c_void_p(x.data_ptr()), _lib.DTYPE_F16, ctypes.c_void_p(q.data_ptr()),
                                        ctypes.c_void_p(s_.data_ptr()), ctypes.c_void_p(z.data_ptr()), None,
                                        _lib.DTYPE_NONE, ctypes.c_void_p(y.data_ptr()), rows, n, k,
                                        ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream))

        label = (f"{name} {n}x{k}, {rows} fp16 row{'s' if rows > 1 else ''}, "
                 f"{algorithmic_bytes(rows, n, k) / 1e6:.2f} MB: {kname}")
        report(label, TIMELINE_PHASES if kname.startswith("gemv_seg") else
               (PIPE_PHASES if kname.startswith("gemv_pipe") else GEMV_PHASES), call)

    # decode attention of one Qwen2-1.5B layer: batch 1, 12 query / 2 key-value heads, position 575 of a
    # 641-position cache (the e2e workload's midpoint); caches stay warm, as in the decode step
    heads, kvh, hd, max_len, pos = 12, 2, 128, 641, 575
    gen = torch.Generator(device="cuda").manual_seed(BASE_SEED + 5)
    qkv = (torch.randn((1, (heads + 2 * kvh) * hd), generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
    ang = torch.arange(hd, device="cuda", dtype=torch.float32) * 0.01 * pos
    cos, sin = ang.cos().to(torch.bfloat16)[None], ang.sin().to(torch.bfloat16)[None]
    kc = (torch.randn((1, kvh, max_len, hd), generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
    vc = (torch.randn((1, kvh, max_len, hd), generator=gen, device="cuda") * 0.5).to(torch.bfloat16)
    position = torch.full((1,), pos, dtype=torch.int64, device="cuda")
    out = torch.empty((1, heads * hd), dtype=torch.bfloat16, device="cuda")
    aws = torch.zeros(max(16, lib.qwen2_decode_attention_workspace_bytes(1, kvh, max_len)), dtype=torch.uint8,
                      device="cuda")
    p_ = lambda t: ctypes.c_void_p(t.data_ptr())
    report(f"decode attention, position {pos} (chunks of 64 positions, one workgroup per chunk and key/value head)",
           ATTENTION_PHASES,
           lambda: _lib.check(lib.qwen2_decode_attention(p_(qkv), p_(cos), p_(sin), p_(kc), p_(vc), p_(position), p_(out),
                                                         1, heads, kvh, hd, max_len, hd ** -0.5, p_(aws), aws.numel(),
                                                         stream)),
           scrubbed=False)
    # the batch-1 decode step's form: the attention leaves its per-chunk partials and the o_proj GEMV merges them
    # in its staging; the plain o_proj over the attention's output beside it
    report(f"decode attention without its merge, position {pos} (partials only)", UNMERGED_ATTENTION_PHASES,
           lambda: _lib.check(lib.qwen2_decode_attention_partials(p_(qkv), p_(cos), p_(sin), p_(kc), p_(vc),
                                                                  p_(position), 1, heads, kvh, hd, max_len,
                                                                  hd ** -0.5, p_(aws), aws.numel(), stream)),
           scrubbed=False)
    qo, so, zo = gen_weights(heads * hd, heads * hd, BASE_SEED + 23, torch)
    yo = torch.empty((1, heads * hd), dtype=torch.bfloat16, device="cuda")
    ows = _workspace(torch.device("cuda"), 1 << 20)
    report(f"o_proj {heads * hd}x{heads * hd} merging the {-(-max_len // 64)} chunks' partials in its staging",
           MERGE_PHASES,
           lambda: _lib.check(lib.w4g64_linear_attention_merge(p_(aws), aws.numel(), max_len, heads, kvh, p_(qo), p_(so),
                                                               p_(zo), None, _lib.DTYPE_NONE, p_(yo), 1, heads * hd,
                                                               stream)),
           scrubbed=False)
    report(f"o_proj {heads * hd}x{heads * hd} over the attention's bf16 output (plain form)", PIPE_PHASES,
           lambda: _lib.check(lib.w4g64_linear(p_(out), _lib.DTYPE_BF16, p_(qo), p_(so), p_(zo), None, _lib.DTYPE_NONE,
                                               p_(yo), 1, heads * hd, heads * hd, p_(ows), ows.numel(), stream)),
           scrubbed=False)
    lib.w4g64_timeline_register(None, 0)

    # residency: the same product kernels with their weights resident in L2 (one copy), in the 256 MB
    # Infinity Cache (~60 MB of copies) or cold (~600 MB of copies), graph replays of back-to-back launches
    hip = Hip()
    print("\n| call (1 fp16 row) | L2-resident | ~60 MB of copies | ~600 MB of copies |")
    print("|---|---:|---:|---:|")
    for name in ("q_proj", "gate_proj", "down_proj"):
        n, k = QWEN2_SHAPES[name]
        wbytes = n * k // 2 + n * (k // 64) * 2 + n * k // 128
        cold = -(-600_000_000 // wbytes)
        cold += cold % 3 == 0  # the replay visits copies with stride 3
        mall = max(2, 60_000_000 // wbytes)
        mall += mall % 3 == 0
        base = gen_weights(n, k, BASE_SEED + n + k, torch)
        pool = [tuple(t.clone() for t in base) for _ in range(cold)]
        x = gen_activations(1, k, BASE_SEED + 11, torch.float16, torch)
        cells = []
        for copies in (1, mall, cold):
            case = {"x": x, "copies": pool[:copies], "copy0": 0}
            d = graph_kernel_durations([case], 10, hip, torch, launches=max(32, copies))[0]
            cells.append(f"{statistics.median(d) * 1e3:.2f} us")
        print(f"| {name} {n}x{k} | " + " | ".join(cells) + " |")
        del pool
        torch.cuda.empty_cache()
    return 0


def committed_traffic():
    try:
        return json.loads(PMC_TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None


# ---------------------------------------------------------------------------
# End to end: Qwen2-1.5B architecture, 512-token prompt, 128 greedy tokens
# ---------------------------------------------------------------------------

QWEN2_1_5B = dict(hidden_size=1536, num_attention_heads=12, num_key_value_heads=2, head_dim=128,
                  intermediate_size=8960, num_hidden_layers=28, vocab_size=151936, rms_norm_eps=1e-6,
                  rope_theta=1_000_000.0)


def build_model(torch, seed: int):
    """Random-init Qwen2-1.5B (N(0, 0.02)); all 196 linears symmetric RTN W4G64."""
    from types import SimpleNamespace

    from qwen_int4_hip import QuantLinear, quantize_symmetric_rtn
    from qwen_int4_hip.model import QwenInt4ForCausalLM

    gen = torch.Generator(device="cuda").manual_seed(seed)
    model = QwenInt4ForCausalLM(SimpleNamespace(**QWEN2_1_5B), packing="canonical", group_size=64).to("cuda")
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


def end_to_end(torch, hip, prompt_len: int = 512, new_tokens: int = 128, prefill_reps: int = 10,
               check_steps: int = 8):
    """Prefill and greedy decode of the full workload on the serving path
    (FusedPrefill + one graph replay of FusedDecodeStep per token), with the
    reference harness's statistics (p50/p95: scripts/benchmark_phase_f_model.py
    :33-50) and, before timing, a check of the served logits against the
    module path (growing cache, same HIP linears, unfused glue) under teacher
    forcing."""
    from qwen_int4_hip.generation import StaticGreedyDecoder

    model = build_model(torch, BASE_SEED)
    gen = torch.Generator().manual_seed(BASE_SEED + 4)
    prompt = torch.randint(0, QWEN2_1_5B["vocab_size"], (1, prompt_len), generator=gen).cuda()
    decoder = StaticGreedyDecoder(model, 1, prompt_len + new_tokens)

    def cos(a, b):
        a, b = a.double().flatten(), b.double().flatten()
        return float(a @ b / (a.norm() * b.norm()))

    with torch.inference_mode():
        served = [decoder.prefill(prompt).clone()]
        want, cache = model(prompt, use_cache=True)
        checks = [cos(served[0], want)]
        token = want[:, -1:].argmax(dim=-1)
        for _ in range(check_steps):
            got = decoder.step(token).clone()
            want, cache = model(token, past_key_values=cache, use_cache=True)
            checks.append(cos(got, want))
            if not bool(torch.isfinite(got).all()):
                raise SystemExit("e2e: non-finite logits on the serving path")
            token = want[:, -1:].argmax(dim=-1)
        del cache, want
    if min(checks) < 0.999:
        raise SystemExit(f"e2e: served logits differ from the module path (min cosine {min(checks):.6f})")
    torch.cuda.synchronize()

    prefill_ms = []
    for _ in range(prefill_reps):
        decoder.length = 0
        t0 = time.perf_counter()
        decoder.prefill(prompt)
        torch.cuda.synchronize()
        prefill_ms.append((time.perf_counter() - t0) * 1e3)
    tokens = [decoder.token.clone()]
    t0 = time.perf_counter()
    for _ in range(new_tokens - 1):
        decoder.step()
        tokens.append(decoder.token.clone())
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - t0
    # per-token distribution: the same decode again, each step between two events
    decoder.length = 0
    decoder.prefill(prompt)
    step_ms = replay_samples(lambda i: decoder.step(), new_tokens - 1, hip, torch)
    linear_bytes = 28 * sum(algorithmic_bytes(1, n, k) for n, k in QWEN2_SHAPES.values())
    head_bytes = QWEN2_1_5B["vocab_size"] * QWEN2_1_5B["hidden_size"] * 2
    per_token = decode_s / (new_tokens - 1)
    prefill_p50 = statistics.median(prefill_ms)
    head = lm_head_rate(torch, decoder, head_bytes)
    return {
        "workload": (f"Qwen2-1.5B architecture (28 layers, hidden 1536, GQA 12/2 x 128, SwiGLU 8960, vocab 151936), "
                     f"random-init N(0,0.02) weights, 196 symmetric RTN W4G64 linears, tied bf16 LM head; batch 1, "
                     f"{prompt_len}-token random prompt then {new_tokens} greedy tokens, static KV cache, one HIP graph "
                     f"replay per decode step"),
        "prefill_ms": round(prefill_p50, 3),
        "prefill_ms_p95": round(percentile(prefill_ms, 95), 3),
        "prefill_samples": len(prefill_ms),
        "prefill_tokens_per_s": round(prompt_len / (prefill_p50 * 1e-3), 1),
        "decode_ms_per_token": round(per_token * 1e3, 4),
        "decode_ms_p50": round(statistics.median(step_ms), 4),
        "decode_ms_p95": round(percentile(step_ms, 95), 4),
        "decode_tokens_per_s": round(1.0 / per_token, 1),
        "decode_weight_bytes_per_token": linear_bytes + head_bytes,
        "decode_weight_GBps": round((linear_bytes + head_bytes) / per_token / 1e9, 1),
        "generated_tokens": int(torch.cat(tokens, dim=1).numel()),
        "served_vs_module_path_min_cosine": round(min(checks), 7),
        "lm_head": head,
    }


def log_e2e(e2e) -> None:
    log(f"e2e: prefill p50 {e2e['prefill_ms']:.2f} ms p95 {e2e['prefill_ms_p95']:.2f} ms "
        f"({e2e['prefill_tokens_per_s']:.0f} tok/s), decode {e2e['decode_ms_per_token']:.3f} ms/token "
        f"(p50 {e2e['decode_ms_p50']:.3f}, p95 {e2e['decode_ms_p95']:.3f}; {e2e['decode_tokens_per_s']:.0f} tok/s)")
    if e2e.get("lm_head"):
        h = e2e["lm_head"]
        log(f"e2e LM head: {h['us_per_call']:.1f} us per call, {h['GBps']:.0f} GB/s ({100 * h['frac']:.1f}% of 8 TB/s)")


def lm_head_rate(torch, decoder, head_bytes: int, reps: int = 64):
    """The decode step's LM head (tied bf16 151936 x 1536 GEMV plus the greedy
    argmax: qwen2_lm_head) timed alone: `reps` back-to-back calls on the
    step's own buffers between two events on the stream they run on."""
    import ctypes

    fused = decoder.fused
    if fused is None or not fused.hip_head:
        return None
    weight = fused.model.lm_head.weight
    logits = torch.empty((fused.batch, fused.vocab), dtype=torch.bfloat16, device="cuda")
    token = torch.empty(fused.batch, dtype=torch.int64, device="cuda")
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = torch.cuda.current_stream()
    call = lambda: fused.lib.qwen2_lm_head(ptr(fused.normed), ptr(weight), ptr(logits), ptr(token), fused.batch,
                                           fused.vocab, fused.hidden, ptr(fused.head_workspace),
                                           fused.head_workspace.numel(), ctypes.c_void_p(stream.cuda_stream))
    for _ in range(4):
        assert call() == 0
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        call()
    stop.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / reps
    gbs = head_bytes / (us * 1e-6) / 1e9
    return {"kernels": "lm_head_kernel<3,1> + lm_head_argmax_kernel", "us_per_call": round(us, 2),
            "weight_bytes": head_bytes, "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


# ---------------------------------------------------------------------------
# main
# ---------------------------------------------------------------------------

def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=512)
    parser.add_argument("--warmup", type=int, default=64)
    parser.add_argument("--kernel-reps", type=int, default=32, help="timed graph replays per decode case (32 launches each) and event-timed calls per GEMM case "
                             "(at least 100)")
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="skip the CPU timing of the baseline leg (its parity check always runs)")
    parser.add_argument("--no-gemm", action="store_true")
    parser.add_argument("--no-e2e", action="store_true", help="skip the end-to-end Qwen2-1.5B generation")
    parser.add_argument("--no-profiles", action="store_true",
                        help="skip the reference's operator profiles and config 3 (AWQ weights)")
    parser.add_argument("--e2e-only", action="store_true",
                        help="run only the end-to-end generation and print its object (for kernel-trace profiles)")
    parser.add_argument("--report", type=str, default="", help="write the detailed JSON report here")
    parser.add_argument("--profile-pass", action="store_true",
                        help="untimed dispatch sequence for rocprofv3 --pmc (calibration, 3 decode steps, GEMMs)")
    parser.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                        help="turn two rocprofv3 --pmc counter_collection.csv files into the traffic file")
    parser.add_argument("--traffic-out", type=str, default=str(PMC_TRAFFIC_FILE))
    parser.add_argument("--mfma-pass", action="store_true",
                        help=f"untimed rows-2048 GEMMs (W4G64, then dense bf16) for rocprofv3 --pmc "
                             f"{MFMA_PASS_COUNTERS}")
    parser.add_argument("--timeline", action="store_true",
                        help="per-workgroup phase timelines of the one-row decode GEMV and a bare stream "
                             "(profiling build libw4g64_hip_timeline.so)")
    parser.add_argument("--sustained", action="store_true",
                        help="steady-state GB/s of the decode GEMV kernels over tall stacked weights (one launch each)")
    parser.add_argument("--summarize-mfma", nargs=2, metavar=("COUNTER_CSV", "OUT_JSON"),
                        help="shader clock and MFMA busy fraction per GEMM kernel from an --mfma-pass counter file")
    args = parser.parse_args()
    if args.summarize_pmc:
        return summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.traffic_out)
    if args.summarize_mfma:
        return summarize_mfma(*args.summarize_mfma)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this build "
              "(the W4G64 path has no multi-GPU component).", file=sys.stderr)
        return 2
    if args.profile_pass:
        return profile_pass()
    if args.mfma_pass:
        return mfma_pass()
    if args.timeline:
        return timeline_pass()
    if args.sustained:
        return sustained_pass()

    import torch

    from qwen_int4_hip import hip_available, linear_canonical_w4g64_hip, linear_kernel_name

    if not hip_available():
        raise SystemExit("bench.py needs a ROCm GPU and the built HIP library")
    hip = Hip()
    props = torch.cuda.get_device_properties(0)
    log(f"device: {props.name} CUs={props.multi_processor_count}")
    if args.e2e_only:
        e2e = end_to_end(torch, hip)
        log_e2e(e2e)
        print(json.dumps({"e2e": e2e}), flush=True)
        return 0

    # ---------------- workloads and parity (before any timing) ----------------
    base, copies, cases = decode_cases(torch, COPIES)
    distinct_mb = sum(sum(t.numel() * t.element_size() for t in c[0]) for c in copies.values()) * COPIES / 1e6
    step_bytes = sum(c["bytes"] for c in cases)
    for c in cases:
        c["out"] = linear_canonical_w4g64_hip(c["x"], *c["w"])
    gemm_cases = []
    if not args.no_gemm:
        for name in PREFILL_SHAPES:
            n, k = QWEN2_SHAPES[name]
            for rows in PREFILL_ROWS:
                x = gen_activations(rows, k, BASE_SEED + 7 * rows + n, torch.bfloat16, torch)
                gemm_cases.append({"name": name, "rows": rows, "n": n, "k": k, "x": x, "w": base[name],
                                   "copies": copies[name][:4], "copy0": 0})
        for c in gemm_cases:
            c["out"] = linear_canonical_w4g64_hip(c["x"], *c["w"])
    parity = cpu_parity(cases, [c for c in gemm_cases if c["rows"] == 2048], torch)

    # ---------------- decode workload ----------------
    # HIP graphs: graph p runs the 21 calls of a step on copies (3p + rows_index) % COPIES
    side = torch.cuda.Stream()
    phases = COPIES
    graphs = []
    with torch.cuda.stream(side):
        for c in cases:  # warm up on the capture stream (creates its workspace outside capture)
            linear_canonical_w4g64_hip(c["x"], *c["copies"][0])
        torch.cuda.synchronize()
        for p in range(phases):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for c in cases:
                    linear_canonical_w4g64_hip(c["x"], *c["copies"][(3 * p + c["copy0"]) % COPIES])
            graphs.append(g)
    torch.cuda.synchronize()
    for i in range(args.warmup):
        graphs[i % phases].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        graphs[i % phases].replay()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"decode: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s whole-step ({step_bytes / 1e6:.1f} MB/step)")
    # distribution of single steps: each replay between two events on the replay stream
    step_samples = replay_samples(lambda i: graphs[i % phases].replay(), max(100, args.kernel_reps), hip, torch)
    step_p50, step_p95 = statistics.median(step_samples), percentile(step_samples, 95)
    log(f"decode step: p50 {step_p50 * 1e3:.1f} us, p95 {step_p95 * 1e3:.1f} us over {len(step_samples)} replays")

    # live per-kernel durations: HIP events around graph replays of each shape
    durations = graph_kernel_durations(cases, max(100, args.kernel_reps), hip, torch)
    per_case = []
    kernel_ms_total = 0.0
    for c, d in zip(cases, durations):
        mean_ms = statistics.fmean(d)
        kernel_ms_total += mean_ms
        per_case.append({
            "name": c["name"], "rows": c["rows"], "n": c["n"], "k": c["k"], "bytes": c["bytes"],
            "kernel": linear_kernel_name(c["rows"], c["n"], c["k"], torch.float16),
            "kernel_us_mean": mean_ms * 1e3, "kernel_us_median": statistics.median(d) * 1e3,
            "kernel_us_p95": percentile(d, 95) * 1e3, "samples": len(d),
            "GBps": c["bytes"] / (mean_ms * 1e-3) / 1e9,
        })
    achieved = step_bytes / (kernel_ms_total * 1e-3) / 1e9
    m1_mlp = [p for p in per_case if p["rows"] == 1 and p["name"] in ("gate_proj", "up_proj", "down_proj")]
    m1_mlp_gbs = sum(p["bytes"] for p in m1_mlp) / (sum(p["kernel_us_mean"] for p in m1_mlp) * 1e-6) / 1e9
    m1 = [p for p in per_case if p["rows"] == 1]
    m1_gbs = sum(p["bytes"] for p in m1) / (sum(p["kernel_us_mean"] for p in m1) * 1e-6) / 1e9
    dominant = max(per_case, key=lambda p: p["kernel_us_mean"])
    for p in per_case:
        log(f"  {p['name']:9s} rows={p['rows']:2d}  {p['kernel_us_mean']:7.2f} us (p50 {p['kernel_us_median']:6.2f}, "
            f"p95 {p['kernel_us_p95']:6.2f})  {p['GBps']:8.1f} GB/s")
    log(f"decode kernels: {achieved:.1f} GB/s over all calls; M=1: {m1_gbs:.1f} GB/s; M=1 MLP shapes "
        f"{m1_mlp_gbs:.1f} GB/s")
    # the same kernels at steady state (one launch over a 28-layer stack of a projection)
    steady = sustained_rates(torch)
    for r in steady:
        log(f"  steady state rows={r['rows']:2d} {r['n']}x{r['k']} ({r['stacks']}): {r['us_p50']:.1f} us, "
            f"{r['GBps']:.0f} GB/s ({r['frac']:.1%})")
    # the bare-stream floor of a launch over the same bytes, measured the same way
    floor = stream_floor(torch, hip)
    for f in floor:
        log(f"  stream floor {f['bytes'] / 1e6:5.2f} MB: p50 {f['us_p50']:.2f} us (p95 {f['us_p95']:.2f}), "
            f"{f['GBps']:.0f} GB/s")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": ("decode step: 7 Qwen2-1.5B W4G64 linear shapes (q/k/v/o 1536x1536 & 256x1536, gate/up "
                         "8960x1536, down 1536x8960) x activation rows {1,4,16}, fp16 N(0,1) activations, symmetric "
                         "RTN weights N(0,0.02); 21 calls per step as one HIP graph"),
            "weight_copies": COPIES,
            "distinct_weight_MB": round(distinct_mb, 1),
            "bytes_per_step": step_bytes,
        },
        "step_us_p50": round(step_p50 * 1e3, 2),
        "step_us_p95": round(step_p95 * 1e3, 2),
        "parity": parity,
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_pipe_kernel (+ split_reduce_kernel for the K-split 4- and 16-row down projections; all 21 "
                      "calls of a step)",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "traffic_source": None,
            "m1_GBps": round(m1_gbs, 2),
            "m1_mlp_GBps": round(m1_mlp_gbs, 2),
            "m1_mlp_frac": round(m1_mlp_gbs / HBM_PEAK_GBS, 4),
            "dominant_kernel": {"call": f"{dominant['name']} rows={dominant['rows']}", "kernel": dominant["kernel"],
                                "us_mean": round(dominant["kernel_us_mean"], 3),
                                "achieved_GBps": round(dominant["GBps"], 1),
                                "frac": round(dominant["GBps"] / HBM_PEAK_GBS, 4)},
            "steady_state": steady,
            "stream_floor": floor,
        },
    }
    traffic = committed_traffic()
    if traffic:
        result["roofline"]["traffic"] = round(traffic["decode"]["traffic_bytes_per_launch"])
        result["roofline"]["traffic_source"] = (f"{PMC_TRAFFIC_FILE.relative_to(REPO_ROOT)}: FETCH_SIZE + WRITE_SIZE "
                                                f"per launch, scaled by the unpack-kernel calibration; algorithmic "
                                                f"{traffic['decode']['algorithmic_bytes_per_launch']:.0f} B/launch")

    # ---------------- prefill GEMM ----------------
    if gemm_cases:
        gd = kernel_durations(gemm_cases, max(100, args.kernel_reps), hip, torch)
        dense = dense_library_gemm_ms(gemm_cases, torch)
        gemm_rows = []
        flops_2048 = 0.0
        ms_2048 = 0.0
        dense_2048 = 0.0
        for c, d, dense_ms in zip(gemm_cases, gd, dense):
            mean_ms = statistics.fmean(d)
            flops = 2.0 * c["rows"] * c["n"] * c["k"]
            tflops = flops / (mean_ms * 1e-3) / 1e12
            gemm_rows.append({"name": c["name"], "rows": c["rows"], "n": c["n"], "k": c["k"],
                              "kernel_us_mean": mean_ms * 1e3, "kernel_us_p50": statistics.median(d) * 1e3,
                              "kernel_us_p95": percentile(d, 95) * 1e3, "samples": len(d), "TFLOPs": tflops,
                              "dense_bf16_library_us": dense_ms * 1e3,
                              "dense_bf16_library_TFLOPs": flops / (dense_ms * 1e-3) / 1e12})
            log(f"  gemm {c['name']:9s} rows={c['rows']:4d}  {mean_ms * 1e3:8.2f} us (p95 {percentile(d, 95) * 1e3:8.2f})"
                f"  {tflops:7.1f} TFLOP/s   (dense bf16 torch.matmul {dense_ms * 1e3:8.2f} us)")
            if c["rows"] == 2048:
                flops_2048 += flops
                ms_2048 += mean_ms
                dense_2048 += dense_ms
        tf = flops_2048 / (ms_2048 * 1e-3) / 1e12
        gemm_traffic = traffic.get("gemm_2048") if traffic else None
        result["gemm"] = {
            "metric": "W4G64 GEMM TFLOP/s at M=2048 (gate/up 8960x1536 and down 1536x8960, bf16)",
            "value": round(tf, 2),
            "unit": "TFLOP/s",
            "dtype": "bf16",
            "roofline": {"bound": "mfma", "kernel": "gemm_kernel<f16 a x int b,128x256> (+ activation staging, split-K reduction)",
                         "achieved": round(tf, 2), "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                         "traffic": (round(gemm_traffic["traffic_bytes_per_call"])
                                     if gemm_traffic and "traffic_bytes_per_call" in gemm_traffic else None)},
            "dense_bf16_library_TFLOPs": round(flops_2048 / (dense_2048 * 1e-3) / 1e12, 2),
            "dense_bf16_library": ("torch.matmul of the same bf16 activations with a dense bf16 [K, N] weight "
                                   "(hipBLASLt): the vendor library's rate on the same shapes, without dequantization"),
            "per_shape": gemm_rows,
        }

    if not args.no_profiles:
        # the reference's own operator profiles and config 3 (asymmetric AWQ weights, outlier activations)
        result["reference_profiles"] = reference_profiles(torch, hip)
        result["awq_config3"] = awq_config3(torch, hip)

    if not args.no_e2e:
        result["e2e"] = end_to_end(torch, hip)
        log_e2e(result["e2e"])

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cases, torch)
        log(f"cpu baseline: {result['cpu_baseline']['value']:.3f} GB/s on {result['cpu_baseline']['cores']} threads; "
            f"q_proj M=1 {result['cpu_baseline']['q_proj_m1']['us_p50']:.0f} us")
    result["decode_per_shape"] = per_case
    if args.report:
        Path(args.report).parent.mkdir(parents=True, exist_ok=True)
        Path(args.report).write_text(json.dumps(result, indent=2) + "\n")
    line = {k: v for k, v in result.items() if k != "decode_per_shape"}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
