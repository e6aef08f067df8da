"""Benchmark of the GDN decode and prefill operators on one MI355X.

Prints ONE JSON line.  The headline ``value`` is the decode step at batch
256 (qk4 / v8 / d128): algorithmic state-stream bytes per second with every
input already resident in HBM.  The prefill at 32 768 packed tokens
(8 varlen sequences, qk16 / v32) is reported in the ``prefill`` object of
the same line.

Work accounting (per v-head and per step):
* decode bytes: 2 * 128 * 128 * 4 (state read + write) + 2 * 256 (v, o)
  + 4 (a, b), plus 2 * 256 (q, k) per qk-head;
* prefill flops per token: 10 * C * d + 6 * d^2 = 180 224 (C = 64, d = 128,
  dense chunk tiles) -- the conservative qk-shared count 8 C d + 6 d^2 is
  printed beside it.

Timing: ``--warmup`` untimed steps, then ``--steps`` timed steps bracketed by
``torch.cuda.synchronize()`` and one pair of HIP events on the launch
stream; a step is one kernel launch, so the mean launch duration (the
roofline's kernel time) is the elapsed time over the step count.  Every
object other than the headline decode also runs untimed launches for at
least ``WARM_MS`` of GPU time first (``warm_ms`` in the line): the clock
ramps up under load, and a compute-bound launch such as the 32k prefill
reaches its steady time only after ~35 ms of it.  Decode rotates 4 (state, new_state)
buffer sets (1 GiB) so the 256 MB Infinity Cache cannot serve the state.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()
from track_c_gdn_amd import backward as gbwd  # noqa: E402
from track_c_gdn_amd import conv as gconv  # noqa: E402
from track_c_gdn_amd import decode as gdec  # noqa: E402
from track_c_gdn_amd import inputs as ginp  # noqa: E402
from track_c_gdn_amd import prefill as gpre  # noqa: E402

METRIC = "decode state GB/s (%HBM peak) at B=256; prefill tokens/s (%MFMA) at 32k tok"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
D = 128
C = 64


def decode_bytes(B: int, HQ: int, HV: int) -> int:
    per_vhead = 2 * D * D * 4 + 2 * D * 2 + 4
    per_qkhead = 2 * D * 2
    return B * (HV * per_vhead + HQ * per_qkhead)


def prefill_flops(T: int, HV: int, qk_shared: bool = False) -> int:
    per_tok = (8 if qk_shared else 10) * C * D + 6 * D * D
    return T * HV * per_tok


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _traffic(name: str, path: str = None):
    """Bytes per launch from profiles/<name>_traffic.json; with ``path``, only
    when the profile was measured on that path."""
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if p.exists():
        try:
            d = json.loads(p.read_text())
        except Exception:
            return None
        if path is not None and d.get("path") != path:
            return None
        return d.get("bytes_per_launch")
    return None


# Untimed prefill launches before the timed ones.
PREFILL_WARMUP = 30
# GPU time of back-to-back untimed launches before a timed region (at least;
# on top of the warmup count).  Under sustained load the chip's clock ramps up
# over tens of milliseconds and drops back within a second of idling: the
# 32 768-token prefill launch takes ~334 us over its first 25 launches, ~278 us
# at launches 75-99 and a steady 266-272 us from about launch 125 (~35 ms of
# load) on; after 30 warmup launches the timed mean was 296 us, after 300 it was
# 267 us (same box, same run).  The operator legs other than the headline
# decode warm up for this long, so that their kernel times are the steady-state
# ones.
WARM_MS = 150.0
# at most this many extra untimed launches (short kernels reach WARM_MS only
# after tens of thousands of launches, which measures the host instead)
WARM_MAX_LAUNCHES = 4000


def timed_launches(launch, n_steps: int, warmup: int, warm_ms: float = 0.0):
    """Run ``launch(i)`` warmup + n_steps times; return (total_ms, mean_launch_ms).

    The timed launches run back to back on the launch stream between one
    pair of HIP events; every launch is one kernel, so the mean launch
    duration is the elapsed time over the launch count (event markers between
    launches would insert gaps of their own).  With ``warm_ms`` > 0, untimed
    launches continue after the ``warmup`` ones until that much GPU time has
    passed since the first of them.
    """
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    i = 0
    for _ in range(max(warmup, 1 if warm_ms > 0 else 0)):
        launch(i)
        i += 1
    e1.record()
    torch.cuda.synchronize()
    if warm_ms > 0:
        done = e0.elapsed_time(e1)
        if done < warm_ms:
            for _ in range(min(math.ceil((warm_ms - done) / max(done / i, 1e-3)), WARM_MAX_LAUNCHES)):
                launch(i)
                i += 1
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for k in range(n_steps):
        launch(i + k)
    t1.record()
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1)
    return total, total / n_steps


def bench_decode(dev, steps, warmup, B=256, HQ=4, HV=8, sets=4, qk_l2norm=False,
                 warm_ms=WARM_MS):
    x = ginp.decode_inputs(B, HQ, HV, seed=1001)
    g = _to(x, dev)
    states = [g["state"]] + [g["state"].clone() for _ in range(sets - 1)]
    outs = [torch.empty_like(g["state"]) for _ in range(sets)]
    o = torch.empty(B, 1, HV, D, dtype=torch.bfloat16, device=dev)
    steps_ = [gdec.PreparedDecode(g["q"], g["k"], g["v"], states[j], g["A_log"], g["a"],
                                  g["dt_bias"], g["b"], g["scale"], o, outs[j],
                                  qk_l2norm=qk_l2norm)
              for j in range(sets)]

    def launch(i):
        steps_[i % sets]()

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    nbytes = decode_bytes(B, HQ, HV)
    return dict(total_ms=total_ms, kernel_ms=kern_ms, bytes=nbytes)


def bench_decode_pool(dev, steps, warmup, B=1024, HQ=16, HV=32, warm_ms=WARM_MS):
    """One decode step of batch B against a [B, HV, 128, 128] pool (slot ids a
    random permutation), updated in place."""
    x = ginp.decode_inputs(B, HQ, HV, seed=1004, with_state=False)
    g = _to(x, dev)
    gen = torch.Generator(device=dev).manual_seed(1004)
    pool = torch.randn(B, HV, D, D, device=dev, generator=gen) * 0.02
    slots = torch.randperm(B, generator=torch.Generator().manual_seed(1004)).to(torch.int32).to(dev)
    o = torch.empty(B, 1, HV, D, dtype=torch.bfloat16, device=dev)

    def launch(i):
        gdec.decode_pool_(g["q"], g["k"], g["v"], pool, slots, g["A_log"], g["a"], g["dt_bias"],
                          g["b"], g["scale"], output=o)

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    return dict(total_ms=total_ms, kernel_ms=kern_ms, bytes=decode_bytes(B, HQ, HV) + 4 * B)


def decode_multi_bytes(B: int, T: int, HQ: int, HV: int) -> int:
    """State read + write once, per-token inputs and outputs T times."""
    return B * HV * 2 * D * D * 4 + T * B * (HV * (2 * D * 2 + 4) + HQ * 2 * D * 2)


def bench_decode_multi(dev, steps, warmup, B=256, T=4, HQ=4, HV=8, sets=4,
                       warm_ms=WARM_MS):
    x = ginp.decode_multi_inputs(B, T, HQ, HV, seed=1006)
    g = _to(x, dev)
    states = [g["state"]] + [g["state"].clone() for _ in range(sets - 1)]
    outs = [torch.empty_like(g["state"]) for _ in range(sets)]
    o = torch.empty(B, T, HV, D, dtype=torch.bfloat16, device=dev)
    calls = [gdec.PreparedDecodeMulti(g["q"], g["k"], g["v"], states[j], g["A_log"], g["a"],
                                      g["dt_bias"], g["b"], g["scale"], o, outs[j])
             for j in range(sets)]

    def launch(i):
        calls[i % sets]()

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    return dict(total_ms=total_ms, kernel_ms=kern_ms, bytes=decode_multi_bytes(B, T, HQ, HV), B=B,
                T=T)


def bench_prefill(dev, steps, warmup, name="prefill_varlen8_t32768_qk16_v32", qk_l2norm=False,
                  warm_ms=WARM_MS):
    w = ginp.WORKLOADS[name]
    lens = ginp.workload_lengths(name)
    x = ginp.prefill_inputs(lens, w["HQ"], w["HV"], seed=w["seed"], with_state=w["with_state"],
                            cu_dtype=w.get("cu_dtype", torch.int64))
    g = _to(x, dev)
    T = sum(lens)
    N = len(lens)
    out = torch.empty(T, w["HV"], D, dtype=torch.bfloat16, device=dev)
    fs = torch.empty(N, w["HV"], D, D, dtype=torch.float32, device=dev)

    call = gpre.PreparedPrefill(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                g["dt_bias"], g["b"], g["cu_seqlens"], g["scale"], out, fs,
                                qk_l2norm=qk_l2norm)

    def launch(i):
        call()

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    return dict(total_ms=total_ms, kernel_ms=kern_ms, T=T, N=N, lens=lens, HQ=w["HQ"],
                HV=w["HV"], flops=prefill_flops(T, w["HV"]),
                flops_qk_shared=prefill_flops(T, w["HV"], qk_shared=True),
                path=call.path, kernels=call.plan.kernels)


# Fused prefill over sequences of one length, qk16/v32: the chunk period at
# 32 / 128 / 256 chains, and the launch's fixed cost (one chunk per chain).
OCCUPANCY_WORKLOADS = (("1x5348", [5348]), ("4x5348", [5348] * 4), ("8x5348", [5348] * 8),
                       ("8x64", [64] * 8))


def bench_prefill_occupancy(dev, steps, warmup, HQ=16, HV=32, warm_ms=WARM_MS):
    res = {}
    for tag, lens in OCCUPANCY_WORKLOADS:
        x = ginp.prefill_inputs(lens, HQ, HV, seed=1004, with_state=True)
        g = _to(x, dev)
        T, N = sum(lens), len(lens)
        out = torch.empty(T, HV, D, dtype=torch.bfloat16, device=dev)
        fs = torch.empty(N, HV, D, D, dtype=torch.float32, device=dev)
        args = [g[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b",
                               "cu_seqlens")]
        _, kern_ms = timed_launches(
            lambda i: gpre.gdn_prefill(*args, g["scale"], output=out, final_state=fs,
                                       validate=False, path="fused"), steps, warmup, warm_ms)
        chunks = max((n + C - 1) // C for n in lens)
        res[tag] = {"chains": N * HV, "chunks_per_chain": chunks,
                    "kernel_us": round(kern_ms * 1e3, 2),
                    "us_per_chunk": round(kern_ms * 1e3 / chunks, 3)}
        print(f"# occupancy {tag}: {N * HV} chains, {kern_ms * 1e3:.1f} us, "
              f"{kern_ms * 1e3 / chunks:.2f} us per chunk", file=sys.stderr, flush=True)
    return res


def bench_prefill_h(dev, steps, warmup, name="prefill_varlen8_t32768_qk16_v32", path="fused",
                    slices=8, warm_ms=WARM_MS):
    """The prefill that also writes the state entering every chunk (bf16 h), on
    the given path (the split path with its workspace allocated once)."""
    w = ginp.WORKLOADS[name]
    lens = ginp.workload_lengths(name)
    x = ginp.prefill_inputs(lens, w["HQ"], w["HV"], seed=w["seed"], with_state=w["with_state"])
    g = _to(x, dev)
    T = sum(lens)
    N = len(lens)
    out = torch.empty(T, w["HV"], D, dtype=torch.bfloat16, device=dev)
    fs = torch.empty(N, w["HV"], D, D, dtype=torch.float32, device=dev)
    NT = gpre.num_chunks(g["cu_seqlens"], T)
    h = torch.empty(NT, w["HV"], D, D, dtype=torch.bfloat16, device=dev)
    args = [g[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    ws = None
    if path == "split":
        ws = torch.empty(gpre.split_workspace_bytes(N, T, w["HQ"], w["HV"]), dtype=torch.uint8,
                         device=dev)

    def launch(i):
        gpre.gdn_prefill(*args, g["scale"], output=out, final_state=fs, validate=False, h=h,
                         path=path, slices=slices, workspace=ws)

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    return dict(total_ms=total_ms, kernel_ms=kern_ms, chunks=NT, h_bytes=h.numel() * 2)


# MFMA products the backward executes per (64-token chunk, v-head): 656 in the
# transition kernel, 256 in the reverse chain, 1360 in the gradient kernel,
# each a 16x16x32 product of 16 384 flops (dense tiles as launched).
BWD_MFMA_PER_CHUNK_HEAD = 656 + 256 + 1360


def bench_backward(dev, steps, warmup, name="prefill_varlen8_t32768_qk16_v32",
                   warm_ms=WARM_MS):
    """Backward of the prefill (gdn_prefill_bwd: transition, reverse chain,
    per-chunk gradients) from the forward's h, one C call per step."""
    w = ginp.WORKLOADS[name]
    lens = ginp.workload_lengths(name)
    x = ginp.prefill_inputs(lens, w["HQ"], w["HV"], seed=w["seed"], with_state=w["with_state"])
    g = _to(x, dev)
    T, N, HQ, HV = sum(lens), len(lens), w["HQ"], w["HV"]
    args = [g[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    _, _, h = gpre.gdn_prefill_h(*args, g["scale"])
    gen = torch.Generator(device=dev).manual_seed(17)
    d_out = torch.randn(T, HV, D, device=dev, generator=gen).to(torch.bfloat16)
    d_fin = torch.randn(N, HV, D, D, device=dev, generator=gen) * 0.1
    outs = [torch.empty(T, HQ, D, device=dev), torch.empty(T, HQ, D, device=dev),
            torch.empty(T, HV, D, device=dev), torch.empty(T, HV, device=dev),
            torch.empty(T, HV, device=dev), torch.empty(N, HV, D, D, device=dev)]
    need = gbwd.workspace_bytes(N, T, HQ, HV)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    lib = gpre._capi.lib()
    p = gpre._capi.ptr
    cu = g["cu_seqlens"]
    call = (p(g["q"]), p(g["k"]), p(g["v"]), p(g["A_log"]), p(g["a"]), p(g["dt_bias"]), p(g["b"]),
            p(cu), 1 if cu.dtype == torch.int32 else 0, N, T, HQ, HV, float(g["scale"]), p(h),
            h.shape[0], p(d_out), p(d_fin), *[p(o) for o in outs], p(ws), need,
            gpre._capi.stream_handle(dev))

    def launch(i):
        lib.gdn_prefill_bwd(*call)

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    flops = h.shape[0] * HV * BWD_MFMA_PER_CHUNK_HEAD * 16384
    return dict(kernel_ms=kern_ms, T=T, N=N, HQ=HQ, HV=HV, chunks=h.shape[0], flops=flops,
                ws_bytes=need)


def bench_run_latency(dev, kernel_us, reps=50):
    """End-to-end latency of the reference-compatible ``run`` entry points
    (validation, allocation of the outputs, the ctypes call, the kernels):
    ``run_us`` with a synchronisation after every call (the median over
    ``reps`` calls), ``back_to_back_us`` per call over ``reps`` calls issued
    back to back with one synchronisation at the end (the host work of a call
    overlaps the previous call's kernels), beside the kernel time alone.
    Prefill ``run`` reads cu_seqlens back once per tensor and version (the
    reference's ``cu_seqlens[-1] == T`` check), so repeated calls on the same
    inputs do not synchronise."""
    res = {}

    def median_call_us(fn):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append((time.perf_counter() - t0) * 1e6)
        ts.sort()
        return ts[len(ts) // 2]

    def back_to_back_us(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / reps

    def record(name, fn):
        us = median_call_us(fn)
        b2b = back_to_back_us(fn)
        k = kernel_us.get(name)
        res[name] = {"run_us": round(us, 1), "back_to_back_us": round(b2b, 1), "kernel_us": k,
                     "host_overhead_us": None if k is None else round(us - k, 1)}

    for name, B in (("decode_b1_qk4_v8", 1), ("decode_b256_qk4_v8", 256)):
        g = _to(ginp.decode_inputs(B, 4, 8, seed=1000 if B == 1 else 1001), dev)
        record(name, lambda: gdec.run(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                      g["dt_bias"], g["b"], g["scale"]))
    for name in ("prefill_t4096_n1_qk4_v8", "prefill_varlen16_qk4_v8"):
        w = ginp.WORKLOADS[name]
        x = ginp.prefill_inputs(ginp.workload_lengths(name), w["HQ"], w["HV"], seed=w["seed"],
                                with_state=w["with_state"], cu_dtype=w.get("cu_dtype", torch.int64))
        g = _to(x, dev)
        record(name, lambda: gpre.run(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                      g["dt_bias"], g["b"], g["cu_seqlens"], g["scale"]))
    res["decode_b1_qk4_v8"]["graph_step_us"] = round(graph_decode_step_us(dev), 2)
    return res


def graph_decode_step_us(dev, B=1, steps=32, replays=50):
    """Decode steps at batch B replayed from one HIP graph (a serving loop's
    way past the host cost of a call): ``steps`` prepared decode calls that
    alternate two state buffers are captured once; the time per step over
    ``replays`` back-to-back replays."""
    g = _to(ginp.decode_inputs(B, 4, 8, seed=1000), dev)
    states = [g["state"], torch.empty_like(g["state"])]
    out = torch.empty(B, 1, 8, D, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        calls = [gdec.PreparedDecode(g["q"], g["k"], g["v"], states[i % 2], g["A_log"], g["a"],
                                     g["dt_bias"], g["b"], g["scale"], out, states[(i + 1) % 2])
                 for i in range(steps)]
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for c in calls:
            c()
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e6 / (replays * steps)


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def bench_conv(dev, steps, warmup, HQ=16, HV=32, W=4, warm_ms=WARM_MS):
    """q/k/v causal conv1d + SiLU over the 32 768-token, 8-sequence workload at
    qk16 / v32 (C = 8192 channels), written as GDN's q, k, v.  Algorithmic
    bytes: x read once, q/k/v written once, conv states read and written."""
    lens = ginp.workload_lengths("prefill_varlen8_t32768_qk16_v32")
    T, N = sum(lens), len(lens)
    C = 256 * HQ + 128 * HV
    gen = torch.Generator(device=dev).manual_seed(90)
    x = torch.randn(T, C, device=dev, generator=gen).to(torch.bfloat16)
    w = torch.randn(C, W, device=dev, generator=gen) * 0.5
    st = torch.randn(N, C, W - 1, device=dev, generator=gen).to(torch.bfloat16)
    cu = torch.zeros(N + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    cu = cu.to(dev)
    q = torch.empty(T, HQ, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(T, HV, D, dtype=torch.bfloat16, device=dev)
    fin = torch.empty_like(st)
    lib = gconv._capi.lib()
    p = gconv._capi.ptr
    args = (p(x), p(w), None, p(cu), 0, N, T, C, W, p(st), p(fin), W - 1, p(q), p(k), p(v),
            D * HQ, D * HQ, gconv._capi.GDN_ACT_SILU, gconv._capi.stream_handle(dev))

    def launch(i):
        lib.gdn_qkv_conv1d_fwd(*args)

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    nbytes = 2 * T * C * 2 + 2 * N * C * (W - 1) * 2
    return dict(kernel_ms=kern_ms, bytes=nbytes, T=T, C=C)


def bench_conv_update(dev, steps, warmup, B=1024, HQ=16, HV=32, W=4, warm_ms=WARM_MS):
    """Decode conv update at batch 1024, qk16 / v32: one token per sequence,
    the [1024, 8192, 3] bf16 conv state updated in place."""
    C = 256 * HQ + 128 * HV
    gen = torch.Generator(device=dev).manual_seed(91)
    x = torch.randn(B, C, device=dev, generator=gen).to(torch.bfloat16)
    w = torch.randn(C, W, device=dev, generator=gen) * 0.5
    st = torch.randn(B, C, W - 1, device=dev, generator=gen).to(torch.bfloat16)
    q = torch.empty(B, 1, HQ, D, dtype=torch.bfloat16, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(B, 1, HV, D, dtype=torch.bfloat16, device=dev)
    lib = gconv._capi.lib()
    p = gconv._capi.ptr
    args = (p(x), p(w), None, p(st), W - 1, None, B, B, C, W, p(q), p(k), p(v), D * HQ, D * HQ,
            gconv._capi.GDN_ACT_SILU, gconv._capi.stream_handle(dev))

    def launch(i):
        lib.gdn_qkv_conv1d_update(*args)

    total_ms, kern_ms = timed_launches(launch, steps, warmup, warm_ms)
    nbytes = 2 * B * C * 2 + 2 * B * C * (W - 1) * 2
    return dict(kernel_ms=kern_ms, bytes=nbytes, B=B, C=C)


def cpu_baseline_decode_b1(budget_s=2.0):
    """Oracle decode step in fp32 at batch 1 (the workload with one sequence,
    qk4/v8): microseconds per step on the host cores."""
    from oracle import gdn_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    x = ginp.decode_inputs(1, 4, 8, seed=1000)
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
    for _ in range(3):
        O.decode_step(*args, x["scale"], dtype=torch.float32)
    n, t0 = 0, time.perf_counter()
    while True:
        O.decode_step(*args, x["scale"], dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 2000:
            break
    return {"value": round(el / n * 1e6, 1), "unit": "us/step", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{n} fp32 oracle decode steps at B=1 qk4/v8 ({el:.1f} s)"}


def cpu_baseline_decode(budget_s=12.0, B=256):
    """Oracle decode step in fp32 on the host cores (bounded sample of B=256)."""
    from oracle import gdn_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    x = ginp.decode_inputs(B, 4, 8, seed=1001)
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
    O.decode_step(*args, x["scale"], dtype=torch.float32)          # warmup
    n, t0 = 0, time.perf_counter()
    while True:
        O.decode_step(*args, x["scale"], dtype=torch.float32)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 400:
            break
    gbs = decode_bytes(B, 4, 8) * n / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{n} fp32 oracle decode steps at B=256 qk4/v8 ({el:.1f} s)"}


def cpu_baseline_prefill_chunked():
    """Chunked (64-token WY) fp32 oracle form over the whole 32 768-token
    qk16 / v32 workload, once: the second CPU line beside the per-token form."""
    from oracle import gdn_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    name = "prefill_varlen8_t32768_qk16_v32"
    w = ginp.WORKLOADS[name]
    lens = ginp.workload_lengths(name)
    x = ginp.prefill_inputs(lens, w["HQ"], w["HV"], seed=w["seed"], with_state=w["with_state"])
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    t0 = time.perf_counter()
    O.prefill_chunked(*args, x["scale"], dtype=torch.float32)
    el = time.perf_counter() - t0
    toks = sum(lens)
    return {"value": round(toks / el, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"the full {toks}-token qk16/v32 workload once, fp32 chunked oracle "
                      f"(64-token chunks) ({el:.1f} s)"}


def cpu_baseline_prefill():
    """Per-token fp32 oracle recurrence (definition-reference style) over the whole
    32 768-token qk16 / v32 workload, once."""
    from oracle import gdn_oracle as O

    torch.set_num_threads(os.cpu_count() or 1)
    name = "prefill_varlen8_t32768_qk16_v32"
    w = ginp.WORKLOADS[name]
    lens = ginp.workload_lengths(name)
    x = ginp.prefill_inputs(lens, w["HQ"], w["HV"], seed=w["seed"], with_state=w["with_state"])
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    t0 = time.perf_counter()
    O.prefill_recurrent(*args, x["scale"], dtype=torch.float32)
    el = time.perf_counter() - t0
    toks = sum(lens)
    return {"value": round(toks / el, 1), "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"the full {toks}-token qk16/v32 workload once, fp32 per-token oracle "
                      f"recurrence ({el:.1f} s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prefill-steps", type=int, default=30)
    ap.add_argument("--only", choices=["all", "decode", "prefill", "conv", "backward",
                                       "occupancy"],
                    default="all",
                    help="occupancy (never part of 'all'): the fused prefill's chunk period at "
                         "32 / 128 / 256 chains of equal length")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-latency", action="store_true",
                    help="skip the end-to-end run() latency measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 5 plain 256 MiB device copies (the reference kernel that "
                         "scales FETCH_SIZE / WRITE_SIZE counter readings to bytes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the GDN operators shard with no communication "
              "(per sequence / per head), so a multi-GPU figure is not measured here.",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    line = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "warm_ms": WARM_MS, "ms_per_step": None,
            "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "decode_b256_qk4_v8", "batch": 256, "qk_heads": 4,
                       "v_heads": 8, "head_dim": 128, "state": "fp32 [256,8,128,128] k-last",
                       "state_buffer_sets": 4}}

    if args.only in ("all", "decode"):
        # the headline: exactly --warmup untimed steps (decode is HBM-bound; a
        # WARM_MS warm-up moves it by under 1%)
        r = bench_decode(dev, args.steps, args.warmup, warm_ms=0.0)
        ms = r["total_ms"] / args.steps
        gbs = r["bytes"] / (ms * 1e-3) / 1e9
        kgbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
        line.update(value=round(gbs, 1), ms_per_step=round(ms, 5))
        line["roofline"] = {"bound": "hbm", "achieved": round(kgbs, 1), "peak": HBM_PEAK_GBS,
                            "unit": "GB/s", "frac": round(kgbs / HBM_PEAK_GBS, 4),
                            "traffic": _traffic("gdn_decode_kernel_b256"),
                            "kernel": "gdn_decode_kernel", "bytes_per_launch": r["bytes"],
                            "kernel_us": round(r["kernel_ms"] * 1e3, 2)}
        print(f"# decode B=256: {ms*1e3:.2f} us/step, kernel {r['kernel_ms']*1e3:.2f} us, "
              f"{kgbs:.0f} GB/s ({kgbs/HBM_PEAK_GBS*100:.1f}% of HBM peak)",
              file=sys.stderr, flush=True)
        # multi-token decode (4 tokens per sequence per launch; an extension)
        r = bench_decode_multi(dev, args.steps // 2, args.warmup)
        kus = r["kernel_ms"] * 1e3
        mgbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
        line["decode_multi"] = {
            "workload": "decode_multi_b256_t4_qk4_v8", "batch": r["B"], "tokens_per_seq": r["T"],
            "kernel_us": round(kus, 2), "tokens_per_s": round(r["B"] * r["T"] / (kus * 1e-6), 1),
            "single_step_us_x4": round(4 * line["roofline"]["kernel_us"], 2),
            "roofline": {"bound": "hbm", "achieved": round(mgbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(mgbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": r["bytes"]}}
        print(f"# decode multi B=256 T=4: kernel {kus:.2f} us ({mgbs:.0f} GB/s of algorithmic "
              f"bytes) vs 4 single steps {4 * line['roofline']['kernel_us']:.1f} us",
              file=sys.stderr, flush=True)
        # slot-pool decode at batch 1024, qk16/v32 (a [1024, 32, 128, 128] pool, 2 GiB)
        r = bench_decode_pool(dev, max(args.steps // 10, 5), args.warmup)
        pgbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
        line["decode_pool"] = {
            "workload": "decode_pool_b1024_qk16_v32", "batch": 1024, "pool": [1024, 32, 128, 128],
            "kernel_us": round(r["kernel_ms"] * 1e3, 2),
            "roofline": {"bound": "hbm", "achieved": round(pgbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(pgbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": r["bytes"]}}
        print(f"# decode pool B=1024 qk16/v32: {r['kernel_ms'] * 1e3:.1f} us, {pgbs:.0f} GB/s "
              f"({pgbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak)", file=sys.stderr, flush=True)
        # the in-kernel q/k L2-normalisation option on the same inputs
        r = bench_decode(dev, args.steps // 2, args.warmup, qk_l2norm=True)
        line["decode_qk_l2norm"] = {"workload": "decode_b256_qk4_v8",
                                    "kernel_us": round(r["kernel_ms"] * 1e3, 2),
                                    "decode_kernel_us": line["roofline"]["kernel_us"]}
        print(f"# decode with q/k L2-norm: {r['kernel_ms'] * 1e3:.2f} us", file=sys.stderr,
              flush=True)

    if args.only in ("all", "prefill"):
        try:
            r = bench_prefill(dev, args.prefill_steps, PREFILL_WARMUP)
            ms = r["total_ms"] / args.prefill_steps
            tfl = r["flops"] / (r["kernel_ms"] * 1e-3) / 1e12
            line["prefill"] = {
                "workload": "prefill_varlen8_t32768_qk16_v32", "tokens": r["T"],
                "seq_lens": r["lens"], "qk_heads": r["HQ"], "v_heads": r["HV"],
                "tokens_per_s": round(r["T"] / (ms * 1e-3), 1), "ms_per_step": round(ms, 4),
                "steps": args.prefill_steps, "dtype": "fp16 MFMA operands, fp32 accumulate",
                "roofline": {"bound": "mfma", "achieved": round(tfl, 2),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tfl / MFMA_BF16_PEAK_TFLOPS, 4),
                             "flops_per_launch": r["flops"],
                             "frac_qk_shared_count": round(
                                 r["flops_qk_shared"] / (r["kernel_ms"] * 1e-3) / 1e12
                                 / MFMA_BF16_PEAK_TFLOPS, 4),
                             "traffic": _traffic("gdn_prefill_t32768_qk16_v32"),
                             "kernel_us": round(r["kernel_ms"] * 1e3, 2)},
            }
            print(f"# prefill 32k qk16/v32: {ms*1e3:.1f} us/step, {tfl:.1f} TFLOP/s "
                  f"({tfl/MFMA_BF16_PEAK_TFLOPS*100:.1f}% of bf16 MFMA peak)",
                  file=sys.stderr, flush=True)
        except Exception as e:  # prefill not available: say so in the line
            line["prefill"] = {"error": f"{type(e).__name__}: {e}"}
            print(f"# prefill failed: {e}", file=sys.stderr, flush=True)
        if "error" not in line["prefill"]:
            # per-chunk states as well (the h a training backward reads; an option)
            r = bench_prefill_h(dev, args.prefill_steps, PREFILL_WARMUP)
            kus = r["kernel_ms"] * 1e3
            line["prefill_h"] = {
                "workload": "prefill_varlen8_t32768_qk16_v32", "chunks": r["chunks"],
                "h_bytes": r["h_bytes"], "kernel_us": round(kus, 2),
                "prefill_kernel_us": line["prefill"]["roofline"]["kernel_us"],
                "h_write_GBs": round(r["h_bytes"] / (r["kernel_ms"] * 1e-3) / 1e9, 1)}
            print(f"# prefill with h (bf16, {r['chunks']} chunks, {r['h_bytes'] / 1e6:.0f} MB): "
                  f"{kus:.1f} us against {line['prefill']['roofline']['kernel_us']:.1f} us without",
                  file=sys.stderr, flush=True)
            # the same at one 4096-token sequence (qk4/v8), on the split path the
            # length-based choice takes (the training forward of a few long chains)
            r = bench_prefill_h(dev, args.prefill_steps, PREFILL_WARMUP,
                                name="prefill_t4096_n1_qk4_v8", path="split", slices=8)
            line["prefill_h_t4096_n1_qk4_v8"] = {
                "workload": "prefill_t4096_n1_qk4_v8", "path": "split8", "chunks": r["chunks"],
                "h_bytes": r["h_bytes"], "kernel_us": round(r["kernel_ms"] * 1e3, 2),
                "time_basis": "both launches of one call"}
            print(f"# prefill with h, 4096 tokens (split8): {r['kernel_ms'] * 1e3:.1f} us",
                  file=sys.stderr, flush=True)
            # the in-kernel q/k L2-normalisation option on the same inputs
            r = bench_prefill(dev, args.prefill_steps, PREFILL_WARMUP, qk_l2norm=True)
            line["prefill_qk_l2norm"] = {
                "workload": "prefill_varlen8_t32768_qk16_v32", "kernel_us": round(r["kernel_ms"] * 1e3, 2),
                "prefill_kernel_us": line["prefill"]["roofline"]["kernel_us"]}
            print(f"# prefill with q/k L2-norm: {r['kernel_ms'] * 1e3:.1f} us", file=sys.stderr,
                  flush=True)
            # the two qk4/v8 prefill workloads: one 4096-token sequence, and 16
            # varlen sequences (lengths ~ U[128, 8192]) with initial states
            for name in ("prefill_t4096_n1_qk4_v8", "prefill_varlen16_qk4_v8"):
                r = bench_prefill(dev, args.prefill_steps, PREFILL_WARMUP, name=name)
                kus = r["kernel_ms"] * 1e3
                tfl = r["flops"] / (r["kernel_ms"] * 1e-3) / 1e12
                kernels = r["kernels"]
                line[name] = {
                    "workload": name, "tokens": r["T"], "sequences": r["N"], "qk_heads": r["HQ"],
                    "v_heads": r["HV"], "path": r["path"], "kernel_us": round(kus, 2),
                    "tokens_per_s": round(r["T"] / (r["kernel_ms"] * 1e-3), 1),
                    "roofline": {"bound": "mfma", "achieved": round(tfl, 2),
                                 "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(tfl / MFMA_BF16_PEAK_TFLOPS, 4),
                                 "flops_per_launch": r["flops"], "kernels": kernels,
                                 "time_basis": "every launch of one call" if len(kernels) > 1
                                 else "one launch"}}
                tag = "split" if r["path"].startswith("split") else "fused"
                tr = _traffic(f"gdn_prefill_{tag}_" + name[len("prefill_"):], path=r["path"])
                if tr is not None:
                    line[name]["roofline"]["traffic"] = tr
                print(f"# {name} ({r['path']}): {kus:.1f} us, {tfl:.1f} TFLOP/s "
                      f"({tfl / MFMA_BF16_PEAK_TFLOPS * 100:.2f}% of bf16 MFMA peak)",
                      file=sys.stderr, flush=True)

    if args.only in ("all", "backward"):
        for key, name in (("prefill_backward", "prefill_varlen8_t32768_qk16_v32"),
                          ("prefill_backward_t4096_n1_qk4_v8", "prefill_t4096_n1_qk4_v8")):
            r = bench_backward(dev, 10, 3, name=name)
            kus = r["kernel_ms"] * 1e3
            tfl = r["flops"] / (r["kernel_ms"] * 1e-3) / 1e12
            line[key] = {
                "workload": name, "tokens": r["T"], "sequences": r["N"], "qk_heads": r["HQ"],
                "v_heads": r["HV"], "kernel_us": round(kus, 2),
                "tokens_per_s": round(r["T"] / (r["kernel_ms"] * 1e-3), 1),
                "kernels": ["gdn_bwd_prep_kernel", "gdn_bwd_chain_kernel", "gdn_bwd_grad_kernel"],
                "roofline": {"bound": "mfma", "achieved": round(tfl, 2),
                             "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tfl / MFMA_BF16_PEAK_TFLOPS, 4),
                             "flops_per_launch": r["flops"],
                             "flops_basis": "executed bf16 MFMA products, 2272 per chunk and v-head",
                             "time_basis": "all launches of one call"}}
            if key == "prefill_backward":
                tr = _traffic("gdn_prefill_bwd_t32768_qk16_v32")
                if tr is not None:
                    line[key]["roofline"]["traffic"] = tr
            print(f"# backward {name}: {kus:.1f} us, {tfl:.1f} TFLOP/s "
                  f"({tfl / MFMA_BF16_PEAK_TFLOPS * 100:.1f}% of bf16 MFMA peak)",
                  file=sys.stderr, flush=True)

    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_calibration_bytes"] = src.numel() * 4

    if args.only in ("all", "conv"):
        for key, fn, wl in (("qkv_conv1d", bench_conv, "conv1d_varlen8_t32768_qk16_v32"),
                            ("qkv_conv1d_update", bench_conv_update, "conv1d_update_b1024_qk16_v32")):
            r = fn(dev, 30, 10)
            gbs = r["bytes"] / (r["kernel_ms"] * 1e-3) / 1e9
            line[key] = {"workload": wl, "channels": r["C"], "kernel_us": round(r["kernel_ms"] * 1e3, 2),
                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                      "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                                      "bytes_per_launch": r["bytes"]}}
            print(f"# {key}: {r['kernel_ms'] * 1e3:.1f} us, {gbs:.0f} GB/s "
                  f"({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak)", file=sys.stderr, flush=True)

    if args.only == "occupancy":
        line["prefill_occupancy"] = bench_prefill_occupancy(dev, args.prefill_steps,
                                                            PREFILL_WARMUP)

    if args.only == "all" and not args.no_latency:
        kus = {"decode_b256_qk4_v8": line.get("roofline", {}).get("kernel_us"),
               "prefill_t4096_n1_qk4_v8": line.get("prefill_t4096_n1_qk4_v8", {}).get("kernel_us"),
               "prefill_varlen16_qk4_v8": line.get("prefill_varlen16_qk4_v8", {}).get("kernel_us")}
        r1 = bench_decode(dev, 50, 10, B=1, sets=1, warm_ms=0.0)   # launch-bound: no warm-up
        kus["decode_b1_qk4_v8"] = round(r1["kernel_ms"] * 1e3, 2)
        line["run_latency"] = bench_run_latency(dev, kus)
        print(f"# run latency: {json.dumps(line['run_latency'])}", file=sys.stderr, flush=True)

    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_decode()
        line["cpu_baseline"]["cpu_model"] = cpu_model()
        line["cpu_baseline"]["decode_b1"] = cpu_baseline_decode_b1()
        if args.only in ("all", "prefill") and "error" not in line.get("prefill", {"error": 1}):
            line["prefill"]["cpu_baseline"] = cpu_baseline_prefill()
            line["prefill"]["cpu_baseline"]["cpu_model"] = line["cpu_baseline"]["cpu_model"]
            line["prefill"]["cpu_baseline"]["chunked"] = cpu_baseline_prefill_chunked()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
