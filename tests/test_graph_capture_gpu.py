"""HIP graph capture of the prepared decode and prefill calls.

The library's launches are kernels only (no allocation, memset, copy or
synchronisation inside a call), so a serving loop can capture them in a
graph.  Each test captures one prepared call on a side stream, then replays
the graph several times; between replays the test writes fresh inputs into
the captured buffers and runs the same call eagerly into separate outputs,
and every replay must equal that eager result bit for bit.
"""

import pytest
import torch

from conftest import pkg_module

pytestmark = pytest.mark.gpu

REPLAYS = 4


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _capture(make_call):
    """Build the call on a side stream (its stream is the capture stream), run
    it once there, then capture one call into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call = make_call()
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call()
    torch.cuda.synchronize()
    return g, call


def test_decode_graph_replays_match_eager(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    B = 256
    print(f"graph capture: decode B={B} qk4/v8", flush=True)
    g = _to(inp.decode_inputs(B, seed=2101), device)
    out_g = torch.empty(B, 1, 8, 128, dtype=torch.bfloat16, device=device)
    ns_g = torch.empty(B, 8, 128, 128, dtype=torch.float32, device=device)
    graph, _ = _capture(lambda: dec.PreparedDecode(
        g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"], g["dt_bias"], g["b"], g["scale"],
        out_g, ns_g))
    for r in range(REPLAYS):
        x = _to(inp.decode_inputs(B, seed=2200 + r), device)
        for name in ("q", "k", "v", "state", "a", "b"):
            g[name].copy_(x[name])
        o_e, s_e = dec.gdn_decode(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                  g["dt_bias"], g["b"], g["scale"])
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, o_e), r
        assert torch.equal(ns_g, s_e), r


@pytest.mark.parametrize("lens,HQ,HV,fused", [
    ([4096], 4, 8, False),                    # split path, 8 slices, one seam
    ([700, 1900, 64, 0, 300], 4, 8, True),    # fused kernel with seams on idle CUs
    ([2000, 1500, 700, 128], 16, 32, False),  # the plan's choice at qk16/v32
])
def test_prefill_graph_replays_match_eager(device, lens, HQ, HV, fused):
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    print(f"graph capture: prefill lens={lens} qk{HQ}/v{HV} fused={fused}", flush=True)
    g = _to(inp.prefill_inputs(lens, HQ, HV, seed=2301, with_state=True), device)
    T, N = sum(lens), len(lens)
    out_g = torch.empty(T, HV, 128, dtype=torch.bfloat16, device=device)
    fs_g = torch.empty(N, HV, 128, 128, dtype=torch.float32, device=device)
    out_e = torch.empty_like(out_g)
    fs_e = torch.empty_like(fs_g)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    graph, call = _capture(lambda: pre.PreparedPrefill(*[g[n] for n in names], g["scale"], out_g,
                                                        fs_g, fused=fused))
    eager = pre.PreparedPrefill(*[g[n] for n in names], g["scale"], out_e, fs_e, fused=fused)
    assert eager.path == call.path
    print(f"  path {call.path}", flush=True)
    for r in range(REPLAYS):
        x = _to(inp.prefill_inputs(lens, HQ, HV, seed=2400 + r, with_state=True), device)
        for name in ("q", "k", "v", "state", "a", "b"):
            g[name].copy_(x[name])
        eager()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), r
        assert torch.equal(fs_g, fs_e), r
