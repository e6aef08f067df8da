"""GPU parity of the fused prefill kernel with seams (the longest sequences
cut in two in time, their tails run from a zero state and as the transition
chain on CUs that shorter chains free, joined by the seam pass), planned on
the host from the lengths (gdn_prefill_plan / gdn_prefill_plan_fwd).

Bars as the other prefill tests: output (bf16) within atol = rtol = 1e-2 of
the fp64 oracle, final state relative error (Frobenius, per sequence and
overall) <= 1e-3; against the same call with every chain whole (the serial
fused kernel) within the same bars.
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

STATE_REL_BAR = 1e-3
NAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _check(o, s, o_ref, s_ref):
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    s = s.cpu().double()
    rel = float((s - s_ref).norm() / s_ref.norm().clamp_min(1e-300))
    assert rel <= STATE_REL_BAR, rel
    for n in range(s.shape[0]):
        nr = float(s_ref[n].norm())
        if nr > 0:
            assert float((s[n] - s_ref[n]).norm()) / nr <= STATE_REL_BAR, n
        else:
            assert float(s[n].abs().max()) == 0.0
    return rel


def _oracle(x):
    x64 = dict(x, cu_seqlens=x["cu_seqlens"].long())
    return O.prefill_recurrent(*[x64[n] for n in NAMES], x["scale"])


def _run(g, **kw):
    pre = pkg_module("prefill")
    return pre.gdn_prefill(*[g[n] for n in NAMES], g["scale"], **kw)


# (lengths, HQ, HV, initial states, int32 cu_seqlens, q/k L2-norm option)
CASES = [
    ([4096], 4, 8, False, False, False),                       # one chain set, half cut
    ([3000, 300, 1100, 77], 4, 8, True, True, False),          # ragged tails, a short sequence
    ([2500, 2300, 640, 1000, 130, 0, 900], 4, 8, True, False, False),   # two seams, an empty sequence
    ([1900, 450, 1700], 16, 32, True, False, False),            # qk16 / v32
    ([2222, 600], 4, 8, True, False, True),                     # L2-norm option
    ([3000, 200, 1300], 1, 4, True, False, False),              # one qk-head, 4 v-heads
    ([2700, 90, 2000, 640], 2, 8, False, True, False),          # two qk-heads, seam units across XCDs
]


@pytest.mark.parametrize("lens,HQ,HV,with_state,cu32,l2", CASES)
def test_fused_seams_match_oracle(device, lens, HQ, HV, with_state, cu32, l2):
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    print(f"fused seams lens={lens} HQ={HQ} HV={HV} l2={l2}", flush=True)
    x = inp.prefill_inputs(lens, HQ=HQ, HV=HV, seed=sum(lens) + 23, with_state=with_state,
                           cu_dtype=torch.int32 if cu32 else torch.int64)
    if l2:
        # unnormalised q / k rows: the kernel normalises them
        x["q"] = (x["q"].float() * 3.0).to(torch.bfloat16)
        x["k"] = (x["k"].float() * 0.5).to(torch.bfloat16)
    plan = pre.Plan(x["cu_seqlens"], sum(lens), HQ, HV, fused=True)
    assert plan.slices == 0 and plan.seams >= 1, (plan.path, plan.seams)
    assert plan.workspace_bytes > 0
    g = _to(x, device)
    o, s = _run(g, path="fused", qk_l2norm=l2)
    o1, s1 = _run(g, path="fused", qk_l2norm=l2, seams=False)
    torch.cuda.synchronize()
    o_ref, s_ref = _oracle(dict(x, q=O.qk_l2norm(x["q"]), k=O.qk_l2norm(x["k"])) if l2 else x)
    _check(o, s, o_ref, s_ref)
    _check(o1, s1, o_ref, s_ref)
    assert float((s - s1).norm() / s1.norm()) <= STATE_REL_BAR
    torch.testing.assert_close(o.float(), o1.float(), atol=1e-2, rtol=1e-2)
    # outside the cut sequences' tails the outputs are the serial kernel's
    cu = x["cu_seqlens"].long()
    split = torch.zeros(sum(lens), dtype=torch.bool)
    ref_o = o1.float().cpu()
    got_o = o.float().cpu()
    for n in range(len(lens)):
        b0, b1 = int(cu[n]), int(cu[n + 1])
        if b1 - b0 > 64 * plan.split_chunk and plan.split_chunk > 0:
            split[b0 + 64 * plan.split_chunk:b1] = True
    assert torch.equal(got_o[~split], ref_o[~split])


def test_fused_seams_repeat_calls_and_stale_workspace(device):
    """Nothing in the seam region has to start cleared: two calls on one
    workspace filled with garbage (NaN bytes) give the same results bit for
    bit, and a call on other lengths in between leaves the next one intact."""
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    lens = [2600, 500, 1300]
    x = inp.prefill_inputs(lens, seed=4242, with_state=True)
    g = _to(x, device)
    plan = pre.Plan(x["cu_seqlens"], sum(lens), 4, 8, fused=True)
    assert plan.seams >= 1
    ws = torch.full((plan.workspace_bytes + 4096,), 0xFF, dtype=torch.uint8, device=device)
    o, s = _run(g, path="fused", workspace=ws)
    y = inp.prefill_inputs([3100, 40], seed=77, with_state=True)
    gy = _to(y, device)
    _run(gy, path="fused", workspace=ws)
    o2, s2 = _run(g, path="fused", workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(s, s2)
    _check(o, s, *_oracle(x))


def test_plan_fwd_rejects_mismatched_plan(device):
    """A plan made for other sizes is refused before any launch."""
    pre = pkg_module("prefill")
    capi = pkg_module("_capi")
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([700, 300], seed=5)
    g = _to(x, device)
    plan = pre.Plan(torch.tensor([0, 500, 1000]), 1000, 4, 8, fused=True)
    T, N = 1000, 2
    out = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=device)
    fs = torch.empty(N, 8, 128, 128, device=device)
    P = capi.ptr
    rc = capi.lib().gdn_prefill_plan_fwd(
        P(g["q"]), P(g["k"]), P(g["v"]), P(g["state"]), P(g["A_log"]), P(g["a"]), P(g["dt_bias"]),
        P(g["b"]), P(g["cu_seqlens"]), 0, N, T, 4, 16, 1.0, P(out), P(fs), plan.buf, None, 0, 0,
        capi.stream_handle(device))
    assert rc == capi.GDN_ERR_SHAPE
    # the right sizes but no workspace for the seams
    rc = capi.lib().gdn_prefill_plan_fwd(
        P(g["q"]), P(g["k"]), P(g["v"]), P(g["state"]), P(g["A_log"]), P(g["a"]), P(g["dt_bias"]),
        P(g["b"]), P(g["cu_seqlens"]), 0, N, T, 4, 8, 1.0, P(out), P(fs), plan.buf, None, 0, 0,
        capi.stream_handle(device))
    assert plan.seams == 0 or rc == capi.GDN_ERR_WORKSPACE
