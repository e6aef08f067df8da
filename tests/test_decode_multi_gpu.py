"""GPU checks of the multi-token decode (T consecutive steps per sequence in
one launch, an extension: the reference decode takes one token per call).

Bars: against the fp64 oracle stepped token by token, outputs within
atol = rtol = 1e-2 and the final state within 1e-3 relative error (the
decode bars); against T successive single-step launches, bit-identical
outputs and states (same per-token arithmetic, state kept in fp32 either way).
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _oracle_steps(x):
    """Oracle decode step (DEC:67-79) applied token by token, fp64 state carried."""
    B, T = x["q"].shape[:2]
    S = x["state"]
    outs = []
    for t in range(T):
        o, S = O.decode_step(x["q"][:, t:t + 1], x["k"][:, t:t + 1], x["v"][:, t:t + 1], S,
                             x["A_log"], x["a"][:, t:t + 1], x["dt_bias"], x["b"][:, t:t + 1],
                             x["scale"])
        outs.append(o)
    return torch.cat(outs, dim=1), S


@pytest.mark.parametrize("B,T,HQ,HV", [(1, 1, 4, 8), (3, 2, 4, 8), (5, 4, 4, 8), (2, 7, 16, 32),
                                       (4, 3, 2, 8)])
def test_decode_multi_matches_oracle(device, B, T, HQ, HV):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    print(f"decode multi B={B} T={T} HQ={HQ} HV={HV}", flush=True)
    x = inp.decode_multi_inputs(B, T, HQ=HQ, HV=HV, seed=2000 + 10 * B + T)
    g = _to(x, device)
    o, s = dec.gdn_decode_multi(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                g["dt_bias"], g["b"], g["scale"])
    torch.cuda.synchronize()
    assert o.shape == (B, T, HV, 128) and o.dtype == torch.bfloat16
    o_ref, s_ref = _oracle_steps(x)
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    s = s.cpu().double()
    rel = float((s - s_ref).norm() / s_ref.norm())
    assert rel <= 1e-3, rel


def test_decode_multi_equals_successive_steps(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    B, T = 6, 5
    x = inp.decode_multi_inputs(B, T, HQ=16, HV=32, seed=2100)
    g = _to(x, device)
    o_m, s_m = dec.gdn_decode_multi(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                    g["dt_bias"], g["b"], g["scale"])
    st = g["state"].clone()
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, st = dec.gdn_decode(g["q"][:, sl], g["k"][:, sl], g["v"][:, sl], st, g["A_log"],
                               g["a"][:, sl], g["dt_bias"], g["b"][:, sl], g["scale"])
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(o_m, torch.cat(outs, dim=1))
    assert torch.equal(s_m, st)


def test_decode_multi_none_state_inplace(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.decode_multi_inputs(3, 4, seed=2200, with_state=False)
    g = _to(x, device)
    o, s = dec.gdn_decode_multi(g["q"], g["k"], g["v"], None, g["A_log"], g["a"], g["dt_bias"],
                                g["b"], None)
    torch.cuda.synchronize()
    o_ref, s_ref = _oracle_steps(x)
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    # in place: the state buffer is both input and output
    x2 = inp.decode_multi_inputs(3, 4, seed=2201)
    g2 = _to(x2, device)
    st = g2["state"].clone()
    _, s2 = dec.gdn_decode_multi(g2["q"], g2["k"], g2["v"], st, g2["A_log"], g2["a"],
                                 g2["dt_bias"], g2["b"], g2["scale"], new_state=st)
    torch.cuda.synchronize()
    assert s2.data_ptr() == st.data_ptr()
    _, s_ref2 = _oracle_steps(x2)
    rel = float((st.cpu().double() - s_ref2).norm() / s_ref2.norm())
    assert rel <= 1e-3, rel


@pytest.mark.parametrize("T,l2", [(17, False), (17, True), (40, False), (40, True)])
def test_decode_multi_past_one_staging_block(device, T, l2):
    """T beyond the 16 tokens the kernel stages in LDS at a time: the second
    and third blocks reuse the staging buffers after a barrier and read tokens
    t0 + t.  Checked against the oracle stepped per token and, bit for bit,
    against T successive single-step launches (with and without q/k L2-norm)."""
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    B = 5
    print(f"decode multi long T={T} l2={l2}", flush=True)
    x = inp.decode_multi_inputs(B, T, HQ=4, HV=8, seed=2300 + T)
    if l2:
        gen = torch.Generator().manual_seed(2400 + T)
        x["q"] = (torch.randn(x["q"].shape, generator=gen) * 2.0).to(torch.bfloat16)
        x["k"] = (torch.randn(x["k"].shape, generator=gen) * 0.7).to(torch.bfloat16)
    g = _to(x, device)
    o_m, s_m = dec.gdn_decode_multi(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                    g["dt_bias"], g["b"], g["scale"], qk_l2norm=l2)
    st = g["state"].clone()
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, st = dec.gdn_decode(g["q"][:, sl], g["k"][:, sl], g["v"][:, sl], st, g["A_log"],
                               g["a"][:, sl], g["dt_bias"], g["b"][:, sl], g["scale"],
                               qk_l2norm=l2)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(o_m, torch.cat(outs, dim=1))
    assert torch.equal(s_m, st)
    xr = dict(x)
    if l2:
        xr["q"], xr["k"] = O.qk_l2norm(x["q"]), O.qk_l2norm(x["k"])
    o_ref, s_ref = _oracle_steps(xr)
    torch.testing.assert_close(o_m.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    rel = float((s_m.cpu().double() - s_ref).norm() / s_ref.norm())
    assert rel <= 1e-3, rel
