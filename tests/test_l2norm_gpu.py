"""GPU checks of the ``qk_l2norm`` option (q and k L2-normalised inside the
kernels, an extension: the reference takes q and k already normalised).

The kernels get raw bf16 q/k of mixed magnitudes (rows far below, near and far
above unit norm, and all-zero rows); the oracle normalises the same bf16
values in fp64 with ``x (sum x^2 + 1e-6)^-1/2`` and then runs the unchanged
decode / prefill definition.  Bars are the operators' own: outputs within
atol = rtol = 1e-2, final state within 1e-3 relative (Frobenius) error.
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

STATE_REL_BAR = 1e-3
PRE_NAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _raw_qk(shape, seed, zero_rows=()):
    """bf16 rows ~ N(0, m^2) with per-row magnitude m in {0.003, 0.05, 1, 9}.

    At m = 0.003 the row's squared norm (about 1.2e-3) is within three
    decades of eps, so the eps term shows in the result.
    """
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g)
    mags = torch.tensor([0.003, 0.05, 1.0, 9.0])
    idx = torch.randint(0, 4, shape[:-1], generator=g)
    x = x * mags[idx][..., None]
    for r in zero_rows:
        x[r] = 0.0
    return x.to(torch.bfloat16)


def _normalised(x):
    return dict(x, q=O.qk_l2norm(x["q"]), k=O.qk_l2norm(x["k"]))


def _check(o, s, o_ref, s_ref):
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    s = s.cpu().double()
    rel = float((s - s_ref).norm() / s_ref.norm().clamp_min(1e-300))
    assert rel <= STATE_REL_BAR, rel
    return rel


def _decode_oracle_steps(x):
    B, T = x["q"].shape[:2]
    S = x["state"]
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, S = O.decode_step(x["q"][:, sl], x["k"][:, sl], x["v"][:, sl], S, x["A_log"],
                             x["a"][:, sl], x["dt_bias"], x["b"][:, sl], x["scale"])
        outs.append(o)
    return torch.cat(outs, dim=1), S


@pytest.mark.parametrize("B,HQ,HV", [(7, 4, 8), (256, 4, 8), (5, 16, 32)])
def test_decode_l2norm_matches_oracle(device, B, HQ, HV):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    print(f"decode l2norm B={B} HQ={HQ} HV={HV}", flush=True)
    x = inp.decode_inputs(B, HQ=HQ, HV=HV, seed=3000 + B)
    x["q"] = _raw_qk((B, 1, HQ, 128), 3100 + B, zero_rows=[(0, 0, 0)])
    x["k"] = _raw_qk((B, 1, HQ, 128), 3200 + B, zero_rows=[(B - 1, 0, HQ - 1)])
    g = _to(x, device)
    o, s = dec.gdn_decode(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"], g["dt_bias"],
                          g["b"], g["scale"], qk_l2norm=True)
    torch.cuda.synchronize()
    _check(o, s, *_decode_oracle_steps(_normalised(x)))
    # the option is not a no-op on raw inputs: without it the result differs
    o0, _ = dec.gdn_decode(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"], g["dt_bias"],
                           g["b"], g["scale"])
    torch.cuda.synchronize()
    assert not torch.equal(o0, o)


def test_decode_l2norm_on_unit_inputs_matches_plain(device):
    """Unit rows rounded to bf16 have norms 1 +- ~5e-4, so the option changes
    the state by a few 1e-4 relative; that change itself must match the
    oracle's (a check of the normalisation well below the parity bar)."""
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.decode_inputs(9, seed=3300)
    g = _to(x, device)
    args = [g[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")] + [g["scale"]]
    o1, s1 = dec.gdn_decode(*args, qk_l2norm=True)
    o0, s0 = dec.gdn_decode(*args)
    torch.cuda.synchronize()
    torch.testing.assert_close(o1.float(), o0.float(), atol=1e-2, rtol=1e-2)
    _, r0 = _decode_oracle_steps(x)
    _, r1 = _decode_oracle_steps(_normalised(x))
    d_ref = r1 - r0
    d = (s1 - s0).cpu().double()
    assert float(d_ref.norm() / r0.norm()) > 1e-5          # the change is real
    rel = float((d - d_ref).norm() / d_ref.norm())
    assert rel <= 2e-2, rel


@pytest.mark.parametrize("B,T,HQ,HV", [(3, 4, 4, 8), (2, 7, 16, 32)])
def test_decode_multi_l2norm(device, B, T, HQ, HV):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    print(f"decode multi l2norm B={B} T={T} HQ={HQ} HV={HV}", flush=True)
    x = inp.decode_multi_inputs(B, T, HQ=HQ, HV=HV, seed=3400 + B + T)
    x["q"] = _raw_qk((B, T, HQ, 128), 3500 + T, zero_rows=[(0, 1, 0)])
    x["k"] = _raw_qk((B, T, HQ, 128), 3600 + T, zero_rows=[(B - 1, T - 2, 0)])
    g = _to(x, device)
    o, s = dec.gdn_decode_multi(g["q"], g["k"], g["v"], g["state"], g["A_log"], g["a"],
                                g["dt_bias"], g["b"], g["scale"], qk_l2norm=True)
    torch.cuda.synchronize()
    _check(o, s, *_decode_oracle_steps(_normalised(x)))
    # the same normalisation as T successive single-step launches: bit-identical
    st = g["state"].clone()
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o1, st = dec.gdn_decode(g["q"][:, sl], g["k"][:, sl], g["v"][:, sl], st, g["A_log"],
                                g["a"][:, sl], g["dt_bias"], g["b"][:, sl], g["scale"],
                                qk_l2norm=True)
        outs.append(o1)
    torch.cuda.synchronize()
    assert torch.equal(o, torch.cat(outs, dim=1))
    assert torch.equal(s, st)


@pytest.mark.parametrize("lens,HQ,HV,with_state", [
    ([100, 37], 4, 8, True), ([1, 63, 64, 65, 129], 4, 8, True), ([0, 300], 4, 8, False),
    ([130, 70], 16, 32, True), ([1000, 777], 4, 8, True)])
@pytest.mark.parametrize("path", ["auto", "fused"])
def test_prefill_l2norm_matches_oracle(device, lens, HQ, HV, with_state, path):
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    print(f"prefill l2norm lens={lens} HQ={HQ} HV={HV}", flush=True)
    x = inp.prefill_inputs(lens, HQ=HQ, HV=HV, seed=3700 + sum(lens), with_state=with_state)
    T = sum(lens)
    x["q"] = _raw_qk((T, HQ, 128), 3800 + T, zero_rows=[(T - 1, 0)])
    x["k"] = _raw_qk((T, HQ, 128), 3900 + T, zero_rows=[(T // 2, HQ - 1)])
    g = _to(x, device)
    o, s = pre.gdn_prefill(*[g[n] for n in PRE_NAMES], g["scale"], qk_l2norm=True, path=path)
    torch.cuda.synchronize()
    xn = _normalised(x)
    o_ref, s_ref = O.prefill_chunked(*[xn[n] for n in PRE_NAMES], x["scale"])
    _check(o, s, o_ref, s_ref)
    for n in range(len(lens)):
        nr = float(s_ref[n].norm())
        if nr > 0:
            assert float((s[n].cpu().double() - s_ref[n]).norm()) / nr <= STATE_REL_BAR, n


def test_prefill_l2norm_single_token_equals_decode(device):
    """A length-1 sequence in prefill is one decode step (softplus forms agree
    to rounding away from the threshold); both normalise q/k the same way."""
    pre = pkg_module("prefill")
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([1, 1, 1], seed=4000, with_state=True)
    x["q"] = _raw_qk((3, 4, 128), 4001)
    x["k"] = _raw_qk((3, 4, 128), 4002)
    g = _to(x, device)
    o_p, s_p = pre.gdn_prefill(*[g[n] for n in PRE_NAMES], g["scale"], qk_l2norm=True)
    o_d, s_d = dec.gdn_decode(g["q"][:, None], g["k"][:, None], g["v"][:, None], g["state"],
                              g["A_log"], g["a"][:, None], g["dt_bias"], g["b"][:, None],
                              g["scale"], qk_l2norm=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(o_p.float(), o_d[:, 0].float(), atol=1e-2, rtol=1e-2)
    rel = float((s_p - s_d).double().norm() / s_d.double().norm())
    assert rel <= STATE_REL_BAR, rel
