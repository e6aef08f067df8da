"""GPU checks of the reference-compatible entry points' contract on device
tensors: the AssertionError cases of the reference's validation (decode
DEC:117-120, prefill ``_validate_inputs`` PRE:1635-1667) raised before any
launch, the accepted cu_seqlens dtypes, and inputs of large magnitude.

Bars for results: output (bf16) within atol = rtol = 1e-2 (relative to the
output scale below where values are large); final state relative error
<= 1e-3 against the fp64 oracle.
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

PNAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
DNAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def _prefill_case(device, lens=(70, 30), cu_dtype=torch.int64):
    inp = pkg_module("inputs")
    x = inp.prefill_inputs(list(lens), seed=501, with_state=True, cu_dtype=cu_dtype)
    return x, _to(x, device)


def test_prefill_run_rejects_bad_totals_dtypes_and_shapes(device):
    pre = pkg_module("prefill")
    x, g = _prefill_case(device)
    args = [g[n] for n in PNAMES]

    def bad(i, t):
        a = list(args)
        a[i] = t
        return a

    T = g["q"].shape[0]
    cases = {
        "cu_seqlens[-1] != T": bad(8, torch.tensor([0, 70, 99], device=device)),
        "q fp16": bad(0, g["q"].half()),
        "v fp32": bad(2, g["v"].float()),
        "A_log bf16": bad(4, g["A_log"].to(torch.bfloat16)),
        "a fp32": bad(5, g["a"].float()),
        "cu_seqlens fp32": bad(8, g["cu_seqlens"].float()),
        "state shape": bad(3, g["state"][:1]),
        "state bf16": bad(3, g["state"].to(torch.bfloat16)),
        "k heads": bad(1, torch.zeros(T, 3, 128, dtype=torch.bfloat16, device=device)),
        "b length": bad(7, g["b"][:-1]),
        "cpu cu_seqlens": bad(8, x["cu_seqlens"]),
    }
    for name, a in cases.items():
        with pytest.raises(AssertionError):
            pre.run(*a, None)
        out = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=device)
        fs = torch.empty(2, 8, 128, 128, dtype=torch.float32, device=device)
        with pytest.raises(AssertionError):
            pre.run_dps(*a, None, out, fs)
        print("rejected:", name, flush=True)


def test_prefill_run_rereads_rewritten_cu_seqlens(device):
    """run reads cu_seqlens back once per tensor object and version: a repeated
    call on the same tensor reuses the host copy, an in-place rewrite through
    torch is read again (and fails the reference's cu_seqlens[-1] == T check
    when it should), and a new tensor at a reused address is read again."""
    pre = pkg_module("prefill")
    x, g = _prefill_case(device, lens=(70, 30))
    args = [g[n] for n in PNAMES]
    cu = g["cu_seqlens"]
    o1, s1 = pre.run(*args, x["scale"])
    o2, s2 = pre.run(*args, x["scale"])
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)
    cu.copy_(torch.tensor([0, 70, 99], dtype=cu.dtype, device=device))      # in place: T mismatch
    with pytest.raises(AssertionError):
        pre.run(*args, x["scale"])
    cu.copy_(torch.tensor([0, 60, 100], dtype=cu.dtype, device=device))     # new split, T again
    o3, s3 = pre.run(*args, x["scale"])
    del args, cu
    g["cu_seqlens"] = None
    fresh = torch.tensor([0, 100], dtype=torch.int64, device=device)        # may reuse the address
    one_state = g["state"][:1].contiguous()
    o4, s4 = pre.run(g["q"], g["k"], g["v"], one_state, g["A_log"], g["a"], g["dt_bias"], g["b"],
                     fresh, x["scale"])
    torch.cuda.synchronize()
    x60 = dict(x, cu_seqlens=torch.tensor([0, 60, 100], dtype=torch.int64))
    o_ref, s_ref = O.prefill_chunked(*[x60[n] for n in PNAMES], x["scale"])
    torch.testing.assert_close(o3.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    x1 = dict(x, cu_seqlens=torch.tensor([0, 100], dtype=torch.int64), state=x["state"][:1])
    o_ref, s_ref = O.prefill_chunked(*[x1[n] for n in PNAMES], x["scale"])
    torch.testing.assert_close(o4.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s4.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


@pytest.mark.parametrize("cu_dtype", [torch.int64, torch.int32])
def test_prefill_run_accepts_int64_and_int32(device, cu_dtype):
    pre = pkg_module("prefill")
    x, g = _prefill_case(device, cu_dtype=cu_dtype)
    o, s = pre.run(*[g[n] for n in PNAMES], None)
    torch.cuda.synchronize()
    x64 = dict(x, cu_seqlens=x["cu_seqlens"].long())
    o_ref, s_ref = O.prefill_recurrent(*[x64[n] for n in PNAMES], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_decode_run_rejects_on_device(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    g = _to(inp.decode_inputs(3, seed=502), device)
    args = [g[n] for n in DNAMES]
    for i, t in [(0, torch.zeros(3, 2, 4, 128, dtype=torch.bfloat16, device=device)),   # T != 1
                 (1, torch.zeros(3, 1, 2, 128, dtype=torch.bfloat16, device=device)),   # k heads
                 (2, torch.zeros(2, 1, 8, 128, dtype=torch.bfloat16, device=device)),   # batch
                 (3, g["state"][:, :4])]:                                                # state heads
        a = list(args)
        a[i] = t
        with pytest.raises(AssertionError):
            dec.run(*a, None)


def test_decode_run_other_float_dtypes(device):
    """fp32 / fp16 activations (the reference kernel loads any float dtype):
    rounded to bf16 on entry; the output takes q's dtype (DEC:122)."""
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.decode_inputs(4, seed=503)
    g = _to(x, device)
    o_bf, s_bf = dec.run(*[g[n] for n in DNAMES], None)
    for dt in (torch.float32, torch.float16):
        gd = dict(g)
        for n in ("q", "k", "v", "a", "b"):
            gd[n] = g[n].to(dt)
        o, s = dec.run(*[gd[n] for n in DNAMES], None)
        torch.cuda.synchronize()
        assert o.dtype == dt
        assert torch.equal(s, s_bf)
        # the bf16 result, converted to the output dtype (fp16 rounds small values)
        torch.testing.assert_close(o.float(), o_bf.float(), rtol=2.0 ** -10, atol=6e-8)


@pytest.mark.parametrize("path", ["auto", "fused"])
def test_prefill_large_magnitude_inputs(device, path):
    """v ~ N(0, 300^2) and an initial state ~ N(0, 30^2): finite, and on the
    oracle bars relative to the output scale.  (The fp16 operands of the
    state path need |values| < 65504; this stays an order of magnitude
    inside.)"""
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([200, 77], seed=504, with_state=True)
    gen = torch.Generator().manual_seed(505)
    x["v"] = (torch.randn(x["v"].shape, generator=gen) * 300.0).to(torch.bfloat16)
    x["state"] = torch.randn(x["state"].shape, generator=gen) * 30.0
    g = _to(x, device)
    o, s = pre.gdn_prefill(*[g[n] for n in PNAMES], g["scale"], path=path)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o.float()).all()) and bool(torch.isfinite(s).all())
    o_ref, s_ref = O.prefill_recurrent(*[x[n] for n in PNAMES], x["scale"])
    o_scale = float(o_ref.abs().max())
    torch.testing.assert_close(o.float().cpu().double() / o_scale, o_ref / o_scale,
                               atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


@pytest.mark.parametrize("path", ["fused", "split"])
def test_prefill_range_overflow_is_reported(device, path):
    """v of the second sequence ~ N(0, 1e5^2) puts X past the fp16 operand
    range: with check_range=True the call raises RangeOverflowError naming
    that sequence only; the in-range sequence keeps its oracle result, and
    the in-range inputs of the test above pass the check."""
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([200, 77], seed=508, with_state=True)
    gen = torch.Generator().manual_seed(509)
    x["v"][200:] = (torch.randn(x["v"][200:].shape, generator=gen) * 1e5).to(torch.bfloat16)
    g = _to(x, device)
    with pytest.raises(pre.RangeOverflowError, match=r"\[1\]"):
        pre.gdn_prefill(*[g[n] for n in PNAMES], g["scale"], path=path, check_range=True)
    o, s = pre.gdn_prefill(*[g[n] for n in PNAMES], g["scale"], path=path)
    torch.cuda.synchronize()
    assert not bool(torch.isfinite(s[1]).all())
    x0 = {n: (x[n][:200] if n in ("q", "k", "v", "a", "b") else x[n]) for n in PNAMES}
    x0["state"] = x["state"][:1]
    x0["cu_seqlens"] = torch.tensor([0, 200], dtype=torch.int64)
    o_ref, s_ref = O.prefill_recurrent(*[x0[n] for n in PNAMES], x["scale"])
    torch.testing.assert_close(o[:200].float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s[:1].cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3
    # in range: the check passes
    y = inp.prefill_inputs([200, 77], seed=504, with_state=True)
    gy = _to(y, device)
    pre.gdn_prefill(*[gy[n] for n in PNAMES], gy["scale"], path=path, check_range=True)


def test_decode_large_magnitude_inputs(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.decode_inputs(8, seed=506)
    gen = torch.Generator().manual_seed(507)
    x["v"] = (torch.randn(x["v"].shape, generator=gen) * 300.0).to(torch.bfloat16)
    x["state"] = torch.randn(x["state"].shape, generator=gen) * 3000.0
    g = _to(x, device)
    o, s = dec.run(*[g[n] for n in DNAMES], x["scale"])
    torch.cuda.synchronize()
    o_ref, s_ref = O.decode_step(*[x[n] for n in DNAMES], x["scale"])
    o_scale = float(o_ref.abs().max())
    torch.testing.assert_close(o.float().cpu().double() / o_scale, o_ref / o_scale,
                               atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3
