"""Runs the reference-side ctypes binding of the repository's integration
guide (the block between its binding markers), as written: decode through
gdn_decode_fwd with q a strided view of a fused qkv projection and A_log in
bf16 (the cases in which the binding converts or copies an argument);
prefill with the reference's validation and the length-based path choice
(gdn_prefill_choose_slices, then gdn_prefill_split_fwd or gdn_prefill_fwd).
Bars: outputs within atol = rtol = 1e-2 and final states within 1e-3
relative error of the fp64 oracle; the fused-path case equal bit for bit to
the package's fused call."""

import re

import pytest
import torch

from conftest import ROOT, pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu


def _binding():
    text = (ROOT / "INTEGRATION.md").read_text()
    code = re.search(r"<!-- binding:begin -->\s*```python\n(.*?)```\s*<!-- binding:end -->", text,
                     re.S).group(1)
    ns = {"LIB_PATH": str(pkg_module("_capi").LIB_PATH)}
    exec(compile(code, "integration_binding", "exec"), ns)
    return ns


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def test_binding_decode(device):
    ns = _binding()
    inp = pkg_module("inputs")
    x = inp.decode_inputs(5, seed=601)
    g = _to(x, device)
    qkv = torch.cat([g["q"], g["k"], torch.zeros_like(g["q"])], dim=-1)   # [B, 1, 4, 384]
    q = qkv[..., :128]
    assert not q.is_contiguous()
    o, s = ns["decode_run"](q, g["k"], g["v"], g["state"], g["A_log"].to(torch.bfloat16), g["a"],
                            g["dt_bias"], g["b"], None)
    torch.cuda.synchronize()
    xr = dict(x, A_log=x["A_log"].to(torch.bfloat16).float())
    o_ref, s_ref = O.decode_step(*[xr[n] for n in ("q", "k", "v", "state", "A_log", "a",
                                                   "dt_bias", "b")], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


@pytest.mark.parametrize("lens,path", [([4096], 8), ([300, 0, 77], 8)])
def test_binding_prefill(device, lens, path):
    """qk4/v8 through the binding, q a strided view: the lengths choose the
    split path (8 state slices per chain)."""
    ns = _binding()
    inp = pkg_module("inputs")
    x = inp.prefill_inputs(lens, seed=602, with_state=True)
    g = _to(x, device)
    assert ns["prefill_plan"](x["cu_seqlens"], sum(lens), 4, 8)[2] == path
    qk = torch.cat([g["q"], g["k"]], dim=-1)                              # [T, 4, 256]
    q = qk[..., :128]
    assert not q.is_contiguous()
    o, s = ns["prefill_run"](q, g["k"], g["v"], g["state"], g["A_log"], g["a"],
                             g["dt_bias"], g["b"], g["cu_seqlens"], None)
    torch.cuda.synchronize()
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    o_ref, s_ref = O.prefill_chunked(*[x[n] for n in names], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_binding_prefill_four_equal_sequences_fused(device):
    """Four 5 348-token sequences at qk16/v32 (128 chains): the lengths choose
    the fused kernel, without seams (cutting two of four equal chains leaves
    two as long), and the binding's results equal the package's automatic
    path bit for bit and the fp64 oracle within the prefill bars."""
    ns = _binding()
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    lens = [5348] * 4
    print("binding prefill 4 x 5348 qk16/v32", flush=True)
    x = inp.prefill_inputs(lens, 16, 32, seed=603, with_state=True)
    g = _to(x, device)
    _, ws, slices, seams = ns["prefill_plan"](x["cu_seqlens"], sum(lens), 16, 32)
    assert (slices, seams, ws) == (0, 0, 0)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    o, s = ns["prefill_run"](*[g[n] for n in names], None)
    of, sf = pre.gdn_prefill(*[g[n] for n in names], None)
    torch.cuda.synchronize()
    assert torch.equal(o, of) and torch.equal(s, sf)
    o_ref, s_ref = O.prefill_chunked(*[x[n] for n in names], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_binding_prefill_fused_with_seams(device):
    """The 16-sequence qk4/v8 batch (128 chains, lengths 244-7 532, int32
    cu_seqlens): the plan runs the fused kernel with seams on the 128 idle
    CUs; the binding equals the package's automatic path bit for bit and
    the fp64 oracle within the prefill bars."""
    ns = _binding()
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    lens = inp.workload_lengths("prefill_varlen16_qk4_v8")
    print("binding prefill varlen16 qk4/v8", flush=True)
    x = inp.prefill_inputs(lens, 4, 8, seed=604, with_state=True, cu_dtype=torch.int32)
    g = _to(x, device)
    _, ws, slices, seams = ns["prefill_plan"](x["cu_seqlens"], sum(lens), 4, 8)
    assert slices == 0 and seams > 0 and ws > 0
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    o, s = ns["prefill_run"](*[g[n] for n in names], None)
    of, sf = pre.gdn_prefill(*[g[n] for n in names], None)
    torch.cuda.synchronize()
    assert torch.equal(o, of) and torch.equal(s, sf)
    x64 = dict(x, cu_seqlens=x["cu_seqlens"].long())
    o_ref, s_ref = O.prefill_chunked(*[x64[n] for n in names], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_binding_prefill_rejects_like_the_reference(device):
    """AssertionError before any launch, as PRE:1635-1667: cu_seqlens[-1] != T,
    and A_log not fp32."""
    ns = _binding()
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([100, 28], seed=604, with_state=True)
    g = _to(x, device)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    bad = dict(g, cu_seqlens=torch.tensor([0, 100, 127], dtype=torch.int64, device=device))
    with pytest.raises(AssertionError):
        ns["prefill_run"](*[bad[n] for n in names], None)
    bad = dict(g, A_log=g["A_log"].to(torch.bfloat16))
    with pytest.raises(AssertionError):
        ns["prefill_run"](*[bad[n] for n in names], None)
