"""Runs the reference-side ctypes binding of the repository's integration
guide (the block between its binding markers), as written, through the plain C entry points gdn_decode_fwd and gdn_prefill_fwd:
with q a strided view of a fused qkv projection and A_log in bf16, the two
cases in which the binding converts or copies an argument.  Bars: outputs
within atol = rtol = 1e-2 and final states within 1e-3 relative error of the
fp64 oracle."""

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


@pytest.mark.parametrize("lens", [[4096], [300, 0, 77]])
def test_binding_prefill(device, lens):
    ns = _binding()
    inp = pkg_module("inputs")
    x = inp.prefill_inputs(lens, seed=602, with_state=True)
    g = _to(x, device)
    qk = torch.cat([g["q"], g["k"]], dim=-1)                              # [T, 4, 256]
    q = qk[..., :128]
    assert not q.is_contiguous()
    o, s = ns["prefill_run"](q, g["k"], g["v"], g["state"], g["A_log"].to(torch.bfloat16), g["a"],
                             g["dt_bias"], g["b"], g["cu_seqlens"], None)
    torch.cuda.synchronize()
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    xr = dict(x, A_log=x["A_log"].to(torch.bfloat16).float())
    o_ref, s_ref = O.prefill_chunked(*[xr[n] for n in names], x["scale"])
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3
