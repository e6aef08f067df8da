"""Empty batches on the GPU: no sequences, sequences of length 0, batch 0.

Empty tensors may carry no storage (a NULL data pointer); the entry points
accept that wherever nothing is read or written.  A batch of empty prefill
sequences still returns its initial states as final states, bit for bit
(the reference's state passthrough for a sequence with no tokens,
gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py:1049, 1121).
"""

import pytest
import torch

from conftest import pkg_module

pytestmark = pytest.mark.gpu

PRE = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
DEC = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")


def _to(x, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in x.items()}


def test_decode_batch_zero(device):
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = _to(inp.decode_inputs(2, seed=4300), device)
    e = {n: (x[n][:0] if n not in ("A_log", "dt_bias") else x[n]) for n in DEC}
    o, s = dec.run(*[e[n] for n in DEC], x["scale"])
    o2, s2 = dec.gdn_decode(*[e[n] for n in DEC], x["scale"], qk_l2norm=True)
    q4 = torch.empty(0, 3, 4, 128, dtype=torch.bfloat16, device=device)
    v4 = torch.empty(0, 3, 8, 128, dtype=torch.bfloat16, device=device)
    ab = torch.empty(0, 3, 8, dtype=torch.bfloat16, device=device)
    o3, s3 = dec.gdn_decode_multi(q4, q4, v4, e["state"], x["A_log"], ab, x["dt_bias"], ab,
                                  x["scale"])
    torch.cuda.synchronize()
    assert o.shape == (0, 1, 8, 128) and s.shape == (0, 8, 128, 128)
    assert o2.shape == (0, 1, 8, 128) and o3.shape == (0, 3, 8, 128) and s3.shape == (0, 8, 128, 128)


def test_prefill_no_sequences(device):
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    x = _to(inp.prefill_inputs([], seed=4301, with_state=False), device)
    assert x["cu_seqlens"].tolist() == [0]
    o, s = pre.run(*[x[n] for n in PRE], x["scale"])
    o2, s2, h = pre.gdn_prefill_h(*[x[n] for n in PRE], x["scale"])
    torch.cuda.synchronize()
    assert o.shape == (0, 8, 128) and s.shape == (0, 8, 128, 128)
    assert h.shape == (0, 8, 128, 128)


@pytest.mark.parametrize("with_state", [True, False])
def test_prefill_all_sequences_empty(device, with_state):
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    x = _to(inp.prefill_inputs([0, 0, 0], seed=4302, with_state=with_state), device)
    o, s = pre.run(*[x[n] for n in PRE], x["scale"])
    o2, s2, h = pre.gdn_prefill_h(*[x[n] for n in PRE], x["scale"], qk_l2norm=True)
    torch.cuda.synchronize()
    assert o.shape == (0, 8, 128) and h.shape == (0, 8, 128, 128)
    expect = x["state"] if with_state else torch.zeros(3, 8, 128, 128, device=device)
    assert torch.equal(s, expect) and torch.equal(s2, expect)
