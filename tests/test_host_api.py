"""CPU checks of the Python entry points' validation (reference error behaviour:
AssertionError before any launch, DEC:117-120 and PRE:1635-1667)."""

import math

import pytest
import torch

from conftest import pkg_module


def test_decode_run_rejects_wrong_shapes_and_cpu_tensors():
    dec = pkg_module("decode")
    inp = pkg_module("inputs")
    x = inp.decode_inputs(2)
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
    with pytest.raises(AssertionError):            # CPU tensors
        dec.run(*args, x["scale"])
    bad = list(args)
    bad[0] = torch.zeros(2, 1, 3, 128, dtype=torch.bfloat16)   # HQ != 4
    with pytest.raises(AssertionError):
        dec.run(*bad, None)
    bad = list(args)
    bad[2] = torch.zeros(3, 1, 8, 128, dtype=torch.bfloat16)   # batch mismatch
    with pytest.raises(AssertionError):
        dec.run(*bad, None)


def test_prefill_run_rejects_like_reference():
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    x = inp.prefill_inputs([10, 5])
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    with pytest.raises(AssertionError):            # not cuda (PRE:1646-1647)
        pre.run(*args, None)


def test_scale_resolution():
    dec = pkg_module("decode")
    pre = pkg_module("prefill")
    assert dec._resolve_scale(None, 128) == 1.0 / math.sqrt(128)
    assert dec._resolve_scale(0.0, 128) == 1.0 / math.sqrt(128)
    assert dec._resolve_scale(0.5, 128) == 0.5
    assert pre._resolve_scale(None) == 1.0 / math.sqrt(128)
    assert pre._resolve_scale(0.0) == 1.0 / math.sqrt(128)


def test_inputs_are_seeded_and_normalised():
    inp = pkg_module("inputs")
    a = inp.decode_inputs(3, seed=7)
    b = inp.decode_inputs(3, seed=7)
    for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b"):
        assert torch.equal(a[k], b[k])
    n = a["q"].float().norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=1e-2)
    lens = inp.workload_lengths("prefill_varlen8_t32768_qk16_v32")
    assert len(lens) == 8 and sum(lens) == 32768 and min(lens) > 0
    lens3 = inp.workload_lengths("prefill_varlen16_qk4_v8")
    assert len(lens3) == 16 and all(128 <= L <= 8192 for L in lens3)
