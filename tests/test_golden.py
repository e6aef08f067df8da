"""The committed golden fixtures (tests/golden/*.safetensors) against the oracle
(CPU) and against the HIP kernels (GPU)."""

from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from conftest import pkg_module
from oracle import gdn_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
DECODE = ["decode_b1_qk4_v8", "decode_b2_qk2_v8"]
PREFILL = ["prefill_varlen3_qk4_v8"]
PNAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")


def _load(name):
    return load_file(str(GOLDEN / f"{name}.safetensors"))


@pytest.mark.parametrize("name", DECODE)
def test_oracle_reproduces_decode_fixture(name):
    t = _load(name)
    o, s = O.decode_step(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"],
                         t["b"], float(t["scale"][0]))
    torch.testing.assert_close(o.float(), t["expected_output"], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(s.float(), t["expected_new_state"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", PREFILL)
def test_oracle_reproduces_prefill_fixture(name):
    t = _load(name)
    args = [t[n] for n in PNAMES]
    o, s = O.prefill_recurrent(*args, float(t["scale"][0]))
    torch.testing.assert_close(o.float(), t["expected_output"], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(s.float(), t["expected_final_state"], rtol=1e-6, atol=1e-7)
    oc, sc = O.prefill_chunked(*args, float(t["scale"][0]))
    torch.testing.assert_close(oc.float(), t["expected_output"], rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(sc.float(), t["expected_final_state"], rtol=1e-6, atol=1e-7)


def test_fixture_inputs_match_generator():
    inp = pkg_module("inputs")
    t = _load("decode_b1_qk4_v8")
    x = inp.decode_inputs(1, 4, 8, seed=1000)
    for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b"):
        assert torch.equal(t[k], x[k]), k


@pytest.mark.gpu
@pytest.mark.parametrize("name", DECODE)
def test_decode_kernel_on_fixture(device, name):
    dec = pkg_module("decode")
    t = {k: v.to(device) for k, v in _load(name).items()}
    o, s = dec.gdn_decode(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"],
                          t["b"], float(t["scale"][0]))
    torch.cuda.synchronize()
    torch.testing.assert_close(o.float(), t["expected_output"], atol=1e-2, rtol=1e-2)
    ref = t["expected_new_state"]
    assert float((s - ref).norm() / ref.norm()) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("name", PREFILL)
def test_prefill_kernel_on_fixture(device, name):
    pre = pkg_module("prefill")
    t = {k: v.to(device) for k, v in _load(name).items()}
    o, s = pre.run(*[t[n] for n in PNAMES], float(t["scale"][0]))
    torch.cuda.synchronize()
    torch.testing.assert_close(o.float(), t["expected_output"], atol=1e-2, rtol=1e-2)
    ref = t["expected_final_state"]
    assert float((s - ref).norm() / ref.norm()) <= 1e-3
