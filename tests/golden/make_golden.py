"""Writes the golden fixtures of this directory from the CPU oracle (float64).

The reference ships no golden vectors for GDN decode / prefill, so the
fixtures are the oracle's own outputs on small seeded inputs, frozen so that
a later change to the oracle or to the input generator is caught.  Each
fixture holds its inputs and expected outputs (safetensors, no pickle):

* decode_b1_qk4_v8.safetensors       -- one decode step, batch 1 (the CPU case)
* decode_b2_qk2_v8.safetensors       -- one decode step, batch 2, 2 qk / 8 v heads
  (4 v-heads per qk-head)
* prefill_varlen3_qk4_v8.safetensors -- varlen prefill, lengths 130, 64, 1,
  with initial states (ragged tails, an exact chunk, a single token)

Expected outputs are the float64 oracle results stored as float32.

Run:  python tests/golden/make_golden.py
"""

import importlib.util
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import gdn_oracle as O  # noqa: E402


def _inputs_module():
    spec = importlib.util.spec_from_file_location("gdn_inputs", ROOT / "track-c-gdn_amd" / "inputs.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def decode_fixture(B, HQ, HV, seed):
    inp = _inputs_module()
    x = inp.decode_inputs(B, HQ, HV, seed=seed)
    o, s = O.decode_step(x["q"], x["k"], x["v"], x["state"], x["A_log"], x["a"], x["dt_bias"],
                         x["b"], x["scale"])
    t = {k: v for k, v in x.items() if torch.is_tensor(v)}
    t["scale"] = torch.tensor([x["scale"]], dtype=torch.float64)
    t["expected_output"] = o.float()
    t["expected_new_state"] = s.float()
    return t


def prefill_fixture(lens, HQ, HV, seed):
    inp = _inputs_module()
    x = inp.prefill_inputs(lens, HQ, HV, seed=seed, with_state=True)
    names = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")
    o, s = O.prefill_recurrent(*[x[n] for n in names], x["scale"])
    t = {n: x[n] for n in names}
    t["scale"] = torch.tensor([x["scale"]], dtype=torch.float64)
    t["expected_output"] = o.float()
    t["expected_final_state"] = s.float()
    return t


FIXTURES = {
    "decode_b1_qk4_v8": lambda: decode_fixture(1, 4, 8, 1000),
    "decode_b2_qk2_v8": lambda: decode_fixture(2, 2, 8, 1010),
    "prefill_varlen3_qk4_v8": lambda: prefill_fixture([130, 64, 1], 4, 8, 1020),
}


def main():
    for name, make in FIXTURES.items():
        t = {k: v.contiguous() for k, v in make().items()}
        save_file(t, str(HERE / f"{name}.safetensors"))
        print(name, sum(v.numel() * v.element_size() for v in t.values()), "bytes")


if __name__ == "__main__":
    main()
