"""bench.py's command-line contract, checked without a GPU.

* ``--gpus N`` with N > 1 exits (status 2) with a message saying why: the
  operators are measured on one GPU only.
* The algorithmic byte and flop counts the roofline figures divide by match
  their closed forms for the benchmark shapes.
"""

import subprocess
import sys

from conftest import ROOT


def test_multi_gpu_request_exits_with_reason():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=300, cwd=str(ROOT))
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


def test_roofline_work_counts():
    sys.path.insert(0, str(ROOT))
    import bench

    # decode: state read + written once (fp32), q/k per qk-head, v/o per v-head
    # (bf16), a/b per v-head (bf16), per sequence
    B, HQ, HV, D = 256, 4, 8, 128
    expect = B * (2 * HV * D * D * 4 + 2 * HQ * D * 2 + 2 * HV * D * 2 + 2 * HV * 2)
    assert bench.decode_bytes(B, HQ, HV) == expect == 270016512
    # multi-token decode: the state once, the per-token arrays T times
    T = 4
    per_tok = B * (2 * HQ * D * 2 + 2 * HV * D * 2 + 2 * HV * 2)
    assert bench.decode_multi_bytes(B, T, HQ, HV) == B * 2 * HV * D * D * 4 + T * per_tok
    # prefill: 180 224 flops per token per v-head at chunk 64, d 128
    assert bench.prefill_flops(32768, 32) == 32768 * 32 * (10 * 64 * D + 6 * D * D)
