"""GPU check of the allocation-free split prefill entry point
(gdn_prefill_split_noalloc_fwd): called through the C ABI twice in a row --
the second call on a smaller batch, so the static workspace holds the first
call's data when the second starts -- and compared with
gdn_prefill_split_fwd on a caller workspace: outputs and final states equal
bit for bit (the same kernels on the same inputs), and within the prefill
bars of the fp64 oracle.  Oversized problems are rejected before any launch.
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")


def _call(lib, capi, g, T, N, slices, ws=None):
    p = capi.ptr
    out = torch.empty(T, 8, 128, dtype=torch.bfloat16, device=g["q"].device)
    fs = torch.empty(N, 8, 128, 128, dtype=torch.float32, device=g["q"].device)
    args = [p(g["q"]), p(g["k"]), p(g["v"]), p(g["state"]), p(g["A_log"]), p(g["a"]),
            p(g["dt_bias"]), p(g["b"]), p(g["cu_seqlens"]), 0, N, T, 4, 8, float(g["scale"]),
            p(out), p(fs), slices]
    st = capi.stream_handle(g["q"].device)
    if ws is None:
        rc = lib.gdn_prefill_split_noalloc_fwd(*args, 0, st)
    else:
        rc = lib.gdn_prefill_split_fwd(*args, p(ws), ws.numel(), 0, st)
    return rc, out, fs


def test_noalloc_matches_workspace_entry_twice(device):
    capi = pkg_module("_capi")
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    lib = capi.lib()
    cap = lib.gdn_prefill_split_noalloc_max_bytes()
    assert cap == 32 << 20
    for lens, slices in (([4096], 8), ([700, 0, 93], 4)):
        print(f"noalloc lens={lens} slices={slices}", flush=True)
        T, N = sum(lens), len(lens)
        x = inp.prefill_inputs(lens, seed=7000 + T, with_state=True)
        g = {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in x.items()}
        need = pre.split_workspace_bytes(N, T, 4, 8)
        assert 0 < need <= cap
        rc, o_na, s_na = _call(lib, capi, g, T, N, slices)
        assert rc == capi.GDN_OK, rc
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        rc, o_ws, s_ws = _call(lib, capi, g, T, N, slices, ws)
        assert rc == capi.GDN_OK, rc
        torch.cuda.synchronize()
        assert torch.equal(o_na, o_ws) and torch.equal(s_na, s_ws)
        o_ref, s_ref = O.prefill_chunked(*[x[n] for n in NAMES], x["scale"])
        torch.testing.assert_close(o_na.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
        assert float((s_na.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_noalloc_rejects_oversized_problem(device):
    """A problem whose workspace exceeds the static array is rejected before
    any launch.  The buffers are real device tensors of the problem's sizes,
    so the call reads nothing out of bounds even if it went further."""
    capi = pkg_module("_capi")
    pre = pkg_module("prefill")
    lib = capi.lib()
    T, N = 32768, 8
    assert pre.split_workspace_bytes(N, T, 4, 8) > lib.gdn_prefill_split_noalloc_max_bytes()
    z = lambda *shape, dt=torch.bfloat16: torch.zeros(*shape, dtype=dt, device=device)
    q, k, v, out = z(T, 4, 128), z(T, 4, 128), z(T, 8, 128), z(T, 8, 128)
    a, b = z(T, 8), z(T, 8)
    A_log, dt_bias = z(8, dt=torch.float32), z(8, dt=torch.float32)
    state, fs = z(N, 8, 128, 128, dt=torch.float32), z(N, 8, 128, 128, dt=torch.float32)
    cu = torch.arange(0, T + 1, T // N, dtype=torch.int64, device=device)
    p = capi.ptr
    rc = lib.gdn_prefill_split_noalloc_fwd(p(q), p(k), p(v), p(state), p(A_log), p(a), p(dt_bias),
                                           p(b), p(cu), 0, N, T, 4, 8, 1.0, p(out), p(fs), 8, 0,
                                           capi.stream_handle(device))
    assert rc == capi.GDN_ERR_WORKSPACE
    torch.cuda.synchronize()
