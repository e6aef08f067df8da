"""CPU checks of the C ABI: the library loads, exports every declared symbol,
and rejects bad arguments before touching the GPU."""

import ctypes
import re
from pathlib import Path

import pytest

from conftest import ROOT, pkg_module

HEADER = ROOT / "include" / "gdn_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted([
        "gdn_abi_version", "gdn_error_string", "gdn_decode_fwd", "gdn_decode_pool_fwd",
        "gdn_decode_multi_fwd", "gdn_decode_ex_fwd", "gdn_prefill_workspace_bytes",
        "gdn_prefill_fwd", "gdn_prefill_ex_fwd", "gdn_prefill_chunk_count", "gdn_prefill_h_fwd",
        "gdn_prefill_split_workspace_bytes", "gdn_prefill_split_fwd", "gdn_prefill_auto_slices",
        "gdn_prefill_split_noalloc_max_bytes", "gdn_prefill_split_noalloc_fwd",
        "gdn_qkv_conv1d_fwd", "gdn_qkv_conv1d_update", "gdn_prefill_bwd_workspace_bytes",
        "gdn_prefill_bwd", "gdn_gate_bwd", "gdn_prefill_choose_slices", "gdn_prefill_split_h_fwd",
        "gdn_prefill_plan", "gdn_prefill_plan_info", "gdn_prefill_plan_fwd"])


def test_library_exports_every_declared_symbol():
    capi = pkg_module("_capi")
    lib = capi.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert name in capi.SIGNATURES, name
    assert lib.gdn_abi_version() == 1


def test_error_strings():
    capi = pkg_module("_capi")
    lib = capi.lib()
    assert lib.gdn_error_string(0) == b"ok"
    assert b"NULL" in lib.gdn_error_string(capi.GDN_ERR_NULL)
    assert b"head" in lib.gdn_error_string(capi.GDN_ERR_SHAPE)
    assert b"workspace" in lib.gdn_error_string(capi.GDN_ERR_WORKSPACE)


def test_argument_errors_return_before_launch():
    # NULL pointers / bad head layouts are rejected on the host: no HIP call is made.
    capi = pkg_module("_capi")
    lib = capi.lib()
    P = 0x1000  # never dereferenced: the checks fail first
    assert lib.gdn_decode_fwd(None, P, P, P, P, P, P, P, P, P, 1, 4, 8, 1.0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_decode_fwd(P, P, P, P, P, P, P, P, P, P, 1, 4, 6, 1.0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_fwd(P, P, P, P, P, P, P, P, P, P, -1, 4, 8, 1.0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_fwd(P, P, P, P, P, P, P, P, P, P, 1, 0, 8, 1.0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_pool_fwd(P, P, P, P, 4, None, P, P, P, P, P, 1, 4, 8, 1.0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_decode_multi_fwd(P, P, P, P, P, P, P, P, P, None, 1, 2, 4, 8, 1.0, 0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_decode_multi_fwd(P, P, P, P, P, P, P, P, P, P, 1, 0, 4, 8, 1.0, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_multi_fwd(P, P, P, P, P, P, P, P, P, P, 1, 2, 4, 6, 1.0, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_multi_fwd(P, P, P, P, P, P, P, P, P, P, 1, 2, 4, 8, 1.0, 2, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_ex_fwd(P, P, P, P, P, P, P, P, P, P, 1, 4, 8, 1.0, 4, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_decode_ex_fwd(None, P, P, P, P, P, P, P, P, P, 1, 4, 8, 1.0, 1, None) == capi.GDN_ERR_NULL
    assert lib.gdn_prefill_ex_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, None, 0, 8, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_fwd(None, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, None, 0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_prefill_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 7, 1.0, P, P, None, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, None, 1, None, 0, 0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_prefill_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, P, -1, None, 0, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, P, 1, None, 0, 4, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 6, 1.0, P, P, P, 1, None, 0, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_chunk_count(None, 0, 1, 1) == -1
    assert lib.gdn_prefill_split_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, None, 1, 8, P, 1 << 30, 0, None) == capi.GDN_ERR_NULL
    assert lib.gdn_prefill_split_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, P, 1, 6, P, 1 << 30, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_split_h_fwd(P, P, P, P, P, P, P, P, P, 0, 1, 1, 4, 8, 1.0, P, P, P, 1, 8, None, 0, 0, None) == capi.GDN_ERR_WORKSPACE
    # the allocation-free split prefill: a workspace above its static array
    assert lib.gdn_prefill_split_workspace_bytes(8, 32768, 4, 8) > lib.gdn_prefill_split_noalloc_max_bytes()
    assert lib.gdn_prefill_split_noalloc_fwd(P, P, P, 0, P, P, P, P, P, 0, 8, 32768, 4, 8, 1.0, P, P, 8,
                                             0, None) == capi.GDN_ERR_WORKSPACE
    # conv1d: tokens with no sequence to hold them (N = 0, T > 0)
    assert lib.gdn_qkv_conv1d_fwd(P, P, None, P, 0, 0, 5, 512, 4, None, None, 3, P, None, None,
                                  0, 0, 1, None) == capi.GDN_ERR_SHAPE


@pytest.mark.parametrize("seed", range(4))
def test_chunk_count_matches_chunk_offsets(seed):
    """Host chunk counter (the h output's first dimension) against the oracle's
    chunk_offsets, int64 and int32, including the kernels' clamping of
    out-of-range and decreasing entries into [0, T]."""
    import torch
    from oracle import gdn_oracle as O

    lib = pkg_module("_capi").lib()
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, 300, (int(torch.randint(1, 12, (1,), generator=g)),), generator=g)
    lens[0] = 0 if seed == 1 else lens[0]
    cu = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens, 0)])
    T = int(cu[-1])
    for dt in (torch.int64, torch.int32):
        c = cu.to(dt).contiguous()
        n = lib.gdn_prefill_chunk_count(c.data_ptr(), int(dt == torch.int32), c.numel() - 1, T)
        assert n == int(O.chunk_offsets(cu, 64)[-1])
    bad = cu.clone()
    bad[-1] = T + 500                      # past T: clamped to T
    if bad.numel() > 2:
        bad[1] = -7                        # negative: clamped to 0
    expect = sum((int(min(max(int(bad[i + 1]), max(int(bad[i]), 0)), T)) - min(max(int(bad[i]), 0), T) + 63) // 64
                 for i in range(bad.numel() - 1))
    n = lib.gdn_prefill_chunk_count(bad.data_ptr(), 0, bad.numel() - 1, T)
    assert n == expect


def _choose(lens, HV, cus=256, dt=None):
    import torch
    lib = pkg_module("_capi").lib()
    cu = torch.tensor([0] + list(__import__("itertools").accumulate(lens)),
                      dtype=dt or torch.int64)
    return lib.gdn_prefill_choose_slices(cu.data_ptr(), int(cu.dtype == torch.int32),
                                         cu.numel() - 1, int(cu[-1]), HV, cus)


def test_choose_slices_on_measured_batches():
    """The length-aware path choice on batches whose three options were timed
    on MI355X (256 CUs): one 4096-token sequence at qk4/v8 (split 8 slices
    78 us, 4 slices 94 us, fused 199 us); 16 varlen sequences at qk4/v8
    (4 slices 279 us, 8 slices 400 us, fused ~370 us); one 5348-token
    sequence at qk16/v32 (8 slices 129 us, fused 257 us); four of them
    (fused 267 us, 4 slices 390 us); the 8-sequence 32k batch (fused)."""
    inp = pkg_module("inputs")
    assert _choose([4096], 8) == 8
    assert _choose([4096], 8, dt=__import__("torch").int32) == 8
    assert _choose(inp.workload_lengths("prefill_varlen16_qk4_v8"), 8) == 4
    assert _choose([5348], 32) == 8
    assert _choose([5348] * 4, 32) == 0
    assert _choose(inp.workload_lengths("prefill_varlen8_t32768_qk16_v32"), 32) == 0
    # past one chain per CU: always the fused kernel
    assert _choose([100] * 64, 8) == 0


def test_choose_slices_edges():
    import torch
    lib = pkg_module("_capi").lib()
    assert lib.gdn_prefill_choose_slices(None, 0, 1, 64, 8, 256) == -1
    cu = torch.zeros(1, dtype=torch.int64)
    assert lib.gdn_prefill_choose_slices(cu.data_ptr(), 0, 0, 0, 8, 256) == 0
    assert lib.gdn_prefill_choose_slices(cu.data_ptr(), 0, 0, 0, 0, 256) == -1
    # empty sequences only: no chunks; any answer is valid, none may fail
    assert _choose([0, 0, 0], 8) in (0, 4, 8)


def _plan(lens, HQ, HV, cus=256, flags=0, dt=None):
    """gdn_prefill_plan on these lengths: (rc, plan buffer, info dict)."""
    import torch
    capi = pkg_module("_capi")
    lib = capi.lib()
    cu = torch.tensor([0] + list(__import__("itertools").accumulate(lens)), dtype=dt or torch.int64)
    buf = ctypes.create_string_buffer(capi.GDN_PREFILL_PLAN_BYTES)
    ws = ctypes.c_size_t(0)
    rc = lib.gdn_prefill_plan(cu.data_ptr(), int(cu.dtype == torch.int32), len(lens), int(cu[-1]),
                              HQ, HV, cus, flags, buf, ctypes.byref(ws))
    info = [ctypes.c_int(0) for _ in range(4)]
    if rc == 0:
        assert lib.gdn_prefill_plan_info(buf, *[ctypes.byref(i) for i in info]) == 0
    keys = ("slices", "seams", "split_chunk", "periods")
    return rc, buf, dict(zip(keys, (i.value for i in info)), workspace=ws.value)


def test_plan_on_measured_batches():
    """The host plan (path and fused seams) on the benchmark batches, 256 CUs.

    Fused seams take only CUs idle at launch: 2 HV tail workgroups per seam
    beside the chains.  The 16-sequence qk4/v8 batch (128 chains, chunk
    counts up to 118): seven sequences cut at chunk 61, so the tails (from a
    zero state and the transition chains) run on the 128 idle CUs, modelled
    finish 61 chunk periods; measured on MI355X 251 us against the split
    path's 279 us.  The 32k batch at qk16/v32 fills the GPU (256 chains): no
    seams; tails there could only start where short chains end, and with
    every CU busy the clock drops (measured: 330 us with seams against 285 us
    serial).  The workspace is the seam region: 512 bytes of plan, three
    64 KiB states per seam and v-head, the tails' OX rows."""
    inp = pkg_module("inputs")
    capi = pkg_module("_capi")
    lens = inp.workload_lengths("prefill_varlen16_qk4_v8")
    rc, _, p = _plan(lens, 4, 8)
    assert rc == 0
    assert (p["slices"], p["seams"], p["split_chunk"], p["periods"]) == (0, 7, 61, 61)
    tails = sorted(lens, reverse=True)[:7]
    ox_rows = sum(n - 64 * 61 for n in tails)
    assert p["workspace"] == 512 + 7 * 8 * 3 * 65536 + ox_rows * 8 * 256
    # int32 lengths plan the same
    assert _plan(lens, 4, 8, dt=__import__("torch").int32)[2] == p
    # no seams on request: the split path the lengths favour then (4 slices)
    rc, _, p = _plan(lens, 4, 8, flags=capi.GDN_NO_SEAMS)
    assert (p["slices"], p["seams"]) == (4, 0)
    # the 32k batch: fused, no seams, the longest chain's 84 periods, no workspace
    rc, _, p = _plan(inp.workload_lengths("prefill_varlen8_t32768_qk16_v32"), 16, 32)
    assert (p["slices"], p["seams"], p["periods"], p["workspace"]) == (0, 0, 84, 0)
    # one 4096-token sequence at qk4/v8: the split path (8 slices: 64 of 256
    # CUs, room for one seam, 2 x 8 x 8 workgroups) and its workspace
    rc, _, p = _plan([4096], 4, 8)
    assert (p["slices"], p["seams"]) == (8, 1)
    assert _plan([4096], 4, 8, flags=capi.GDN_NO_SEAMS)[2]["seams"] == 0
    assert p["workspace"] == capi.lib().gdn_prefill_split_workspace_bytes(1, 4096, 4, 8)
    # ... or, asked for the fused kernel, cut a little past half (the tail
    # workgroups' start-up) on the idle CUs
    rc, _, p = _plan([4096], 4, 8, flags=capi.GDN_PLAN_FUSED)
    assert (p["slices"], p["seams"]) == (0, 1) and 32 < p["split_chunk"] < 40
    # four equal chains per CU half: cutting two leaves two as long -- no seams
    assert _plan([5348] * 4, 16, 32)[2]["seams"] == 0
    # Split seams are counted XCD by XCD (a seam's tails and transition
    # chains are two groups of G * slices workgroups on the XCDs the chains
    # leave free).  Batches timed on MI355X with every path in rotation:
    # chunk counts 113, 44 at qk4/v8 -- 8 slices with one seam 96.8 us
    # (16 chain + 16 seam workgroups on each XCD), 4 slices 107.4 us;
    rc, _, p = _plan([113 * 64, 44 * 64], 4, 8)
    assert (p["slices"], p["seams"]) == (8, 1)
    # 56, 22, 8, 4 at qk4/v8 -- at 8 slices the chains fill every XCD, at 4
    # two seams fit: 4 slices 61.9 us, 8 slices 74.6 us; without seams the
    # model takes 8 slices
    rc, _, p = _plan([56 * 64, 22 * 64, 8 * 64, 4 * 64], 4, 8)
    assert (p["slices"], p["seams"]) == (4, 2)
    assert _plan([56 * 64, 22 * 64, 8 * 64, 4 * 64], 4, 8, flags=capi.GDN_NO_SEAMS)[2]["slices"] == 8
    # six chains at qk4/v8 at 4 slices: 24 workgroups on each XCD, one seam
    # (8 more each) fits -- 4 slices 191.4 us, 8 slices 208.8 us
    rc, _, p = _plan([117 * 64, 100 * 64, 84 * 64, 82 * 64, 59 * 64, 36 * 64], 4, 8)
    assert (p["slices"], p["seams"]) == (4, 1)
    # 118, 84 at qk16/v32: the fused kernel with two seams 231.3 us, the
    # split path (no room for a seam at 4 or 8 slices) 258.6 / 341.8 us
    rc, _, p = _plan([118 * 64, 84 * 64], 16, 32)
    assert (p["slices"], p["seams"], p["split_chunk"]) == (0, 2, 61)
    # past one chain per CU, chains too short to cut, or no idle CU: no seams
    assert _plan([100] * 64, 4, 8)[2]["seams"] == 0
    assert _plan([300] * 20, 4, 8, flags=capi.GDN_PLAN_FUSED)[2]["seams"] == 0
    assert _plan([4096] * 8, 16, 32)[2]["seams"] == 0


def test_plan_argument_errors():
    capi = pkg_module("_capi")
    lib = capi.lib()
    P = 0x1000  # never dereferenced: the checks fail first
    buf = ctypes.create_string_buffer(capi.GDN_PREFILL_PLAN_BYTES)
    assert lib.gdn_prefill_plan(None, 0, 1, 64, 4, 8, 256, 0, buf, None) == capi.GDN_ERR_NULL
    rc, good, _ = _plan([700, 300], 4, 8)
    assert rc == 0
    cu = good  # any host memory: the shape checks fail first
    assert lib.gdn_prefill_plan(cu, 0, 1, 64, 4, 6, 256, 0, buf, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_plan(cu, 0, 1, 64, 4, 8, 256, 8, buf, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_plan_info(None, None, None, None, None) == capi.GDN_ERR_NULL
    assert lib.gdn_prefill_plan_info(ctypes.create_string_buffer(512), None, None, None, None) == capi.GDN_ERR_SHAPE
    # plan_fwd: a missing plan, a plan of other sizes, unknown flags, a missing seam workspace
    args = [P] * 9 + [0, 2, 1000, 4, 8, 1.0, P, P]
    assert lib.gdn_prefill_plan_fwd(*args, None, None, 0, 0, None) == capi.GDN_ERR_NULL
    args_t = [P] * 9 + [0, 2, 999, 4, 8, 1.0, P, P]
    assert lib.gdn_prefill_plan_fwd(*args_t, good, None, 0, 0, None) == capi.GDN_ERR_SHAPE
    args_h = [P] * 9 + [0, 2, 1000, 4, 16, 1.0, P, P]
    assert lib.gdn_prefill_plan_fwd(*args_h, good, None, 0, 0, None) == capi.GDN_ERR_SHAPE
    assert lib.gdn_prefill_plan_fwd(*args, good, None, 0, 8, None) == capi.GDN_ERR_SHAPE
    rc, fused, p = _plan([700, 300], 4, 8, flags=capi.GDN_PLAN_FUSED)
    assert rc == 0 and p["seams"] >= 1 and p["workspace"] > 0
    assert lib.gdn_prefill_plan_fwd(*args, fused, None, 0, 0, None) == capi.GDN_ERR_WORKSPACE
    assert lib.gdn_prefill_plan_fwd(*args, fused, P, p["workspace"] - 1, 0, None) == capi.GDN_ERR_WORKSPACE


def test_check_final_range_names_new_nonfinite_states():
    """The prefill's range check (host logic over device-reduced flags, here
    on CPU tensors): sequences whose final state holds inf or NaN are named,
    unless their initial state already did."""
    import torch
    pre = pkg_module("prefill")
    fs = torch.zeros(4, 2, 128, 128)
    pre.check_final_range(fs)                       # all finite: no error
    fs[1, 0, 3, 4] = float("inf")
    fs[3, 1, 0, 0] = float("nan")
    with pytest.raises(pre.RangeOverflowError, match=r"\[1, 3\]"):
        pre.check_final_range(fs)
    s0 = torch.zeros(4, 2, 128, 128)
    s0[3, 0, 0, 0] = float("-inf")                  # sequence 3 started non-finite
    with pytest.raises(pre.RangeOverflowError, match=r"\[1\]"):
        pre.check_final_range(fs, s0)


def test_plan_fwd_checks_the_plan_against_itself():
    """A plan whose seam entries disagree with the region it sizes (OX rows
    out of order, a sequence cut twice, a short row count) is refused before
    any launch.  Offsets are those of the library's plan layout: seam count
    at byte 28, then 8-int arrays seq, sp, bos, len, ox_row from byte 32,
    ox_rows at 192 (layout 1)."""
    import struct
    capi = pkg_module("_capi")
    lib = capi.lib()
    P = 0x1000  # never dereferenced: the checks fail first
    lens = [2500, 2300, 640, 1000]
    rc, plan, p = _plan(lens, 4, 8, flags=capi.GDN_PLAN_FUSED)
    assert rc == 0 and p["seams"] == 2
    T = sum(lens)
    args = [P] * 9 + [0, len(lens), T, 4, 8, 1.0, P, P]
    raw = bytearray(plan.raw)
    count, = struct.unpack_from("<i", raw, 28)
    assert count == 2
    seq = struct.unpack_from("<8i", raw, 32)
    ox_row = struct.unpack_from("<8i", raw, 160)
    assert sorted(seq[:2]) == [0, 1] and ox_row[0] == 0 and ox_row[1] > 0

    def call(buf):
        b = ctypes.create_string_buffer(bytes(buf), capi.GDN_PREFILL_PLAN_BYTES)
        return lib.gdn_prefill_plan_fwd(*args, b, P, 1 << 40, 0, None)

    bad = bytearray(raw)
    struct.pack_into("<i", bad, 160 + 4, ox_row[1] + 64)          # seam 1's OX rows moved
    assert call(bad) == capi.GDN_ERR_SHAPE
    bad = bytearray(raw)
    struct.pack_into("<i", bad, 32 + 4, seq[0])                   # one sequence cut twice
    assert call(bad) == capi.GDN_ERR_SHAPE
    bad = bytearray(raw)
    struct.pack_into("<i", bad, 192, struct.unpack_from("<i", raw, 192)[0] - 1)   # region one row short
    assert call(bad) == capi.GDN_ERR_SHAPE
