"""GPU parity of the q/k/v causal conv1d kernels (the short convolution ahead
of GDN in a Qwen3-Next-style layer) against the fp64 oracle.

Bars: outputs (bf16) equal the oracle's fp64 result rounded to bf16 within
one bf16 unit in the last place (rtol 2^-7; the kernel sums in fp32); conv
states bit for bit (they are copies of bf16 inputs); the decode update equal
bit for bit to the prefill kernel on length-1 sequences and, token by token,
to the prefill kernel on whole sequences.
"""

import pytest
import torch

from conftest import pkg_module
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

ULP = 2.0 ** -7


def _inputs(lens, C, W, S, with_state, with_bias, seed, cu_dtype=torch.int64):
    gen = torch.Generator().manual_seed(seed)
    T, N = sum(lens), len(lens)
    cu = torch.zeros(N + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(torch.tensor(lens, dtype=torch.int64), 0)
    x = torch.randn(T, C, generator=gen).to(torch.bfloat16)
    w = (torch.randn(C, W, generator=gen) * 0.5).to(torch.bfloat16).float()
    b = torch.randn(C, generator=gen) * 0.1 if with_bias else None
    st = torch.randn(N, C, S, generator=gen).to(torch.bfloat16) if with_state else None
    return x, w, b, cu.to(cu_dtype), st


def _close_bf16(y, ref):
    ref = ref.to(torch.bfloat16).double()
    y = y.double().cpu()
    tol = ref.abs() * ULP + 1e-6
    bad = (y - ref).abs() > tol
    assert not bool(bad.any()), (int(bad.sum()), float((y - ref).abs().max()))


@pytest.mark.parametrize("W,S", [(4, 3), (4, 4), (3, 2), (2, 8)])
@pytest.mark.parametrize("with_state,with_bias,act", [(True, False, "silu"), (False, True, "silu"),
                                                      (True, True, None)])
def test_qkv_conv1d_matches_oracle(device, W, S, with_state, with_bias, act):
    conv = pkg_module("conv")
    HQ, HV = 1, 2
    C = 256 * HQ + 128 * HV
    lens = [0, 1, 2, 7, 100, 0, 33, 65]
    print(f"conv W={W} S={S} state={with_state} bias={with_bias} act={act}", flush=True)
    x, w, b, cu, st = _inputs(lens, C, W, S, with_state, with_bias, seed=11 * W + S)
    g = lambda t: None if t is None else t.to(device)
    q, k, v, fin = conv.qkv_conv1d(g(x), g(w), g(b), g(cu), g(st), num_q_heads=HQ, num_v_heads=HV,
                                   activation=act, state_len=S)
    torch.cuda.synchronize()
    y_ref, fin_ref = O.causal_conv1d(x, w, b, cu, st, act, state_len=S)
    y = torch.cat([q.reshape(-1, 128 * HQ), k.reshape(-1, 128 * HQ), v.reshape(-1, 128 * HV)], dim=1)
    _close_bf16(y, y_ref)
    assert torch.equal(fin.cpu(), fin_ref.to(torch.bfloat16))


def test_qkv_split_equals_single_output(device):
    """The q/k/v split writes exactly the channel ranges of the [T, C] output."""
    capi = pkg_module("_capi")
    conv = pkg_module("conv")
    HQ, HV, W = 2, 4, 4
    C = 256 * HQ + 128 * HV
    x, w, b, cu, st = _inputs([50, 77], C, W, 3, True, True, seed=5, cu_dtype=torch.int32)
    x, w, b, cu, st = (t.to(device) for t in (x, w, b, cu, st))
    q, k, v, fin = conv.qkv_conv1d(x, w, b, cu, st, num_q_heads=HQ, num_v_heads=HV)
    out = torch.empty_like(x)
    fin2 = torch.empty_like(fin)
    p = capi.ptr
    rc = capi.lib().gdn_qkv_conv1d_fwd(p(x), p(w), p(b), p(cu), 1, 2, 127, C, W, p(st), p(fin2), 3,
                                       p(out), None, None, 0, 0, capi.GDN_ACT_SILU,
                                       capi.stream_handle(device))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out[:, :256], q.reshape(127, -1))
    assert torch.equal(out[:, 256:512], k.reshape(127, -1))
    assert torch.equal(out[:, 512:], v.reshape(127, -1))
    assert torch.equal(fin, fin2)


def test_padded_batch_tokens_past_last_sequence(device):
    """cu_seqlens[-1] < T (a padded batch): the sequences' tokens and states
    match the unpadded call bit for bit, the padding rows are zero, and the
    launch ends (the tile holding the last sequence end continues past it)."""
    capi = pkg_module("_capi")
    HQ, HV, W, S = 1, 2, 4, 3
    C = 256 * HQ + 128 * HV
    lens = [50, 7, 0, 20]
    T_used, pad = sum(lens), 70                       # 77 tokens in sequences, 70 padding rows
    print(f"conv padded batch lens={lens} pad={pad}", flush=True)
    x, w, b, cu, st = _inputs(lens, C, W, S, True, True, seed=17, cu_dtype=torch.int32)
    gen = torch.Generator().manual_seed(18)
    xp = torch.cat([x, torch.randn(pad, C, generator=gen).to(torch.bfloat16)])
    x, xp, w, b, cu, st = (t.to(device) for t in (x, xp, w, b, cu, st))
    p = capi.ptr
    stream = capi.stream_handle(device)
    out = torch.empty(T_used, C, dtype=torch.bfloat16, device=device)
    fin = torch.empty(len(lens), C, S, dtype=torch.bfloat16, device=device)
    rc = capi.lib().gdn_qkv_conv1d_fwd(p(x), p(w), p(b), p(cu), 1, len(lens), T_used, C, W, p(st),
                                       p(fin), S, p(out), None, None, 0, 0, capi.GDN_ACT_SILU, stream)
    assert rc == 0
    outp = torch.full((T_used + pad, C), 7.0, dtype=torch.bfloat16, device=device)
    finp = torch.empty_like(fin)
    rc = capi.lib().gdn_qkv_conv1d_fwd(p(xp), p(w), p(b), p(cu), 1, len(lens), T_used + pad, C, W,
                                       p(st), p(finp), S, p(outp), None, None, 0, 0,
                                       capi.GDN_ACT_SILU, stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(outp[:T_used], out)
    assert torch.equal(finp, fin)
    assert not bool(outp[T_used:].float().abs().sum() > 0)


@pytest.mark.parametrize("S", [3, 4])
def test_update_equals_prefill_token_by_token(device, S):
    """T decode updates (state in place) reproduce the prefill conv over the
    whole sequences bit for bit, and the final states agree."""
    conv = pkg_module("conv")
    HQ, HV, W, T, B = 1, 2, 4, 9, 3
    C = 256 * HQ + 128 * HV
    gen = torch.Generator().manual_seed(71)
    x = torch.randn(B, T, C, generator=gen).to(torch.bfloat16).to(device)
    w = (torch.randn(C, W, generator=gen) * 0.5).to(device)
    st0 = torch.randn(B, C, S, generator=gen).to(torch.bfloat16).to(device)
    cu = torch.arange(0, (B + 1) * T, T, dtype=torch.int64, device=device)
    q, k, v, fin = conv.qkv_conv1d(x.reshape(B * T, C), w, None, cu, st0, num_q_heads=HQ,
                                   num_v_heads=HV)
    st = st0.clone()
    for t in range(T):
        qt, kt, vt = conv.qkv_conv1d_update(x[:, t], st, w, None, num_q_heads=HQ, num_v_heads=HV)
        torch.cuda.synchronize()
        assert torch.equal(qt[:, 0], q.reshape(B, T, HQ, 128)[:, t])
        assert torch.equal(kt[:, 0], k.reshape(B, T, HQ, 128)[:, t])
        assert torch.equal(vt[:, 0], v.reshape(B, T, HV, 128)[:, t])
    assert torch.equal(st, fin)


def test_update_slot_pool(device):
    """Slot-indexed update: rows slot_ids[b] of a pool are read and updated;
    an out-of-range slot yields zeros and touches nothing."""
    conv = pkg_module("conv")
    HQ, HV, W, S, B, P = 1, 2, 4, 3, 4, 7
    C = 256 * HQ + 128 * HV
    gen = torch.Generator().manual_seed(73)
    x = torch.randn(B, C, generator=gen).to(torch.bfloat16)
    w = torch.randn(C, W, generator=gen) * 0.5
    pool = torch.randn(P, C, S, generator=gen).to(torch.bfloat16)
    slots = torch.tensor([5, 0, 9, 2], dtype=torch.int32)
    pg = pool.to(device)
    q, k, v = conv.qkv_conv1d_update(x.to(device), pg, w.to(device), None, num_q_heads=HQ,
                                     num_v_heads=HV, slot_ids=slots.to(device))
    torch.cuda.synchronize()
    y = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1).cpu()
    expect_pool = pool.clone()
    for b, sl in enumerate(slots.tolist()):
        if 0 <= sl < P:
            yr, sr = O.causal_conv1d_update(x[b:b + 1], pool[sl:sl + 1], w, None, "silu")
            _close_bf16(y[b:b + 1], yr)
            expect_pool[sl] = sr[0].to(torch.bfloat16)
        else:
            assert float(y[b].abs().max()) == 0.0
    assert torch.equal(pg.cpu(), expect_pool)


@pytest.mark.parametrize("B,with_bias", [(1024, True), (7, False)])
def test_update_batch_qk16_v32_matches_oracle(device, B, with_bias):
    """The decode update at the benchmark's width (qk16 / v32: 8192 channels,
    four channel blocks of 2048 per row of workgroups) over a batch whose
    size is and is not a multiple of the sequences a lane takes."""
    conv = pkg_module("conv")
    HQ, HV, W, S = 16, 32, 4, 3
    C = 256 * HQ + 128 * HV
    gen = torch.Generator().manual_seed(B + 5)
    x = torch.randn(B, C, generator=gen).to(torch.bfloat16)
    w = torch.randn(C, W, generator=gen) * 0.5
    bias = torch.randn(C, generator=gen) * 0.1 if with_bias else None
    st = torch.randn(B, C, S, generator=gen).to(torch.bfloat16)
    sg = st.to(device)
    q, k, v = conv.qkv_conv1d_update(x.to(device), sg, w.to(device),
                                     None if bias is None else bias.to(device),
                                     num_q_heads=HQ, num_v_heads=HV)
    torch.cuda.synchronize()
    y = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1).cpu()
    yr, sr = O.causal_conv1d_update(x, st, w, bias, "silu")
    _close_bf16(y, yr)
    assert torch.equal(sg.cpu(), sr.to(torch.bfloat16))


def test_conv_then_prefill_matches_oracle_chain(device):
    """conv1d + SiLU -> GDN prefill with in-kernel q/k L2-norm, against the
    fp64 chain (oracle conv, rounded to bf16 as the kernel stores it, then
    the normalisation and the chunked prefill)."""
    conv = pkg_module("conv")
    pre = pkg_module("prefill")
    inp = pkg_module("inputs")
    HQ, HV, W = 4, 8, 4
    C = 256 * HQ + 128 * HV
    lens = [150, 3, 90]
    x, w, _, cu, st = _inputs(lens, C, W, 3, True, False, seed=79)
    y = inp.prefill_inputs(lens, HQ, HV, seed=80, with_state=True)
    q, k, v, _ = conv.qkv_conv1d(x.to(device), w.to(device), None, cu.to(device), st.to(device),
                                 num_q_heads=HQ, num_v_heads=HV)
    names = ("state", "A_log", "a", "dt_bias", "b")
    g = {n: y[n].to(device) for n in names}
    o, s = pre.gdn_prefill(q, k, v, g["state"], g["A_log"], g["a"], g["dt_bias"], g["b"],
                           cu.to(device), None, qk_l2norm=True)
    torch.cuda.synchronize()
    y_ref, _ = O.causal_conv1d(x, w, None, cu, st, "silu")
    y_ref = y_ref.to(torch.bfloat16)
    T = sum(lens)
    qr = y_ref[:, :128 * HQ].reshape(T, HQ, 128)
    kr = y_ref[:, 128 * HQ:256 * HQ].reshape(T, HQ, 128)
    vr = y_ref[:, 256 * HQ:].reshape(T, HV, 128)
    o_ref, s_ref = O.prefill_chunked(O.qk_l2norm(qr), O.qk_l2norm(kr), vr, y["state"], y["A_log"],
                                     y["a"], y["dt_bias"], y["b"], cu, None)
    torch.testing.assert_close(o.float().cpu().double(), o_ref, atol=1e-2, rtol=1e-2)
    assert float((s.cpu().double() - s_ref).norm() / s_ref.norm()) <= 1e-3


def test_conv_full_size_qk16_v32(device):
    """The 32 768-token workload with 8 varlen sequences at qk16 / v32
    (C = 8192 channels): every output column against the q/k/v split of the
    single-output mode, and a 512-channel slice against the oracle (the
    convolution is channel-separable)."""
    conv = pkg_module("conv")
    inp = pkg_module("inputs")
    HQ, HV, W = 16, 32, 4
    C = 256 * HQ + 128 * HV
    lens = inp.workload_lengths("prefill_varlen8_t32768_qk16_v32")
    T = sum(lens)
    print(f"conv full size T={T} C={C}", flush=True)
    gen = torch.Generator(device=device).manual_seed(83)
    x = torch.randn(T, C, device=device, generator=gen).to(torch.bfloat16)
    w = torch.randn(C, W, device=device, generator=gen) * 0.5
    st = torch.randn(len(lens), C, 3, device=device, generator=gen).to(torch.bfloat16)
    cu = torch.zeros(len(lens) + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(torch.tensor(lens), 0)
    q, k, v, fin = conv.qkv_conv1d(x, w, None, cu.to(device), st, num_q_heads=HQ, num_v_heads=HV)
    torch.cuda.synchronize()
    sl = slice(4096 - 256, 4096 + 256)         # straddles the k / v boundary
    y = torch.cat([k.reshape(T, -1)[:, -256:], v.reshape(T, -1)[:, :256]], dim=1).cpu()
    y_ref, fin_ref = O.causal_conv1d(x[:, sl].cpu(), w[sl].cpu(), None, cu, st[:, sl].cpu(), "silu",
                                     dtype=torch.float32)
    _close_bf16(y, y_ref.double())
    assert torch.equal(fin[:, sl].cpu(), fin_ref.to(torch.bfloat16))
