"""Pins the CPU oracle (oracle/gdn_oracle.py) with checks independent of its formulas.

The reference ships no golden vectors, known-answer tests or fixtures for
this path, so each oracle function is pinned by closed forms, library
routines, invariants and compositions of separately pinned functions.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_oracle as O

DT = torch.float64


def _rand_decode(B=3, HQ=2, HV=4, D=8, seed=0, state=True):
    g = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(B, 1, HQ, D, generator=g, dtype=DT), dim=-1)
    k = F.normalize(torch.randn(B, 1, HQ, D, generator=g, dtype=DT), dim=-1)
    v = torch.randn(B, 1, HV, D, generator=g, dtype=DT)
    S = torch.randn(B, HV, D, D, generator=g, dtype=DT) * 0.3 if state else None
    A_log = torch.rand(HV, generator=g, dtype=DT) * 2 - 2
    a = torch.randn(B, 1, HV, generator=g, dtype=DT)
    dt_bias = torch.randn(HV, generator=g, dtype=DT) * 0.1
    b = torch.randn(B, 1, HV, generator=g, dtype=DT)
    return q, k, v, S, A_log, a, dt_bias, b


# --------------------------------------------------------------------------- gating

def test_softplus_thresh20_matches_torch_softplus():
    x = torch.cat([torch.linspace(-60, 60, 2001, dtype=DT), torch.tensor([20.0, 20.0 + 1e-9], dtype=DT)])
    # torch's softplus(beta=1, threshold=20) is the reference's decode form
    torch.testing.assert_close(O.softplus_thresh20(x), F.softplus(x), rtol=1e-14, atol=1e-300)


def test_softplus_stable_matches_logaddexp():
    x = torch.linspace(-700, 700, 5001, dtype=DT)
    torch.testing.assert_close(O.softplus_stable(x), torch.logaddexp(torch.zeros_like(x), x),
                               rtol=1e-14, atol=1e-300)


def test_softplus_forms_agree_within_bound():
    # both forms differ only above the threshold, by at most log1p(e^-20)
    x = torch.linspace(-30, 60, 9001, dtype=DT)
    d = (O.softplus_thresh20(x) - O.softplus_stable(x)).abs().max()
    assert float(d) <= math.log1p(math.exp(-20.0)) * 1.0001


def test_decode_gates_special_cases():
    HV = 4
    A_log = torch.tensor([-math.inf, 0.0, math.log(2.0), -1.0], dtype=DT)
    dt_bias = torch.zeros(HV, dtype=DT)
    a = torch.tensor([[3.0, 0.0, 1.5, -800.0]], dtype=DT)
    b = torch.tensor([[0.0, 800.0, -800.0, 2.0]], dtype=DT)
    g, beta = O.decode_gates(A_log, a, dt_bias, b)
    assert float(g[0, 0]) == 1.0                                   # exp(A_log) = 0
    assert abs(float(g[0, 1]) - 0.5) < 1e-15                       # exp(-log 2)
    assert abs(float(g[0, 2]) - math.exp(-2.0 * math.log1p(math.exp(1.5)))) < 1e-15
    assert abs(float(g[0, 3]) - 1.0) < 1e-15                       # softplus(-800) ~ 0
    assert float(beta[0, 0]) == 0.5
    assert float(beta[0, 1]) == 1.0
    assert float(beta[0, 2]) < 1e-300
    assert abs(float(beta[0, 3]) - 1.0 / (1.0 + math.exp(-2.0))) < 1e-15
    ld, bt = O.prefill_log_decay_beta(a.reshape(1, HV), b.reshape(1, HV), A_log, dt_bias)
    torch.testing.assert_close(torch.exp(ld), g, rtol=1e-15, atol=0)
    torch.testing.assert_close(bt, torch.sigmoid(b.reshape(1, HV)), rtol=0, atol=0)


# --------------------------------------------------------------------------- decode

def test_decode_zero_state_closed_form():
    q, k, v, _, A_log, a, dt_bias, b = _rand_decode(state=False)
    scale = 0.37
    o, S = O.decode_step(q, k, v, None, A_log, a, dt_bias, b, scale)
    _, beta = O.decode_gates(A_log, a, dt_bias, b)
    kh = k[:, 0].repeat_interleave(2, dim=1)
    qh = q[:, 0].repeat_interleave(2, dim=1)
    # S_new = beta v k^T ; o = scale beta (k.q) v
    S_exp = beta[:, :, None, None] * v[:, 0, :, :, None] * kh[:, :, None, :]
    o_exp = scale * beta[:, :, None] * (kh * qh).sum(-1, keepdim=True) * v[:, 0]
    torch.testing.assert_close(S, S_exp, rtol=1e-13, atol=1e-15)
    torch.testing.assert_close(o[:, 0], o_exp, rtol=1e-13, atol=1e-15)


def test_decode_beta_zero_is_pure_decay():
    q, k, v, S0, A_log, a, dt_bias, _ = _rand_decode()
    b = torch.full((3, 1, 4), -1e4, dtype=DT)          # beta = 0 exactly
    o, S = O.decode_step(q, k, v, S0, A_log, a, dt_bias, b, 1.0)
    g, _ = O.decode_gates(A_log, a, dt_bias, b)
    torch.testing.assert_close(S, g[:, :, None, None] * S0, rtol=1e-14, atol=0)
    qh = q[:, 0].repeat_interleave(2, dim=1)
    o_exp = torch.einsum("nhvk,nhk->nhv", g[:, :, None, None] * S0, qh)
    torch.testing.assert_close(o[:, 0], o_exp, rtol=1e-13, atol=1e-15)


def test_decode_delta_rule_projection_identity():
    # For any inputs: S_new k = (1 - beta |k|^2) g S k + beta |k|^2 v
    q, k, v, S0, A_log, a, dt_bias, b = _rand_decode(seed=3)
    k = k * 1.7                                           # |k| != 1 on purpose
    _, S = O.decode_step(q, k, v, S0, A_log, a, dt_bias, b, 1.0)
    g, beta = O.decode_gates(A_log, a, dt_bias, b)
    kh = k[:, 0].repeat_interleave(2, dim=1)
    kk = (kh * kh).sum(-1)
    lhs = torch.einsum("nhvk,nhk->nhv", S, kh)
    Sk = torch.einsum("nhvk,nhk->nhv", S0, kh)
    rhs = ((1 - beta * kk) * g)[:, :, None] * Sk + (beta * kk)[:, :, None] * v[:, 0]
    torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-13)
    # and the write is exact when g = beta = 1 and |k| = 1
    k1 = F.normalize(k, dim=-1)
    _, S1 = O.decode_step(q, k1, v, S0, torch.full((4,), -math.inf, dtype=DT), a, dt_bias,
                          torch.full((3, 1, 4), 1e4, dtype=DT), 1.0)
    torch.testing.assert_close(torch.einsum("nhvk,nhk->nhv", S1, k1[:, 0].repeat_interleave(2, 1)),
                               v[:, 0], rtol=1e-12, atol=1e-13)


def test_decode_linear_in_v_at_zero_state():
    q, k, v1, _, A_log, a, dt_bias, b = _rand_decode(state=False, seed=5)
    v2 = torch.randn_like(v1)
    o1, S1 = O.decode_step(q, k, v1, None, A_log, a, dt_bias, b, 0.5)
    o2, S2 = O.decode_step(q, k, v2, None, A_log, a, dt_bias, b, 0.5)
    o3, S3 = O.decode_step(q, k, 2.0 * v1 - 3.0 * v2, None, A_log, a, dt_bias, b, 0.5)
    torch.testing.assert_close(o3, 2 * o1 - 3 * o2, rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(S3, 2 * S1 - 3 * S2, rtol=1e-12, atol=1e-13)


def test_decode_head_map_is_consecutive_pairs():
    # v-head h must read qk-head h // (HV/HQ) (repeat_interleave), not h % HQ
    B, HQ, HV, D = 1, 4, 8, 8
    q = torch.zeros(B, 1, HQ, D, dtype=DT)
    k = torch.zeros(B, 1, HQ, D, dtype=DT)
    k[0, 0, 1, 0] = 1.0                                    # only qk-head 1 is non-zero
    q[0, 0, 1, 0] = 1.0
    v = torch.ones(B, 1, HV, D, dtype=DT)
    A_log = torch.zeros(HV, dtype=DT)
    o, S = O.decode_step(q, k, v, None, A_log, torch.zeros(B, 1, HV, dtype=DT),
                         torch.zeros(HV, dtype=DT), torch.zeros(B, 1, HV, dtype=DT), 1.0)
    touched = [h for h in range(HV) if float(S[0, h].abs().sum()) > 0]
    assert touched == [2, 3]
    assert [h for h in range(HV) if float(o[0, 0, h].abs().sum()) > 0] == [2, 3]


def test_decode_default_scale():
    assert O.default_scale(None, 128) == 1.0 / math.sqrt(128)
    assert O.default_scale(0.0, 128) == 1.0 / math.sqrt(128)
    assert O.default_scale(0.25, 128) == 0.25


# --------------------------------------------------------------------------- metadata

@pytest.mark.parametrize("lens", [[0], [64], [1, 63, 64, 65, 128, 0, 200], [0, 0, 5], [130] * 5])
@pytest.mark.parametrize("C", [16, 64, 128])
def test_chunk_metadata_against_vectorised_form(lens, C):
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int64)
    idx = O.chunk_indices(cu, C)
    off = O.chunk_offsets(cu, C)
    n_chunks = (torch.tensor(lens) + C - 1) // C
    total = int(n_chunks.sum())
    assert idx.shape == (total, 2) and idx.dtype == torch.int32
    seq = torch.repeat_interleave(torch.arange(len(lens)), n_chunks)
    local = torch.arange(total) - torch.repeat_interleave(
        torch.cat([torch.zeros(1, dtype=torch.long), n_chunks.cumsum(0)[:-1]]), n_chunks)
    assert torch.equal(idx[:, 0].long(), seq) and torch.equal(idx[:, 1].long(), local)
    assert off.tolist() == [0] + n_chunks.cumsum(0).tolist()
    # every chunk starts inside its sequence and the chunks tile it exactly
    for (n, c) in idx.tolist():
        assert c * C < lens[n]
    for n, L in enumerate(lens):
        covered = sum(min(C, L - c * C) for (m, c) in idx.tolist() if m == n)
        assert covered == L


# --------------------------------------------------------------------------- inverse

@pytest.mark.parametrize("C,block,mag", [(64, 16, 0.3), (64, 16, 1.0), (32, 8, 0.5), (16, 16, 0.9)])
def test_unit_lower_inverse(C, block, mag):
    g = torch.Generator().manual_seed(C + block)
    A = torch.tril(torch.randn(3, C, C, generator=g, dtype=DT) * mag, diagonal=-1)
    Ti = O.unit_lower_inverse_blocked(A, block)
    eye = torch.eye(C, dtype=DT).expand(3, C, C)
    ref = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
    big = max(1.0, float(ref.abs().max()))
    torch.testing.assert_close(Ti, ref, rtol=1e-10, atol=1e-12 * big)
    torch.testing.assert_close((eye + A) @ Ti, eye, rtol=0, atol=1e-12 * big)
    assert torch.equal(torch.triu(Ti, 1), torch.zeros_like(Ti))


# --------------------------------------------------------------------------- prefill

def _rand_prefill(lens, HQ=2, HV=4, D=16, seed=0, state=True, alog=(-2.0, 0.0)):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1)
    k = F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1)
    v = torch.randn(T, HV, D, generator=g, dtype=DT)
    S = torch.randn(len(lens), HV, D, D, generator=g, dtype=DT) * 0.1 if state else None
    A_log = torch.rand(HV, generator=g, dtype=DT) * (alog[1] - alog[0]) + alog[0]
    a = torch.randn(T, HV, generator=g, dtype=DT)
    dt_bias = torch.randn(HV, generator=g, dtype=DT) * 0.1
    b = torch.randn(T, HV, generator=g, dtype=DT)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int64)
    return q, k, v, S, A_log, a, dt_bias, b, cu


def test_prefill_recurrent_equals_repeated_decode():
    lens = [7]
    q, k, v, S, A_log, a, dt_bias, b, cu = _rand_prefill(lens, seed=1)
    o, Sf = O.prefill_recurrent(q, k, v, S, A_log, a, dt_bias, b, cu, 0.3)
    St = S
    for t in range(7):
        ot, St = O.decode_step(q[t:t + 1, None], k[t:t + 1, None], v[t:t + 1, None], St, A_log,
                               a[t:t + 1, None], dt_bias, b[t:t + 1, None], 0.3)
        # the two softplus forms agree to ~1e-16 for |x| < 20
        torch.testing.assert_close(o[t], ot[0, 0], rtol=1e-12, atol=1e-13)
    torch.testing.assert_close(Sf, St, rtol=1e-12, atol=1e-13)


def test_prefill_varlen_equals_separate_runs_and_none_state():
    lens = [5, 0, 9, 3]
    q, k, v, S, A_log, a, dt_bias, b, cu = _rand_prefill(lens, seed=2)
    o, Sf = O.prefill_recurrent(q, k, v, S, A_log, a, dt_bias, b, cu, 0.5)
    for n in range(len(lens)):
        s, e = int(cu[n]), int(cu[n + 1])
        on, Sn = O.prefill_recurrent(q[s:e], k[s:e], v[s:e], S[n:n + 1], A_log, a[s:e], dt_bias,
                                     b[s:e], torch.tensor([0, e - s]), 0.5)
        torch.testing.assert_close(o[s:e], on, rtol=0, atol=0)
        torch.testing.assert_close(Sf[n], Sn[0], rtol=0, atol=0)
    torch.testing.assert_close(Sf[1], S[1], rtol=0, atol=0)        # empty sequence keeps its state
    o0, S0 = O.prefill_recurrent(q, k, v, None, A_log, a, dt_bias, b, cu, 0.5)
    oz, Sz = O.prefill_recurrent(q, k, v, torch.zeros_like(S), A_log, a, dt_bias, b, cu, 0.5)
    torch.testing.assert_close(o0, oz, rtol=0, atol=0)
    torch.testing.assert_close(S0, Sz, rtol=0, atol=0)


@pytest.mark.parametrize("split", [1, 64, 100, 127])
def test_prefill_split_invariance(split):
    lens = [150]
    q, k, v, S, A_log, a, dt_bias, b, cu = _rand_prefill(lens, seed=3)
    o, Sf = O.prefill_chunked(q, k, v, S, A_log, a, dt_bias, b, cu, 0.4)
    t = split
    o1, S1 = O.prefill_chunked(q[:t], k[:t], v[:t], S, A_log, a[:t], dt_bias, b[:t],
                               torch.tensor([0, t]), 0.4)
    o2, S2 = O.prefill_chunked(q[t:], k[t:], v[t:], S1, A_log, a[t:], dt_bias, b[t:],
                               torch.tensor([0, 150 - t]), 0.4)
    torch.testing.assert_close(torch.cat([o1, o2]), o, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(S2, Sf, rtol=1e-10, atol=1e-11)


@pytest.mark.parametrize("C", [1, 16, 32, 64, 128])
@pytest.mark.parametrize("alog", [(-2.0, 0.0), (-9.0, -7.0)])
def test_prefill_chunked_equals_recurrent(C, alog):
    lens = [1, 64, 130, 0, 77]
    q, k, v, S, A_log, a, dt_bias, b, cu = _rand_prefill(lens, seed=4, alog=alog)
    o_r, S_r = O.prefill_recurrent(q, k, v, S, A_log, a, dt_bias, b, cu, 0.2)
    o_c, S_c = O.prefill_chunked(q, k, v, S, A_log, a, dt_bias, b, cu, 0.2, chunk_size=C)
    torch.testing.assert_close(o_c, o_r, rtol=1e-10, atol=1e-11)
    torch.testing.assert_close(S_c, S_r, rtol=1e-10, atol=1e-11)


def test_prefill_reference_storage_error_is_bf16_sized():
    # The reference's bf16 intermediates cost ~1e-3 relative state error: a
    # measured property of the reference's choices, not a parity target.
    lens = [300]
    q, k, v, S, A_log, a, dt_bias, b, cu = _rand_prefill(lens, D=32, seed=6)
    _, S_ex = O.prefill_chunked(q, k, v, S, A_log, a, dt_bias, b, cu, None)
    _, S_bf = O.prefill_chunked(q, k, v, S, A_log, a, dt_bias, b, cu, None, reference_storage=True)
    rel = float((S_bf - S_ex).norm() / S_ex.norm())
    assert 1e-4 < rel < 1e-2


# --------------------------------------------------------------------------- q/k L2-norm

def test_qk_l2norm_matches_normalize_when_eps_negligible():
    g = torch.Generator().manual_seed(41)
    x = torch.randn(5, 3, 128, generator=g, dtype=DT) * 7.0      # |x|^2 ~ 6e3 >> eps
    ref = F.normalize(x, dim=-1)
    out = O.qk_l2norm(x)
    # relative effect of eps on the norm is eps / (2 |x|^2) < 1e-9
    torch.testing.assert_close(out, ref, atol=1e-9, rtol=1e-9)
    assert out.dtype == DT and out.shape == x.shape


@pytest.mark.parametrize("c", [0.0, 1e-4, 1e-3, 0.5, 1.0, 3.0])
def test_qk_l2norm_closed_form_on_scaled_unit_vectors(c):
    D = 128
    for i in (0, 17, 127):
        x = torch.zeros(D, dtype=DT)
        x[i] = -c if i == 17 else c
        out = O.qk_l2norm(x)
        expect = torch.zeros(D, dtype=DT)
        expect[i] = x[i] / math.sqrt(c * c + 1e-6)
        torch.testing.assert_close(out, expect, atol=0.0, rtol=1e-14)


def test_qk_l2norm_equivariance_and_eps_argument():
    g = torch.Generator().manual_seed(42)
    x = torch.randn(4, 128, generator=g, dtype=DT) * 0.01       # eps matters at this size
    perm = torch.randperm(128, generator=g)
    sign = torch.where(torch.rand(128, generator=g) < 0.5, -1.0, 1.0).to(DT)
    out = O.qk_l2norm(x)
    torch.testing.assert_close(O.qk_l2norm(x[:, perm] * sign), out[:, perm] * sign,
                               atol=1e-15, rtol=1e-13)
    # the output norm is |x| / sqrt(|x|^2 + eps), strictly below 1
    n2 = (x * x).sum(-1)
    torch.testing.assert_close(out.norm(dim=-1), torch.sqrt(n2 / (n2 + 1e-6)), atol=0, rtol=1e-13)
    assert bool((out.norm(dim=-1) < 1).all())
    # eps = 0 is plain normalisation; bf16 input is widened, not rounded
    torch.testing.assert_close(O.qk_l2norm(x, eps=0.0), F.normalize(x, dim=-1), atol=0, rtol=1e-14)
    xb = x.to(torch.bfloat16)
    assert O.qk_l2norm(xb).dtype == DT


# --------------------------------------------------------------------------- per-chunk states

@pytest.mark.parametrize("lens,C", [([150, 0, 64, 1, 129], 64), ([40, 33], 16)])
def test_prefill_chunk_states_against_prefix_runs(lens, C):
    g = torch.Generator().manual_seed(sum(lens) + C)
    HQ, HV, D = 2, 4, 8
    T = sum(lens)
    q = F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1)
    k = F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1)
    v = torch.randn(T, HV, D, generator=g, dtype=DT)
    a = torch.randn(T, HV, generator=g, dtype=DT)
    b = torch.randn(T, HV, generator=g, dtype=DT)
    A_log = torch.rand(HV, generator=g, dtype=DT) * 2 - 2
    dt_bias = torch.randn(HV, generator=g, dtype=DT) * 0.1
    S0 = torch.randn(len(lens), HV, D, D, generator=g, dtype=DT) * 0.3
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)), dtype=torch.int64)
    h = O.prefill_chunk_states(q, k, v, S0, A_log, a, dt_bias, b, cu, chunk_size=C)
    offs = O.chunk_offsets(cu, C)
    assert h.shape == (int(offs[-1]), HV, D, D)
    for n, L in enumerate(lens):
        bos = int(cu[n])
        for i in range((L + C - 1) // C):
            slot = int(offs[n]) + i
            if i == 0:
                torch.testing.assert_close(h[slot], S0[n], atol=0, rtol=0)
                continue
            sl = slice(bos, bos + C * i)
            _, s_ref = O.prefill_recurrent(q[sl], k[sl], v[sl], S0[n:n + 1], A_log, a[sl], dt_bias,
                                           b[sl], torch.tensor([0, C * i]), 1.0)
            torch.testing.assert_close(h[slot], s_ref[0], atol=1e-12, rtol=1e-12)
    h0 = O.prefill_chunk_states(q, k, v, None, A_log, a, dt_bias, b, cu, chunk_size=C)
    assert float(h0[0].abs().max()) == 0.0


# ---------------------------------------------------------------------------
# causal conv1d (the short convolution ahead of GDN in a Qwen3-Next-style layer)


def _conv_brute(x, w, bias, cu, state, act):
    """Elementwise loops: y[t, c] = act(bias + sum_w w[c, w] * hist(t - (W-1) + w))."""
    T, C = x.shape
    W = w.shape[1]
    N = cu.numel() - 1
    S = state.shape[2] if state is not None else W - 1
    y = torch.zeros(T, C, dtype=torch.float64)
    for n in range(N):
        bos, eos = int(cu[n]), int(cu[n + 1])
        for t in range(bos, eos):
            for c in range(C):
                acc = float(bias[c]) if bias is not None else 0.0
                for j in range(W):
                    u = t - (W - 1) + j
                    if u >= bos:
                        val = float(x[u, c])
                    else:
                        si = S - (bos - u)
                        val = float(state[n, c, si]) if (state is not None and si >= 0) else 0.0
                    acc += float(w[c, j]) * val
                y[t, c] = acc / (1.0 + math.exp(-acc)) if act == "silu" else acc
    return y


@pytest.mark.parametrize("W,S", [(4, 3), (4, 4), (3, 2), (2, 5)])
def test_causal_conv1d_matches_brute_force(W, S):
    gen = torch.Generator().manual_seed(31 + W + S)
    lens = [0, 1, 2, 7, 3]
    cu = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0).tolist()))
    T, C, N = sum(lens), 6, len(lens)
    x = torch.randn(T, C, generator=gen, dtype=torch.float64)
    w = torch.randn(C, W, generator=gen, dtype=torch.float64)
    bias = torch.randn(C, generator=gen, dtype=torch.float64)
    state = torch.randn(N, C, S, generator=gen, dtype=torch.float64)
    for act in ("silu", None):
        y, fin = O.causal_conv1d(x, w, bias, cu, state, act)
        torch.testing.assert_close(y, _conv_brute(x, w, bias, cu, state, act), rtol=1e-12, atol=1e-12)
    # final state: the last S entries of [state, x_seq] per sequence
    for n in range(N):
        h = torch.cat([state[n], x[int(cu[n]):int(cu[n + 1])].T], dim=1)
        assert torch.equal(fin[n], h[:, -S:])


def test_causal_conv1d_matches_torch_conv1d():
    """Library routine: F.conv1d with groups = C and W - 1 zeros of left padding
    (no state) on each sequence."""
    gen = torch.Generator().manual_seed(41)
    lens = [5, 17, 1]
    cu = torch.tensor([0, 5, 22, 23])
    C, W = 8, 4
    x = torch.randn(23, C, generator=gen, dtype=torch.float64)
    w = torch.randn(C, W, generator=gen, dtype=torch.float64)
    y, _ = O.causal_conv1d(x, w, None, cu, None, None)
    for n in range(3):
        seq = x[int(cu[n]):int(cu[n + 1])].T[None]                   # [1, C, L]
        ref = torch.nn.functional.conv1d(seq, w[:, None, :], padding=W - 1, groups=C)[0, :, :lens[n]]
        torch.testing.assert_close(y[int(cu[n]):int(cu[n + 1])], ref.T, rtol=1e-12, atol=1e-12)


def test_causal_conv1d_impulse_and_linearity():
    C, W = 4, 4
    w = torch.arange(1, C * W + 1, dtype=torch.float64).reshape(C, W)
    x = torch.zeros(6, C, dtype=torch.float64)
    x[1] = 1.0
    y, _ = O.causal_conv1d(x, w, None, torch.tensor([0, 6]), None, None)
    # token 1 + d sees the impulse through tap W - 1 - d
    for d in range(W):
        torch.testing.assert_close(y[1 + d], w[:, W - 1 - d])
    assert float(y[0].abs().max()) == 0.0 and float(y[5].abs().max()) == 0.0
    gen = torch.Generator().manual_seed(43)
    a, b = torch.randn(6, C, generator=gen, dtype=torch.float64), torch.randn(6, C, generator=gen, dtype=torch.float64)
    ya, _ = O.causal_conv1d(a, w, None, torch.tensor([0, 6]), None, None)
    yb, _ = O.causal_conv1d(b, w, None, torch.tensor([0, 6]), None, None)
    yab, _ = O.causal_conv1d(2 * a - b, w, None, torch.tensor([0, 6]), None, None)
    torch.testing.assert_close(yab, 2 * ya - yb)


def test_causal_conv1d_split_invariance_and_update():
    gen = torch.Generator().manual_seed(47)
    C, W, S, T = 5, 4, 3, 11
    x = torch.randn(T, C, generator=gen, dtype=torch.float64)
    w = torch.randn(C, W, generator=gen, dtype=torch.float64)
    s0 = torch.randn(1, C, S, generator=gen, dtype=torch.float64)
    y, fin = O.causal_conv1d(x, w, None, torch.tensor([0, T]), s0, "silu")
    for t in (1, 2, 6):
        y1, s1 = O.causal_conv1d(x[:t], w, None, torch.tensor([0, t]), s0, "silu")
        y2, s2 = O.causal_conv1d(x[t:], w, None, torch.tensor([0, T - t]), s1, "silu")
        torch.testing.assert_close(torch.cat([y1, y2]), y)
        torch.testing.assert_close(s2, fin)
    # decode: token by token through the update form
    st = s0.clone()
    for t in range(T):
        yt, st = O.causal_conv1d_update(x[t:t + 1], st, w, None, "silu")
        torch.testing.assert_close(yt[0], y[t])
    torch.testing.assert_close(st, fin)


# --------------------------------------------------------------------------- prefill backward

def _rand_prefill_bwd(lens, HQ=2, HV=4, D=6, seed=0, state=True):
    g = torch.Generator().manual_seed(seed)
    T = sum(lens)
    x = dict(
        q=F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1),
        k=F.normalize(torch.randn(T, HQ, D, generator=g, dtype=DT), dim=-1),
        v=torch.randn(T, HV, D, generator=g, dtype=DT),
        state=torch.randn(len(lens), HV, D, D, generator=g, dtype=DT) * 0.3 if state else None,
        A_log=torch.rand(HV, generator=g, dtype=DT) * 2 - 2,
        a=torch.randn(T, HV, generator=g, dtype=DT),
        dt_bias=torch.randn(HV, generator=g, dtype=DT) * 0.1,
        b=torch.randn(T, HV, generator=g, dtype=DT),
        cu_seqlens=torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int64))
    d_out = torch.randn(T, HV, D, generator=g, dtype=DT)
    d_fin = torch.randn(len(lens), HV, D, D, generator=g, dtype=DT)
    return x, d_out, d_fin


def _loss(x, d_out, d_fin, scale):
    o, fin = O.prefill_recurrent(x["q"], x["k"], x["v"], x["state"], x["A_log"], x["a"],
                                 x["dt_bias"], x["b"], x["cu_seqlens"], scale)
    return (o * d_out).sum() + (fin * d_fin).sum()


def _all_grads(x, d_out, d_fin, scale):
    gr = O.prefill_backward(x["q"], x["k"], x["v"], x["state"], x["A_log"], x["a"], x["dt_bias"],
                            x["b"], x["cu_seqlens"], scale, d_out, d_fin)
    gg = O.gate_backward(x["A_log"], x["a"], x["dt_bias"], x["b"], gr["dg"], gr["dbeta"])
    return {"q": gr["dq"], "k": gr["dk"], "v": gr["dv"], "state": gr["dh0"], "a": gg["da"],
            "b": gg["db"], "A_log": gg["dA_log"], "dt_bias": gg["ddt_bias"]}


@pytest.mark.parametrize("lens,state", [([5, 0, 9], True), ([70], False), ([1, 3], True)])
def test_prefill_backward_matches_finite_differences(lens, state):
    """Central differences of L = <o, R1> + <S_final, R2> along random
    directions, per input, against <grad, direction> (fp64, eps 1e-6)."""
    x, d_out, d_fin = _rand_prefill_bwd(lens, seed=len(lens) + sum(lens), state=state)
    scale = 0.37
    grads = _all_grads(x, d_out, d_fin, scale)
    gen = torch.Generator().manual_seed(5)
    for name, gval in grads.items():
        if x[name] is None:
            continue
        dirn = torch.randn(x[name].shape, generator=gen, dtype=DT)
        eps = 1e-6
        xp = dict(x); xp[name] = x[name] + eps * dirn
        xm = dict(x); xm[name] = x[name] - eps * dirn
        fd = (_loss(xp, d_out, d_fin, scale) - _loss(xm, d_out, d_fin, scale)) / (2 * eps)
        an = (gval * dirn).sum()
        assert abs(float(fd - an)) <= 1e-6 * max(1.0, abs(float(an))), (name, float(fd), float(an))


def test_prefill_backward_matches_autograd():
    """torch.autograd through the forward oracle gives the same gradients."""
    x, d_out, d_fin = _rand_prefill_bwd([13, 6], HQ=1, HV=2, D=5, seed=3)
    scale = -0.5
    leaves = {n: x[n].clone().requires_grad_(True) for n in ("q", "k", "v", "state", "A_log", "a",
                                                           "dt_bias", "b")}
    xa = dict(x, **leaves)
    L = _loss(xa, d_out, d_fin, scale)
    auto = dict(zip(leaves, torch.autograd.grad(L, list(leaves.values()))))
    mine = _all_grads(x, d_out, d_fin, scale)
    for n in leaves:
        torch.testing.assert_close(mine[n], auto[n], rtol=1e-10, atol=1e-12)


def test_prefill_backward_zero_state_and_no_final_grad():
    """With d_final = None and no initial state: the gradient of <o, R1> alone
    (autograd), and dh0 equals the gradient through a zero initial state."""
    x, d_out, _ = _rand_prefill_bwd([4, 8], HQ=2, HV=2, D=4, seed=9, state=False)
    gr = O.prefill_backward(x["q"], x["k"], x["v"], None, x["A_log"], x["a"], x["dt_bias"], x["b"],
                            x["cu_seqlens"], 1.0, d_out, None)
    s0 = torch.zeros(2, 2, 4, 4, dtype=DT, requires_grad=True)
    o, _ = O.prefill_recurrent(x["q"], x["k"], x["v"], s0, x["A_log"], x["a"], x["dt_bias"], x["b"],
                               x["cu_seqlens"], 1.0)
    (ds0,) = torch.autograd.grad((o * d_out).sum(), [s0])
    torch.testing.assert_close(gr["dh0"], ds0, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("lens,C,state", [([5, 0, 9], 4, True), ([70, 33], 16, True),
                                          ([130], 64, False), ([1, 64, 65], 64, True)])
def test_prefill_backward_chunked_equals_per_token(lens, C, state):
    """The chunked backward (state-gradient transitions M, R per chunk, then the
    per-chunk gradients from S and dSn) equals the per-token reverse recurrence."""
    x, d_out, d_fin = _rand_prefill_bwd(lens, HQ=2, HV=4, D=8, seed=1, state=state)
    args = [x[n] for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")]
    r1 = O.prefill_backward(*args, 0.3, d_out, d_fin)
    r2 = O.prefill_backward_chunked(*args, 0.3, d_out, d_fin, chunk_size=C)
    for k in r1:
        torch.testing.assert_close(r2[k], r1[k], rtol=1e-10, atol=1e-12)
