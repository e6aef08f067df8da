"""CPU oracle for the Gated DeltaNet (GDN) decode and prefill operators.

TEST INFRASTRUCTURE ONLY.  This module is the oracle the HIP kernels are held
against: only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline leg may import it.  No product code path routes through it.

It restates, in plain PyTorch on the CPU (float64 by default, float32 for the
timed CPU baseline), the arithmetic of the two reference operators:

* decode  -- ``gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py`` (DEC)
* prefill -- ``gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py`` (PRE)

Every function cites the reference lines it follows.  Head counts are
generic: v-head ``h`` reads qk-head ``h // (HV // HQ)`` (DEC:47, PRE:495, the
reference hard-codes ratio 2).  The recurrent state is "k-last":
``state[n, h, v, k]`` fp32 with K contiguous (DEC:53,70; PRE:1129).

How each function is pinned (tests/test_oracle.py):

* gating           -- torch.nn.functional.softplus / sigmoid closed forms and
                      special cases (A_log -> -inf gives g = 1, b = 0 gives 0.5).
* decode_step      -- closed forms at state = 0 and beta = 0, the delta-rule
                      write invariant (g = beta = 1, |k| = 1 gives S' k = v),
                      linearity in v, and an elementwise brute-force loop.
* chunk metadata   -- brute-force enumeration over random cu_seqlens including
                      empty sequences and exact multiples of the chunk size.
* unit_lower_inverse_blocked -- (I + A) Tm = I and torch.linalg.solve_triangular.
* prefill_recurrent -- equals repeated decode_step with the prefill softplus,
                      closed forms at T = 1, split / varlen invariances.
* prefill_chunked  -- equals prefill_recurrent in float64 at chunk sizes
                      1, 16, 32, 64, 128 including ragged tails.
* prefill_chunk_states -- the first state of each sequence is its initial
                      state; state i equals prefill_recurrent's final state
                      over the first 64 i tokens; the count and order follow
                      chunk_offsets.
* qk_l2norm        -- torch.nn.functional.normalize where eps is negligible,
                      the closed form c/sqrt(c^2 + eps) on scaled unit vectors,
                      zero maps to zero, sign/permutation equivariance.
* prefill_backward -- central finite differences of <o, R1> + <S_final, R2>
                      along random directions for every input, and
                      torch.autograd through prefill_recurrent.
* prefill_backward_chunked -- equals prefill_backward in float64 at chunk
                      sizes 4, 16, 64 with ragged tails and empty sequences.
* gate_backward    -- through the finite-difference and autograd checks of
                      prefill_backward (a, b, A_log, dt_bias directions).
* causal_conv1d, causal_conv1d_update -- the short causal convolution that
                      precedes GDN in a Qwen3-Next-style layer (no reference
                      counterpart): torch.nn.functional.conv1d with groups =
                      channels and left zero padding, an elementwise
                      brute-force loop, the impulse response (the reversed
                      taps), split invariance through the returned state, and
                      update == a length-1 sequence.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

__all__ = [
    "softplus_thresh20",
    "softplus_stable",
    "decode_gates",
    "prefill_log_decay_beta",
    "decode_step",
    "chunk_indices",
    "chunk_offsets",
    "unit_lower_inverse_blocked",
    "prefill_recurrent",
    "prefill_chunked",
    "prefill_chunk_states",
    "default_scale",
    "qk_l2norm",
    "causal_conv1d",
    "causal_conv1d_update",
    "prefill_backward",
    "prefill_backward_chunked",
    "gate_backward",
]


def default_scale(scale: Optional[float], head_dim: int) -> float:
    """``None`` or ``0.0`` means ``1/sqrt(D)`` (DEC:112-115, PRE:1777-1778)."""
    if scale is None or float(scale) == 0.0:
        return 1.0 / math.sqrt(head_dim)
    return float(scale)


L2NORM_EPS = 1e-6


def qk_l2norm(x: torch.Tensor, eps: float = L2NORM_EPS, dtype=torch.float64) -> torch.Tensor:
    """``x * (sum_d x_d^2 + eps)^(-1/2)`` over the last (head) dimension.

    The reference has no counterpart: its operators take q and k already
    L2-normalised by the caller (the benchmark inputs are drawn that way).
    This is the normalisation the ``qk_l2norm`` option applies inside the
    kernels to raw bf16 q/k before the decode step (DEC:72-76) or the chunked
    prefill (PRE:1049-1129); the result is not rounded back to bf16.
    """
    x = x.to(dtype)
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


# ----------------------------------------------------------------------------
# gating
# ----------------------------------------------------------------------------

def softplus_thresh20(x: torch.Tensor) -> torch.Tensor:
    """Decode softplus: ``x <= 20 ? log(1 + e^x) : x`` (DEC:21-23)."""
    return torch.where(x <= 20.0, torch.log1p(torch.exp(torch.clamp(x, max=20.0))), x)


def softplus_stable(x: torch.Tensor) -> torch.Tensor:
    """Prefill softplus: ``x > 0 ? x + log(1 + e^-x) : log(1 + e^x)`` (PRE:1711-1720)."""
    pos = x + torch.log1p(torch.exp(-torch.clamp(x, min=0.0)))
    neg = torch.log1p(torch.exp(torch.clamp(x, max=0.0)))
    return torch.where(x > 0, pos, neg)


def decode_gates(A_log, a, dt_bias, b, dtype=torch.float64) -> Tuple[torch.Tensor, torch.Tensor]:
    """Decode decay ``g`` and write strength ``beta`` per (batch, v-head).

    ``g = exp(-exp(A_log[h]) * softplus20(a[n,h] + dt_bias[h]))`` and
    ``beta = 1 / (1 + exp(-b[n,h]))`` (DEC:59-65).  ``a``/``b`` may be
    ``[B, HV]`` or ``[B, 1, HV]``.
    """
    HV = A_log.shape[-1]
    a = a.reshape(-1, HV).to(dtype)
    b = b.reshape(-1, HV).to(dtype)
    log_g = -torch.exp(A_log.to(dtype))[None, :] * softplus_thresh20(a + dt_bias.to(dtype)[None, :])
    g = torch.exp(log_g)
    beta = 1.0 / (1.0 + torch.exp(-b))
    return g, beta


def prefill_log_decay_beta(a, b, A_log, dt_bias, dtype=torch.float64):
    """Per-token log-decay and beta for prefill, ``[T, HV]`` each.

    ``log_decay = -exp(A_log) * softplus_stable(a + dt_bias)`` and
    ``beta = sigmoid(b)`` (PRE:1706-1722).  The reference then cumsums the
    log-decay inside each 64-token chunk (PRE:1721); :func:`prefill_chunked`
    does that step itself so that the per-token form stays available.
    """
    ld = -torch.exp(A_log.to(dtype))[None, :] * softplus_stable(a.to(dtype) + dt_bias.to(dtype)[None, :])
    beta = torch.sigmoid(b.to(dtype))
    return ld, beta


# ----------------------------------------------------------------------------
# decode
# ----------------------------------------------------------------------------

def _expand_heads(x: torch.Tensor, HV: int) -> torch.Tensor:
    """qk-head -> v-head map ``h -> h // (HV//HQ)`` (repeat_interleave; DEC:47)."""
    HQ = x.shape[-2]
    assert HV % HQ == 0
    return x.repeat_interleave(HV // HQ, dim=-2)


def decode_step(q, k, v, state, A_log, a, dt_bias, b, scale=None, dtype=torch.float64):
    """One GDN decode step for every (batch, v-head) (DEC:67-79).

    Shapes: ``q, k [B, 1, HQ, D]``, ``v [B, 1, HV, D]``, ``state [B, HV, V, K]``
    or ``None`` (zeros, DEC:86-94).  Per (n, h), in ``dtype``::

        S'    = g * S                      (DEC:72)
        delta = beta * (v - S' k)          (DEC:73-74, decayed state)
        S_new = S' + delta k^T             (DEC:75)
        o     = scale * S_new q            (DEC:56, 76)

    Returns ``(o [B, 1, HV, D], S_new [B, HV, V, K])`` in ``dtype``; the
    caller casts ``o`` to bf16 as DEC:78 does.
    """
    B, _, HQ, D = q.shape
    HV = v.shape[2]
    scale = default_scale(scale, D)
    qh = _expand_heads(q.reshape(B, HQ, D).to(dtype), HV)
    kh = _expand_heads(k.reshape(B, HQ, D).to(dtype), HV)
    vh = v.reshape(B, HV, D).to(dtype)
    if state is None:
        S = torch.zeros(B, HV, D, D, dtype=dtype)
    else:
        S = state.to(dtype)
    g, beta = decode_gates(A_log, a, dt_bias, b, dtype)
    S1 = g[:, :, None, None] * S
    sk = torch.einsum("nhvk,nhk->nhv", S1, kh)
    delta = beta[:, :, None] * (vh - sk)
    S_new = S1 + delta[:, :, :, None] * kh[:, :, None, :]
    o = scale * torch.einsum("nhvk,nhk->nhv", S_new, qh)
    return o.reshape(B, 1, HV, D), S_new


# ----------------------------------------------------------------------------
# varlen chunk metadata
# ----------------------------------------------------------------------------

def chunk_indices(cu_seqlens: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """``[(seq_id, local_chunk_id)]`` int32 ``[NT, 2]`` (PRE:175-202).

    Sequences of length 0 contribute no chunks; a ragged tail is one chunk.
    """
    cu = [int(x) for x in cu_seqlens.tolist()]
    rows = []
    for n in range(len(cu) - 1):
        length = cu[n + 1] - cu[n]
        for c in range((length + chunk_size - 1) // chunk_size):
            rows.append((n, c))
    if not rows:
        return torch.empty((0, 2), dtype=torch.int32)
    return torch.tensor(rows, dtype=torch.int32)


def chunk_offsets(cu_seqlens: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """Exclusive prefix sum of per-sequence chunk counts, int64 ``[N+1]`` (PRE:204-209)."""
    cu = [int(x) for x in cu_seqlens.tolist()]
    out = [0]
    for n in range(len(cu) - 1):
        out.append(out[-1] + (cu[n + 1] - cu[n] + chunk_size - 1) // chunk_size)
    return torch.tensor(out, dtype=torch.int64)


# ----------------------------------------------------------------------------
# (I + A)^-1 for a strictly lower-triangular A
# ----------------------------------------------------------------------------

def unit_lower_inverse_blocked(A: torch.Tensor, block: int = 16) -> torch.Tensor:
    """``(I + A)^-1`` for strictly lower-triangular ``A [..., C, C]``.

    Follows the reference's blocked scheme (PRE:661-737): each ``block x
    block`` diagonal block is inverted by row-wise forward substitution
    (PRE:680-703) and the off-diagonal blocks are merged with block products
    ``Ti_ij = -Ti_ii * sum_{j<=m<i} A_im Ti_mj`` (PRE:718-737), generalised
    here from 4 blocks to ``C / block``.
    """
    C = A.shape[-1]
    assert C % block == 0
    nb = C // block
    L = torch.tril(A, diagonal=-1)
    Ti = torch.zeros_like(L)
    eye = torch.eye(block, dtype=A.dtype)
    for bi in range(nb):
        s = bi * block
        blk = L[..., s:s + block, s:s + block]
        inv = torch.zeros_like(blk)
        inv[...] = eye
        for i in range(1, block):
            # row i of (I + blk)^-1 = e_i - sum_{j<i} blk[i, j] * inv[j, :]
            inv[..., i, :] = eye[i] - torch.einsum("...j,...jc->...c", blk[..., i, :i], inv[..., :i, :])
        Ti[..., s:s + block, s:s + block] = inv
    for bi in range(1, nb):
        for bj in range(bi - 1, -1, -1):
            si, sj = bi * block, bj * block
            acc = torch.zeros_like(Ti[..., si:si + block, sj:sj + block])
            for bm in range(bj, bi):
                sm = bm * block
                acc = acc + L[..., si:si + block, sm:sm + block] @ Ti[..., sm:sm + block, sj:sj + block]
            Ti[..., si:si + block, sj:sj + block] = -Ti[..., si:si + block, si:si + block] @ acc
    return Ti


# ----------------------------------------------------------------------------
# prefill
# ----------------------------------------------------------------------------

def _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens):
    T, HQ, D = q.shape
    HV = v.shape[1]
    assert k.shape == (T, HQ, D) and v.shape == (T, HV, D)
    assert a.shape == (T, HV) and b.shape == (T, HV)
    N = cu_seqlens.numel() - 1
    assert int(cu_seqlens[-1]) == T and int(cu_seqlens[0]) == 0
    if state is not None:
        assert state.shape == (N, HV, D, D)
    return T, HQ, HV, D, N


def prefill_recurrent(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None,
                      dtype=torch.float64):
    """Token-by-token GDN prefill: the definition of what the chunked form computes.

    For each sequence ``[cu[n], cu[n+1])`` starting from ``state[n]`` (zeros if
    ``state`` is ``None``, PRE:1049, 1121), every token applies the decode
    step of DEC:72-76 with ``g_t = exp(log_decay_t)`` from the prefill gating
    (PRE:1711-1722).  Returns ``(o [T, HV, D], final_state [N, HV, V, K])``.
    """
    T, HQ, HV, D, N = _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens)
    scale = default_scale(scale, D)
    ld, beta = prefill_log_decay_beta(a, b, A_log, dt_bias, dtype)
    qh = _expand_heads(q.to(dtype), HV)
    kh = _expand_heads(k.to(dtype), HV)
    vh = v.to(dtype)
    o = torch.zeros(T, HV, D, dtype=dtype)
    final = torch.zeros(N, HV, D, D, dtype=dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    for n in range(N):
        S = torch.zeros(HV, D, D, dtype=dtype) if state is None else state[n].to(dtype).clone()
        for t in range(cu[n], cu[n + 1]):
            S = torch.exp(ld[t])[:, None, None] * S
            sk = torch.einsum("hvk,hk->hv", S, kh[t])
            delta = beta[t][:, None] * (vh[t] - sk)
            S = S + delta[:, :, None] * kh[t][:, None, :]
            o[t] = scale * torch.einsum("hvk,hk->hv", S, qh[t])
        final[n] = S
    return o, final


def prefill_chunk_states(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, chunk_size: int = 64,
                         dtype=torch.float64):
    """States entering every chunk, ``h [NT, HV, V, K]`` (PRE:1341-1398).

    ``chunk_gated_delta_rule_fwd_h`` stores the running state of sequence
    ``n`` into ``h[chunk_offsets[n] + i]`` before it applies chunk ``i``
    (PRE:1153-1160), starting from the initial state (zeros if ``None``);
    ``chunk_offsets`` counts the chunks of the earlier sequences (PRE:172-209).
    The states come from the token recurrence of :func:`prefill_recurrent`.
    """
    T, HQ, HV, D, N = _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens)
    ld, beta = prefill_log_decay_beta(a, b, A_log, dt_bias, dtype)
    kh = _expand_heads(k.to(dtype), HV)
    vh = v.to(dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    hs = []
    for n in range(N):
        S = torch.zeros(HV, D, D, dtype=dtype) if state is None else state[n].to(dtype).clone()
        for t in range(cu[n], cu[n + 1]):
            if (t - cu[n]) % chunk_size == 0:
                hs.append(S.clone())
            S = torch.exp(ld[t])[:, None, None] * S
            sk = torch.einsum("hvk,hk->hv", S, kh[t])
            S = S + (beta[t][:, None] * (vh[t] - sk))[:, :, None] * kh[t][:, None, :]
    if not hs:
        return torch.zeros(0, HV, D, D, dtype=dtype)
    return torch.stack(hs)


def _round_bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(x.dtype)


def prefill_chunked(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None,
                    chunk_size: int = 64, dtype=torch.float64,
                    reference_storage: bool = False):
    """Chunked (WY / UT transform) GDN prefill, the reference's algorithm.

    Per sequence and per chunk of ``C`` tokens (ragged tail allowed), with
    ``gam`` the chunk-local cumsum of the log-decay (PRE:1721) and ``S`` the
    state at chunk start (``[HV, V, K]``):

    1. ``A_ij = beta_i e^{gam_i - gam_j} k_i . k_j`` for ``i > j`` (PRE:509-525)
    2. ``Tm = (I + A)^-1`` (PRE:661-737)
    3. ``U = Tm diag(beta) V``, ``W = Tm diag(beta e^gam) K`` (PRE:739-796)
    4. ``Vn = U - W S^T`` (PRE:1179-1211)
    5. ``O = scale [e^gam (Q S^T) + tril_incl(Q K^T e^{gam_i-gam_j}) Vn]`` (PRE:1447-1496)
    6. ``S <- e^{gam_L} S + (e^{gam_L - gam} Vn)^T K`` (PRE:1213-1225, 1286-1314)

    ``reference_storage=True`` additionally rounds to bf16 where the
    reference stores or casts bf16: ``W``, ``U`` (PRE:1002-1003), the chunk
    state used by steps 4-5 (PRE:1159, 1182, 1365), ``Vn`` (PRE:1368) and the
    intra-chunk attention weights before their product with ``Vn``
    (PRE:1494).  It is used to measure the reference's own rounding error,
    not as a parity target.
    """
    T, HQ, HV, D, N = _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens)
    scale = default_scale(scale, D)
    C = int(chunk_size)
    ld, beta = prefill_log_decay_beta(a, b, A_log, dtype=dtype, dt_bias=dt_bias)
    qh = _expand_heads(q.to(dtype), HV)
    kh = _expand_heads(k.to(dtype), HV)
    vh = v.to(dtype)
    rnd = _round_bf16 if reference_storage else (lambda x: x)
    o = torch.zeros(T, HV, D, dtype=dtype)
    final = torch.zeros(N, HV, D, D, dtype=dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    for n in range(N):
        S = torch.zeros(HV, D, D, dtype=dtype) if state is None else state[n].to(dtype).clone()
        for s in range(cu[n], cu[n + 1], C):
            e = min(s + C, cu[n + 1])
            L = e - s
            gam = torch.cumsum(ld[s:e], dim=0).transpose(0, 1)          # [HV, L]
            bet = beta[s:e].transpose(0, 1)                             # [HV, L]
            Kc = kh[s:e].transpose(0, 1)                                # [HV, L, D]
            Qc = qh[s:e].transpose(0, 1)
            Vc = vh[s:e].transpose(0, 1)
            dec = torch.exp(gam[:, :, None] - gam[:, None, :])          # [HV, L, L]
            strict = torch.tril(torch.ones(L, L, dtype=torch.bool), diagonal=-1)
            incl = torch.tril(torch.ones(L, L, dtype=torch.bool), diagonal=0)
            A = torch.where(strict, bet[:, :, None] * dec * (Kc @ Kc.transpose(1, 2)),
                            torch.zeros((), dtype=dtype))
            eye = torch.eye(L, dtype=dtype).expand(HV, L, L)
            Tm = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
            U = rnd(Tm @ (bet[:, :, None] * Vc))
            W = rnd(Tm @ ((bet * torch.exp(gam))[:, :, None] * Kc))
            Sx = rnd(S)
            Vn = U - W @ Sx.transpose(1, 2)                             # [HV, L, V]
            P = torch.where(incl, (Qc @ Kc.transpose(1, 2)) * dec, torch.zeros((), dtype=dtype))
            Oc = torch.exp(gam)[:, :, None] * (Qc @ Sx.transpose(1, 2)) + rnd(P) @ rnd(Vn)
            o[s:e] = (scale * Oc).transpose(0, 1)
            gl = gam[:, L - 1]                                          # [HV]
            Vd = torch.exp(gl[:, None] - gam)[:, :, None] * Vn          # [HV, L, V]
            S = torch.exp(gl)[:, None, None] * S + rnd(Vd).transpose(1, 2) @ Kc
        final[n] = S
    return o, final


# ---------------------------------------------------------------------------
# Backward of the prefill (no reference counterpart: the reference is
# forward-only, PRE:1).  Gradients of a loss L(o, final_state) with respect to
# q, k, v, the per-token log-decay g and beta, and the initial state, given
# dL/do and dL/d(final_state); then through the gating to a, b, A_log and
# dt_bias.


def prefill_backward(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, d_out, d_final=None,
                     dtype=torch.float64):
    """Per-token reverse recurrence of :func:`prefill_recurrent`.

    Forward per token (v-head h, state ``S [V, K]``)::

        S' = e^{g_t} S_{t-1};  u = beta_t (v_t - S' k_t);  S_t = S' + u k_t^T;  o_t = scale S_t q_t

    Reverse, with ``dS`` the gradient of ``S_t`` (``d_final`` after the last
    token of a sequence, zeros if ``None``)::

        dS += scale do_t q_t^T;        dq_t = scale S_t^T do_t
        du  = dS k_t;                  dk_t = dS^T u
        dbeta_t = du . (v_t - S' k_t); dv_t = beta_t du
        dS' = dS - beta_t du k_t^T;    dk_t -= beta_t S'^T du
        dg_t = <dS', S'>;              dS_{t-1} = e^{g_t} dS'

    ``dq`` / ``dk`` are summed over the v-heads that share a qk-head.  Returns
    a dict with ``dq, dk [T, HQ, D]``, ``dv [T, HV, D]``, ``dg, dbeta [T, HV]``
    and ``dh0 [N, HV, V, K]``.  The states ``S_t`` are recomputed forward
    from checkpoints at every 64th token.
    """
    T, HQ, HV, D, N = _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens)
    scale = default_scale(scale, D)
    G = HV // HQ
    ld, beta = prefill_log_decay_beta(a, b, A_log, dt_bias, dtype)
    qh = _expand_heads(q.to(dtype), HV)
    kh = _expand_heads(k.to(dtype), HV)
    vh = v.to(dtype)
    do = d_out.to(dtype)
    dq = torch.zeros(T, HV, D, dtype=dtype)
    dk = torch.zeros(T, HV, D, dtype=dtype)
    dv = torch.zeros(T, HV, D, dtype=dtype)
    dg = torch.zeros(T, HV, dtype=dtype)
    db = torch.zeros(T, HV, dtype=dtype)
    dh0 = torch.zeros(N, HV, D, D, dtype=dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    bl = 64

    def step(S, t):
        Sp = torch.exp(ld[t])[:, None, None] * S
        sk = torch.einsum("hvk,hk->hv", Sp, kh[t])
        u = beta[t][:, None] * (vh[t] - sk)
        return Sp, sk, u, Sp + u[:, :, None] * kh[t][:, None, :]

    for n in range(N):
        bos, eos = cu[n], cu[n + 1]
        S = torch.zeros(HV, D, D, dtype=dtype) if state is None else state[n].to(dtype).clone()
        ckpt = {}
        for t in range(bos, eos):
            if (t - bos) % bl == 0:
                ckpt[t] = S.clone()
            S = step(S, t)[3]
        dS = torch.zeros(HV, D, D, dtype=dtype) if d_final is None else d_final[n].to(dtype).clone()
        for blk in sorted(ckpt, reverse=True):
            S = ckpt[blk]
            rec = []
            for t in range(blk, min(blk + bl, eos)):
                Sp, sk, u, S = step(S, t)
                rec.append((t, Sp, sk, u, S))
            for t, Sp, sk, u, St in reversed(rec):
                dS = dS + scale * do[t][:, :, None] * qh[t][:, None, :]
                dq[t] = scale * torch.einsum("hvk,hv->hk", St, do[t])
                du = torch.einsum("hvk,hk->hv", dS, kh[t])
                dk[t] = torch.einsum("hvk,hv->hk", dS, u)
                db[t] = (du * (vh[t] - sk)).sum(-1)
                dv[t] = beta[t][:, None] * du
                dsk = -beta[t][:, None] * du
                dS = dS + dsk[:, :, None] * kh[t][:, None, :]
                dk[t] += torch.einsum("hvk,hv->hk", Sp, dsk)
                dg[t] = (dS * Sp).sum((-1, -2))
                dS = torch.exp(ld[t])[:, None, None] * dS
        dh0[n] = dS
    dq = dq.view(T, HQ, G, D).sum(2)
    dk = dk.view(T, HQ, G, D).sum(2)
    return {"dq": dq, "dk": dk, "dv": dv, "dg": dg, "dbeta": db, "dh0": dh0}


def prefill_backward_chunked(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, d_out,
                             d_final=None, h=None, chunk_size: int = 64, dtype=torch.float64):
    """Chunked backward: the algorithm of the HIP backward, in ``dtype``.

    Per chunk (``gam`` chunk-local cumsum of g, ``E = e^gam``,
    ``Dc = e^{gam_L - gam}``, ``S`` the state entering the chunk -- ``h``
    from :func:`prefill_chunk_states` when not given -- and ``dSn`` the
    gradient of the state leaving it), with the forward quantities
    ``Ar = tril_strict(e^{gam_i-gam_j} K K^T)``, ``A = diag(beta) Ar``,
    ``Tm = (I + A)^-1``, ``P = scale tril_incl(e^{gam_i-gam_j} Q K^T)``,
    ``Xr = V - E K S^T``, ``X = beta Xr``, ``Vn = Tm X``:

    1. the state-gradient chain, one product per chunk::

           W2 = Tm^T Dc K;  M = e^{gam_L} I - W2^T (beta E K)
           G1 = Tm^T P^T dO;  R = dO^T (scale E Q) - G1^T (beta E K)
           dS_prev = dSn M + R

    2. per chunk, given ``S`` and ``dSn``::

           dVn = P^T dO + Dc K dSn^T;  dX = Tm^T dVn;  dV = beta dX
           dP = dO Vn^T;  dTm = dVn X^T;  dA = -Tm^T dTm Tm^T (strictly lower)
           dQ = scale E dO S + (scale e^{gam_i-gam_j} dP)_incl K
           dK = Dc Vn dSn - beta E dX S + (...)_incl^T Q + dAb K + dAb^T K,
                dAb = beta_i e^{gam_i-gam_j} dA
           dbeta = rowsum(dA * Ar) + rowsum(dX * Xr)
           dgam  = rowsum - colsum of (dP * P) and of (dA * A)
                   + scale E rowsum(Q * (dO S)) - beta E rowsum(dX * K S^T)
                   - Dc rowsum(Vn * K dSn^T);  dgam_L += sum(Dc rowsum(Vn * K dSn^T)) + e^{gam_L} <dSn, S>
           dg = reverse cumsum of dgam over the chunk

    Pinned equal to :func:`prefill_backward` in float64.
    """
    T, HQ, HV, D, N = _check_prefill_shapes(q, k, v, state, a, b, cu_seqlens)
    scale = default_scale(scale, D)
    G = HV // HQ
    C = int(chunk_size)
    if h is None:
        h = prefill_chunk_states(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, C, dtype)
    ld, beta = prefill_log_decay_beta(a, b, A_log, dt_bias, dtype)
    qh = _expand_heads(q.to(dtype), HV)
    kh = _expand_heads(k.to(dtype), HV)
    vh = v.to(dtype)
    do = d_out.to(dtype)
    out = {n: torch.zeros(T, HV, D, dtype=dtype) for n in ("dq", "dk", "dv")}
    dg = torch.zeros(T, HV, dtype=dtype)
    db = torch.zeros(T, HV, dtype=dtype)
    dh0 = torch.zeros(N, HV, D, D, dtype=dtype)
    cu = [int(x) for x in cu_seqlens.tolist()]
    slot = 0
    for n in range(N):
        starts = list(range(cu[n], cu[n + 1], C))
        chunks = []
        for i, s in enumerate(starts):
            e = min(s + C, cu[n + 1])
            L = e - s
            gam = torch.cumsum(ld[s:e], 0).transpose(0, 1)                 # [HV, L]
            bet = beta[s:e].transpose(0, 1)
            E = torch.exp(gam)
            Dc = torch.exp(gam[:, L - 1:L] - gam)
            Kc, Qc = kh[s:e].transpose(0, 1), qh[s:e].transpose(0, 1)       # [HV, L, D]
            Vc, dOc = vh[s:e].transpose(0, 1), do[s:e].transpose(0, 1)
            dec = torch.exp(gam[:, :, None] - gam[:, None, :])
            strict = torch.tril(torch.ones(L, L, dtype=torch.bool), -1)
            incl = torch.tril(torch.ones(L, L, dtype=torch.bool), 0)
            zero = torch.zeros((), dtype=dtype)
            Ar = torch.where(strict, dec * (Kc @ Kc.transpose(1, 2)), zero)
            A = bet[:, :, None] * Ar
            eye = torch.eye(L, dtype=dtype).expand(HV, L, L)
            Tm = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
            P = scale * torch.where(incl, dec * (Qc @ Kc.transpose(1, 2)), zero)
            BEK = (bet * E)[:, :, None] * Kc
            W2 = Tm.transpose(1, 2) @ (Dc[:, :, None] * Kc)
            M = torch.exp(gam[:, L - 1])[:, None, None] * torch.eye(D, dtype=dtype) \
                - W2.transpose(1, 2) @ BEK
            G1 = Tm.transpose(1, 2) @ (P.transpose(1, 2) @ dOc)
            R = dOc.transpose(1, 2) @ ((scale * E)[:, :, None] * Qc) - G1.transpose(1, 2) @ BEK
            chunks.append(dict(s=s, e=e, L=L, gam=gam, bet=bet, E=E, Dc=Dc, Kc=Kc, Qc=Qc, Vc=Vc,
                               dOc=dOc, Ar=Ar, A=A, Tm=Tm, P=P, M=M, R=R, incl=incl, strict=strict,
                               dec=dec, S=h[slot + i].to(dtype)))
        dS = torch.zeros(HV, D, D, dtype=dtype) if d_final is None else d_final[n].to(dtype).clone()
        for c in reversed(chunks):
            c["dSn"] = dS
            dS = dS @ c["M"] + c["R"]
        dh0[n] = dS
        slot += len(starts)
        for c in chunks:
            s, e, L = c["s"], c["e"], c["L"]
            S, dSn, Tm, P, Kc, Qc = c["S"], c["dSn"], c["Tm"], c["P"], c["Kc"], c["Qc"]
            bet, E, Dc, dOc, gam = c["bet"], c["E"], c["Dc"], c["dOc"], c["gam"]
            KS = Kc @ S.transpose(1, 2)
            Xr = c["Vc"] - E[:, :, None] * KS
            X = bet[:, :, None] * Xr
            Vn = Tm @ X
            KdS = Kc @ dSn.transpose(1, 2)
            dVn = P.transpose(1, 2) @ dOc + Dc[:, :, None] * KdS
            dX = Tm.transpose(1, 2) @ dVn
            dP = torch.where(c["incl"], dOc @ Vn.transpose(1, 2), torch.zeros((), dtype=dtype))
            dTm = dVn @ X.transpose(1, 2)
            dA = torch.where(c["strict"], -(Tm.transpose(1, 2) @ dTm @ Tm.transpose(1, 2)),
                             torch.zeros((), dtype=dtype))
            dPm = scale * c["dec"] * dP
            dAb = bet[:, :, None] * c["dec"] * dA
            dOS = dOc @ S
            dQ = scale * E[:, :, None] * dOS + dPm @ Kc
            dK = Dc[:, :, None] * (Vn @ dSn) - (bet * E)[:, :, None] * (dX @ S) \
                + dPm.transpose(1, 2) @ Qc + dAb @ Kc + dAb.transpose(1, 2) @ Kc
            dbet = (dA * c["Ar"]).sum(-1) + (dX * Xr).sum(-1)
            pp = dP * P
            aa = dA * c["A"]
            vk = Dc * (Vn * KdS).sum(-1)
            dgam = pp.sum(-1) - pp.sum(-2) + aa.sum(-1) - aa.sum(-2) \
                + scale * E * (Qc * dOS).sum(-1) - bet * E * (dX * KS).sum(-1) - vk
            dgam[:, L - 1] += vk.sum(-1) + torch.exp(gam[:, L - 1]) * (dSn * S).sum((-1, -2))
            dgc = torch.flip(torch.cumsum(torch.flip(dgam, [1]), 1), [1])
            out["dq"][s:e] = dQ.transpose(0, 1)
            out["dk"][s:e] = dK.transpose(0, 1)
            out["dv"][s:e] = (bet[:, :, None] * dX).transpose(0, 1)
            dg[s:e] = dgc.transpose(0, 1)
            db[s:e] = dbet.transpose(0, 1)
    dq = out["dq"].view(T, HQ, G, D).sum(2)
    dk = out["dk"].view(T, HQ, G, D).sum(2)
    return {"dq": dq, "dk": dk, "dv": out["dv"], "dg": dg, "dbeta": db, "dh0": dh0}


def gate_backward(A_log, a, dt_bias, b, dg, dbeta, dtype=torch.float64):
    """Gradients of the prefill gating (PRE:1706-1722) given dL/dg and dL/dbeta.

    ``g = -exp(A_log) softplus(x)``, ``x = a + dt_bias``, ``beta = sigmoid(b)``:
    ``da = dg (-exp(A_log) sigmoid(x))``, ``ddt_bias = sum_t da``,
    ``dA_log = sum_t dg g``, ``db = dbeta beta (1 - beta)``.
    """
    A_log = A_log.to(dtype)
    x = a.to(dtype) + dt_bias.to(dtype)[None, :]
    g = -torch.exp(A_log)[None, :] * softplus_stable(x)
    da = dg.to(dtype) * (-torch.exp(A_log)[None, :] * torch.sigmoid(x))
    beta = torch.sigmoid(b.to(dtype))
    db = dbeta.to(dtype) * beta * (1.0 - beta)
    return {"da": da, "db": db, "dA_log": (dg.to(dtype) * g).sum(0), "ddt_bias": da.sum(0)}


# ---------------------------------------------------------------------------
# Short causal convolution ahead of GDN (no reference counterpart).  In a
# Qwen3-Next-style layer the q, k, v projections, concatenated channel-wise
# (mixed_qkv), pass through a depthwise causal conv1d of kernel size W (4)
# and SiLU before they become GDN's q, k, v; decode keeps the last inputs of
# every sequence as a conv state.


def _silu(y):
    return y * torch.sigmoid(y)


def causal_conv1d(x, weight, bias, cu_seqlens, conv_state=None, activation: Optional[str] = "silu",
                  state_len: Optional[int] = None, dtype=torch.float64):
    """Depthwise causal conv1d over packed varlen sequences.

    ``x [T, C]`` (token-major), ``weight [C, W]``, ``bias [C]`` or ``None``,
    ``cu_seqlens [N+1]``, ``conv_state [N, C, S]`` (S >= W - 1; the inputs
    that preceded each sequence, oldest first) or ``None`` for zeros.  For a
    sequence with history ``h = [state, x_bos .. x_eos-1]`` (index S + i for
    token bos + i):

        y[bos + i, c] = act(bias[c] + sum_w weight[c, w] h[S + i - (W - 1) + w, c])

    Returns ``(y [T, C], final_state [N, C, S])``, the final state being the
    last S entries of h.
    """
    T, C = x.shape
    W = weight.shape[1]
    N = cu_seqlens.numel() - 1
    S = state_len if state_len is not None else (conv_state.shape[2] if conv_state is not None else W - 1)
    assert S >= W - 1
    xf = x.to(dtype)
    wf = weight.to(dtype)
    y = torch.zeros(T, C, dtype=dtype)
    final = torch.zeros(N, C, S, dtype=dtype)
    for n in range(N):
        bos, eos = int(cu_seqlens[n]), int(cu_seqlens[n + 1])
        st = conv_state[n].to(dtype) if conv_state is not None else torch.zeros(C, S, dtype=dtype)
        h = torch.cat([st, xf[bos:eos].T], dim=1)                   # [C, S + L]
        L = eos - bos
        for i in range(L):
            win = h[:, S + i - (W - 1): S + i + 1]                  # [C, W]
            y[bos + i] = (win * wf).sum(dim=1)
        final[n] = h[:, -S:]
    if bias is not None:
        y = y + bias.to(dtype)[None, :]
    if activation == "silu":
        y = _silu(y)
    else:
        assert activation is None
    return y, final


def causal_conv1d_update(x, conv_state, weight, bias, activation: Optional[str] = "silu",
                         dtype=torch.float64):
    """One decode token per sequence: ``x [B, C]``, ``conv_state [B, C, S]``.
    Returns ``(y [B, C], new_state [B, C, S])`` (the state shifted by one,
    x appended), the same as :func:`causal_conv1d` on length-1 sequences."""
    B = x.shape[0]
    cu = torch.arange(B + 1, dtype=torch.int64)
    return causal_conv1d(x, weight, bias, cu, conv_state, activation, dtype=dtype)
