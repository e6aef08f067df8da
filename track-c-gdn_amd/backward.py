"""Backward of the GDN chunked prefill on the GPU, and an autograd operator.

The reference prefill is forward-only (PRE:1, ``gdn_prefill_qk4_v8_d128_k_last/
solution/triton/kernel.py``).  A training step needs the gradients of its
inputs; they are computed from ``h``, the state entering every 64-token
chunk, which the forward writes on request (``prefill.gdn_prefill_h``, the h
of the reference's ``chunk_gated_delta_rule_fwd_h``, PRE:1341-1398).

* :func:`gdn_prefill_backward` -- ``dq, dk, dv`` (fp32), ``dg, dbeta`` (per
  token and v-head: the gradients of the log-decay ``g`` and of ``beta``) and
  the gradient of the initial state, given ``d_out`` and optionally the
  gradient of the final state.
* :func:`gdn_gate_backward` -- ``dg, dbeta`` through the gating to the raw
  inputs ``a, b, A_log, dt_bias`` (``g = -exp(A_log) softplus(a + dt_bias)``,
  ``beta = sigmoid(b)``, PRE:1706-1722).
* :func:`chunk_gated_delta_rule` -- the prefill as a differentiable torch
  operator (forward with ``h``, backward through the two calls above).

All arithmetic runs in the HIP kernels of libgdn_hip.so on torch's current
stream.  The backward's products take bf16 operands with fp32 accumulation;
``h`` is the forward's bf16 copy of the chunk states.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _capi
from . import prefill as _pre

HEAD_SIZE = 128


def workspace_bytes(N: int, T: int, HQ: int, HV: int) -> int:
    """Device workspace of :func:`gdn_prefill_backward`: per chunk slot and
    v-head the chunk's state-gradient transition (M and R, 32 KiB bf16 each)
    and the gradient of the state leaving it (32 KiB bf16)."""
    return int(_capi.lib().gdn_prefill_bwd_workspace_bytes(N, T, HQ, HV))


@torch.no_grad()
def gdn_prefill_backward(q, k, v, A_log, a, dt_bias, b, cu_seqlens, scale, h, d_out,
                         d_final_state=None, *, need_initial_state_grad: bool = True,
                         workspace=None):
    """Gradients of the prefill's inputs.

    Inputs as for ``prefill.gdn_prefill`` (``q, k [T, HQ, 128]``, ``v [T, HV,
    128]``, ``a, b [T, HV]`` bf16; ``A_log, dt_bias [HV]`` fp32;
    ``cu_seqlens [N + 1]`` int64 / int32), ``h`` from
    ``prefill.gdn_prefill_h`` on the same inputs, ``d_out [T, HV, 128]``
    (cast to bf16) and ``d_final_state [N, HV, 128, 128]`` fp32 or ``None``
    (zero).  Returns a dict of fp32 tensors: ``dq, dk [T, HQ, 128]``,
    ``dv [T, HV, 128]``, ``dg, dbeta [T, HV]`` and ``dh0 [N, HV, 128, 128]``
    (``None`` unless ``need_initial_state_grad``).
    """
    T, HQ, d = q.shape
    HV = v.shape[1]
    N = cu_seqlens.numel() - 1
    assert d == HEAD_SIZE and HV % HQ == 0
    assert q.is_cuda and k.is_cuda and v.is_cuda and h.is_cuda and d_out.is_cuda
    assert h.dtype == torch.bfloat16 and h.dim() == 4 and h.shape[1:] == (HV, HEAD_SIZE, HEAD_SIZE)
    assert cu_seqlens.dtype in (torch.int64, torch.int32)
    assert d_out.shape == (T, HV, HEAD_SIZE)
    assert h.shape[0] >= _pre.num_chunks(cu_seqlens, T), "h holds fewer chunks than the batch has"
    dev = q.device
    scale = _pre._resolve_scale(scale)
    q, k, v, a, b = (t.to(torch.bfloat16).contiguous() for t in (q, k, v, a, b))
    A_log = A_log.to(torch.float32).contiguous()
    dt_bias = dt_bias.to(torch.float32).contiguous()
    cu = cu_seqlens.contiguous()
    h = h.contiguous()
    d_out = d_out.to(torch.bfloat16).contiguous()
    dfin = None
    if d_final_state is not None:
        assert d_final_state.shape == (N, HV, HEAD_SIZE, HEAD_SIZE)
        dfin = d_final_state.to(torch.float32).contiguous()
    out = {
        "dq": torch.empty(T, HQ, HEAD_SIZE, dtype=torch.float32, device=dev),
        "dk": torch.empty(T, HQ, HEAD_SIZE, dtype=torch.float32, device=dev),
        "dv": torch.empty(T, HV, HEAD_SIZE, dtype=torch.float32, device=dev),
        "dg": torch.empty(T, HV, dtype=torch.float32, device=dev),
        "dbeta": torch.empty(T, HV, dtype=torch.float32, device=dev),
        "dh0": (torch.empty(N, HV, HEAD_SIZE, HEAD_SIZE, dtype=torch.float32, device=dev)
                if need_initial_state_grad else None),
    }
    need = workspace_bytes(N, T, HQ, HV)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    p = _capi.ptr
    rc = _capi.lib().gdn_prefill_bwd(
        p(q), p(k), p(v), p(A_log), p(a), p(dt_bias), p(b), p(cu),
        1 if cu.dtype == torch.int32 else 0, N, T, HQ, HV, float(scale), p(h), h.shape[0],
        p(d_out), p(dfin), p(out["dq"]), p(out["dk"]), p(out["dv"]), p(out["dg"]),
        p(out["dbeta"]), p(out["dh0"]), p(workspace), workspace.numel() * workspace.element_size(),
        _capi.stream_handle(dev))
    _capi.check(rc, "gdn_prefill_bwd")
    return out


@torch.no_grad()
def gdn_gate_backward(A_log, a, dt_bias, b, dg, dbeta):
    """``dg, dbeta [T, HV]`` -> ``da, db [T, HV]``, ``dA_log, ddt_bias [HV]`` (fp32)."""
    T, HV = a.shape
    dev = a.device
    A_log = A_log.to(torch.float32).contiguous()
    dt_bias = dt_bias.to(torch.float32).contiguous()
    a = a.to(torch.bfloat16).contiguous()
    b = b.to(torch.bfloat16).contiguous()
    dg = dg.to(torch.float32).contiguous()
    dbeta = dbeta.to(torch.float32).contiguous()
    out = {"da": torch.empty(T, HV, dtype=torch.float32, device=dev),
           "db": torch.empty(T, HV, dtype=torch.float32, device=dev),
           "dA_log": torch.empty(HV, dtype=torch.float32, device=dev),
           "ddt_bias": torch.empty(HV, dtype=torch.float32, device=dev)}
    p = _capi.ptr
    rc = _capi.lib().gdn_gate_bwd(p(A_log), p(a), p(dt_bias), p(b), p(dg), p(dbeta), T, HV,
                                  p(out["da"]), p(out["db"]), p(out["dA_log"]),
                                  p(out["ddt_bias"]), _capi.stream_handle(dev))
    _capi.check(rc, "gdn_gate_bwd")
    return out


class _GatedDeltaRule(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, A_log, a, dt_bias, b, initial_state, cu_seqlens, scale):
        o, final, h = _pre.gdn_prefill_h(q, k, v, initial_state, A_log, a, dt_bias, b,
                                         cu_seqlens, scale)
        ctx.save_for_backward(q, k, v, A_log, a, dt_bias, b, cu_seqlens, h)
        ctx.scale = scale
        ctx.has_state = initial_state is not None
        ctx.dtypes = (q.dtype, k.dtype, v.dtype, A_log.dtype, a.dtype, dt_bias.dtype, b.dtype,
                      None if initial_state is None else initial_state.dtype)
        return o, final

    @staticmethod
    def backward(ctx, d_o, d_final):
        q, k, v, A_log, a, dt_bias, b, cu_seqlens, h = ctx.saved_tensors
        if d_o is None:
            d_o = torch.zeros(v.shape, dtype=torch.bfloat16, device=v.device)
        g = gdn_prefill_backward(q, k, v, A_log, a, dt_bias, b, cu_seqlens, ctx.scale, h, d_o,
                                 d_final, need_initial_state_grad=ctx.has_state)
        gg = gdn_gate_backward(A_log, a, dt_bias, b, g["dg"], g["dbeta"])
        tq, tk, tv, tA, ta, tdt, tb, ts = ctx.dtypes
        ds = g["dh0"].to(ts) if ctx.has_state else None
        return (g["dq"].to(tq), g["dk"].to(tk), g["dv"].to(tv), gg["dA_log"].to(tA),
                gg["da"].to(ta), gg["ddt_bias"].to(tdt), gg["db"].to(tb), ds, None, None)


def chunk_gated_delta_rule(q, k, v, A_log, a, dt_bias, b, cu_seqlens, initial_state=None,
                           scale: Optional[float] = None):
    """Differentiable GDN prefill: ``(output [T, HV, 128] bf16, final_state
    [N, HV, 128, 128] fp32)`` with gradients for q, k, v, A_log, a, dt_bias,
    b and the initial state.  The forward keeps ``h`` (bf16, 32 KiB per
    chunk and v-head) for the backward."""
    return _GatedDeltaRule.apply(q, k, v, A_log, a, dt_bias, b, initial_state, cu_seqlens, scale)
