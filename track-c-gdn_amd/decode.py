"""GDN decode operator: one recurrent step per sequence on the GPU.

Host-side mirror of the reference decode entry point
``gdn_decode_qk4_v8_d128_k_last/solution/triton/kernel.py`` (DEC):

* :func:`run` -- same positional signature, defaults, asserts and return
  tuple as ``run`` at DEC:100-146 (value-returning, qk4/v8/d128).
* :func:`run_dps` -- destination-passing variant: ``output`` and
  ``new_state`` are appended as trailing parameters and written in place.
* :func:`gdn_decode` -- the same step for any head layout with
  ``HV % HQ == 0`` (e.g. 16 qk-heads / 32 v-heads).
* :func:`decode_pool_` -- in-place step against a slot-indexed state pool.
* :func:`gdn_decode_multi` -- T consecutive steps per sequence in one launch
  (multi-token / speculative decode; the reference accepts one token per
  call, DEC:117-119).

All compute runs in the HIP kernel of libgdn_hip.so on torch's current
stream; there is no CPU path.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _capi

HQ = 4
HV = 8
D = 128


def _resolve_scale(scale, head_dim: int) -> float:
    # DEC:112-115
    if scale is None or float(scale) == 0.0:
        return 1.0 / math.sqrt(head_dim)
    return float(scale)


def _check_common(q, k, v, A_log, a, dt_bias, b):
    assert q.is_cuda and k.is_cuda and v.is_cuda, "decode inputs must be GPU tensors"
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
    assert a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
    B, T1, nq, d = q.shape
    assert T1 == 1 and d == D
    assert k.shape == q.shape
    assert v.dim() == 4 and v.shape[0] == B and v.shape[1] == 1 and v.shape[3] == D
    nv = v.shape[2]
    assert nv % nq == 0, "v-heads must be a multiple of qk-heads"
    assert A_log.numel() == nv and dt_bias.numel() == nv
    assert a.numel() == B * nv and b.numel() == B * nv
    return B, nq, nv


def _gates(A_log, dt_bias):
    # DEC:131-133 (A_log.float(), dt_bias.float())
    return A_log.float().contiguous(), dt_bias.float().contiguous()


def _launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, nq, nv,
            flags=0):
    A_log, dt_bias = _gates(A_log, dt_bias)
    q = q.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    a = a.contiguous()
    b = b.contiguous()
    rc = _capi.lib().gdn_decode_ex_fwd(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(new_state),
        _capi.ptr(A_log), _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(output),
        B, nq, nv, float(scale), flags, _capi.stream_handle(q.device))
    _capi.check(rc, "gdn_decode_ex_fwd")


@torch.no_grad()
def gdn_decode(q, k, v, state, A_log, a, dt_bias, b, scale=None, *, output=None,
               new_state=None, qk_l2norm: bool = False):
    """One decode step for any ``HV % HQ == 0`` head layout.

    ``q, k [B, 1, HQ, 128]``, ``v [B, 1, HV, 128]`` bf16; ``state
    [B, HV, 128, 128]`` fp32 or ``None``; ``a, b [B, 1, HV]`` bf16; ``A_log,
    dt_bias [HV]``.  Returns ``(output [B, 1, HV, 128] bf16, new_state)``.
    ``new_state`` may be the ``state`` tensor itself (in-place update).
    ``qk_l2norm=True`` uses q and k L2-normalised, ``x (sum x^2 + 1e-6)^-1/2``
    in fp32 inside the kernel (an option the reference does not have).
    """
    return _decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output=output,
                        new_state=new_state, qk_l2norm=qk_l2norm)


def _decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale=None, *, output=None,
                 new_state=None, qk_l2norm: bool = False):
    """:func:`gdn_decode` without its no-grad wrapper (the callers hold one)."""
    B, nq, nv = _check_common(q, k, v, A_log, a, dt_bias, b)
    scale = _resolve_scale(scale, q.shape[-1])
    if state is not None:
        assert state.is_cuda and state.dtype == torch.float32
        assert state.shape == (B, nv, D, D)
        if not state.is_contiguous():   # DEC:95-96
            state = state.contiguous()
    if output is None:
        output = torch.empty(B, 1, nv, D, dtype=q.dtype, device=q.device)
    if new_state is None:
        new_state = torch.empty(B, nv, D, D, dtype=torch.float32, device=q.device)
    assert output.dtype == torch.bfloat16 and output.is_contiguous() and output.numel() == B * nv * D
    assert new_state.dtype == torch.float32 and new_state.is_contiguous()
    assert new_state.shape == (B, nv, D, D)
    _launch(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, B, nq, nv,
            _capi.GDN_QK_L2NORM if qk_l2norm else 0)
    return output, new_state


@torch.no_grad()
def run(q, k, v, state, A_log, a, dt_bias, b, scale):
    """Reference-compatible decode entry (DEC:100-146), qk4 / v8 / d128.

    Returns ``(output [B, 1, 8, 128], new_state [B, 8, 128, 128] fp32)``;
    the input state is not modified.  As at DEC:122 the output has q's dtype.
    The reference kernel loads q, k, v, a and b of any float dtype; here
    fp16 / fp32 inputs are rounded to bf16 (the operator definition's dtype)
    before the kernel reads them.
    """
    assert q.shape[1:] == (1, HQ, D)    # DEC:117-120
    assert k.shape[1:] == (1, HQ, D)
    assert v.shape[1:] == (1, HV, D)
    assert q.shape[0] == v.shape[0]
    out_dtype = q.dtype
    assert out_dtype.is_floating_point
    q, k, v, a, b = (t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)
                     for t in (q, k, v, a, b))
    o, s = _decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale)
    return (o if out_dtype == torch.bfloat16 else o.to(out_dtype)), s


@torch.no_grad()
def run_dps(q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state):
    """Destination-passing decode: writes ``output`` and ``new_state``, returns None."""
    assert q.shape[1:] == (1, HQ, D)
    assert k.shape[1:] == (1, HQ, D)
    assert v.shape[1:] == (1, HV, D)
    assert q.shape[0] == v.shape[0]
    _decode_impl(q, k, v, state, A_log, a, dt_bias, b, scale, output=output, new_state=new_state)


@torch.no_grad()
def gdn_decode_multi(q, k, v, state, A_log, a, dt_bias, b, scale=None, *, output=None,
                     new_state=None, qk_l2norm: bool = False):
    """T decode steps per sequence, applied in token order, in one launch.

    ``q, k [B, T, HQ, 128]``, ``v [B, T, HV, 128]`` bf16; ``a, b [B, T, HV]``
    bf16; ``state [B, HV, 128, 128]`` fp32 or ``None``; ``A_log, dt_bias
    [HV]``.  Returns ``(output [B, T, HV, 128] bf16, new_state)``, equal bit
    for bit to T successive :func:`gdn_decode` calls; ``new_state`` may be the
    ``state`` tensor itself.
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda, "decode inputs must be GPU tensors"
    assert q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
    assert a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
    assert q.dim() == 4 and q.shape[3] == D and k.shape == q.shape
    B, T, nq, _ = q.shape
    assert T >= 1, "at least one token per sequence"
    assert v.dim() == 4 and v.shape[:2] == (B, T) and v.shape[3] == D
    nv = v.shape[2]
    assert nv % nq == 0, "v-heads must be a multiple of qk-heads"
    assert A_log.numel() == nv and dt_bias.numel() == nv
    assert a.numel() == B * T * nv and b.numel() == B * T * nv
    scale = _resolve_scale(scale, D)
    if state is not None:
        assert state.is_cuda and state.dtype == torch.float32 and state.shape == (B, nv, D, D)
        if not state.is_contiguous():
            state = state.contiguous()
    if output is None:
        output = torch.empty(B, T, nv, D, dtype=q.dtype, device=q.device)
    if new_state is None:
        new_state = torch.empty(B, nv, D, D, dtype=torch.float32, device=q.device)
    assert output.dtype == torch.bfloat16 and output.is_contiguous()
    assert output.numel() == B * T * nv * D
    assert new_state.dtype == torch.float32 and new_state.is_contiguous()
    assert new_state.shape == (B, nv, D, D)
    A_log, dt_bias = _gates(A_log, dt_bias)
    q, k, v, a, b = (t.contiguous() for t in (q, k, v, a, b))
    rc = _capi.lib().gdn_decode_multi_fwd(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(new_state),
        _capi.ptr(A_log), _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(output),
        B, T, nq, nv, float(scale), _capi.GDN_QK_L2NORM if qk_l2norm else 0,
        _capi.stream_handle(q.device))
    _capi.check(rc, "gdn_decode_multi_fwd")
    return output, new_state


@torch.no_grad()
def decode_pool_(q, k, v, state_pool, slot_ids, A_log, a, dt_bias, b, scale=None, *,
                 output=None, check_slots: bool = False):
    """One decode step against ``state_pool[slot_ids[n]]``, updated in place.

    ``state_pool [P, HV, 128, 128]`` fp32, ``slot_ids [B]`` int32 (distinct:
    two sequences naming one slot would update it concurrently, with a
    result that is not specified).  A slot outside ``[0, P)`` leaves the pool
    untouched and gives a zero output row.  ``check_slots=True`` checks the
    slots on the device before the launch (a sort and one synchronisation)
    and raises ``ValueError`` naming repeated slots inside the pool (slots
    outside it touch no state and may repeat), launching nothing.
    Returns ``output [B, 1, HV, 128]`` bf16.
    """
    B, nq, nv = _check_common(q, k, v, A_log, a, dt_bias, b)
    scale = _resolve_scale(scale, q.shape[-1])
    assert state_pool.is_cuda and state_pool.dtype == torch.float32 and state_pool.is_contiguous()
    assert state_pool.dim() == 4 and state_pool.shape[1:] == (nv, D, D)
    assert slot_ids.is_cuda and slot_ids.dtype == torch.int32 and slot_ids.numel() == B
    slot_ids = slot_ids.contiguous()
    if check_slots and B > 1:
        srt = torch.sort(slot_ids.flatten()).values
        rep = (srt[1:] == srt[:-1]) & (srt[1:] >= 0) & (srt[1:] < state_pool.shape[0])
        dup = srt[1:][rep].unique()
        if dup.numel():
            raise ValueError(f"slot_ids repeat slot(s) {dup[:16].tolist()}: each sequence "
                             "needs its own slot")
    if output is None:
        output = torch.empty(B, 1, nv, D, dtype=q.dtype, device=q.device)
    A_log, dt_bias = _gates(A_log, dt_bias)
    q, k, v, a, b = (t.contiguous() for t in (q, k, v, a, b))
    rc = _capi.lib().gdn_decode_pool_fwd(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state_pool), state_pool.shape[0],
        _capi.ptr(slot_ids), _capi.ptr(A_log), _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b),
        _capi.ptr(output), B, nq, nv, float(scale), _capi.stream_handle(q.device))
    _capi.check(rc, "gdn_decode_pool_fwd")
    return output


class PreparedDecode:
    """A decode step on fixed buffers, validated once and launched by one C call.

    For serving loops (and the benchmark) that step the same buffers
    repeatedly: arguments are checked and resolved to device pointers at
    construction, the stream is torch's current stream at that time, and
    ``__call__`` only enqueues the kernel.  ``new_state`` may be ``state``.
    ``qk_l2norm`` as for :func:`gdn_decode`.
    """

    def __init__(self, q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, *,
                 qk_l2norm: bool = False):
        B, nq, nv = _check_common(q, k, v, A_log, a, dt_bias, b)
        assert state is None or (state.is_contiguous() and state.dtype == torch.float32
                                 and state.shape == (B, nv, D, D))
        assert output.dtype == torch.bfloat16 and output.is_contiguous()
        assert output.numel() == B * nv * D
        assert new_state.dtype == torch.float32 and new_state.is_contiguous()
        assert new_state.shape == (B, nv, D, D)
        for t in (q, k, v, a, b):
            assert t.is_contiguous()
        A_log, dt_bias = _gates(A_log, dt_bias)
        self._keep = (q, k, v, state, A_log, a, dt_bias, b, output, new_state)
        self._fn = _capi.lib().gdn_decode_ex_fwd
        self._args = (
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(new_state),
            _capi.ptr(A_log), _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(output),
            B, nq, nv, float(_resolve_scale(scale, q.shape[-1])),
            _capi.GDN_QK_L2NORM if qk_l2norm else 0, _capi.stream_handle(q.device))

    def __call__(self) -> None:
        rc = self._fn(*self._args)
        if rc:
            _capi.check(rc, "gdn_decode_ex_fwd")


class PreparedDecodeMulti:
    """T decode steps per sequence on fixed buffers, launched by one C call.

    The multi-token counterpart of :class:`PreparedDecode` (same contract:
    validated once, ``__call__`` only enqueues the kernel).
    """

    def __init__(self, q, k, v, state, A_log, a, dt_bias, b, scale, output, new_state, *,
                 qk_l2norm: bool = False):
        assert q.dim() == 4 and q.shape[3] == D and k.shape == q.shape
        B, T, nq, _ = q.shape
        assert T >= 1 and v.dim() == 4 and v.shape[:2] == (B, T) and v.shape[3] == D
        nv = v.shape[2]
        assert nv % nq == 0 and a.numel() == B * T * nv and b.numel() == B * T * nv
        assert state is None or (state.is_contiguous() and state.dtype == torch.float32
                                 and state.shape == (B, nv, D, D))
        assert output.dtype == torch.bfloat16 and output.is_contiguous()
        assert output.numel() == B * T * nv * D
        assert new_state.dtype == torch.float32 and new_state.is_contiguous()
        assert new_state.shape == (B, nv, D, D)
        for t in (q, k, v, a, b):
            assert t.is_contiguous() and t.dtype == torch.bfloat16
        A_log, dt_bias = _gates(A_log, dt_bias)
        self._keep = (q, k, v, state, A_log, a, dt_bias, b, output, new_state)
        self._fn = _capi.lib().gdn_decode_multi_fwd
        self._args = (
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(new_state),
            _capi.ptr(A_log), _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(output),
            B, T, nq, nv, float(_resolve_scale(scale, D)), _capi.GDN_QK_L2NORM if qk_l2norm else 0,
            _capi.stream_handle(q.device))

    def __call__(self) -> None:
        rc = self._fn(*self._args)
        if rc:
            _capi.check(rc, "gdn_decode_multi_fwd")
