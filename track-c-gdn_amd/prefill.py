"""GDN chunked varlen prefill operator on the GPU.

Host-side mirror of the reference prefill entry point
``gdn_prefill_qk4_v8_d128_k_last/solution/triton/kernel.py`` (PRE):

* :func:`run` -- same positional signature, validation (``_validate_inputs``,
  PRE:1635-1667), scale default (PRE:1777-1778) and return tuple
  ``(output [T, 8, 128] bf16, final_state [N, 8, 128, 128] fp32)`` as
  PRE:1762-1802.  ``cu_seqlens`` may be int64 (as the reference asserts) or
  int32.
* :func:`run_dps` -- destination-passing variant (``output``,
  ``final_state`` appended).
* :func:`gdn_prefill` -- any ``HV % HQ == 0`` head layout, optional
  validation, caller-provided outputs.
* :func:`gdn_prefill_h` -- also returns ``h``, the state entering every
  64-token chunk (the h output of ``chunk_gated_delta_rule_fwd_h``,
  PRE:1341-1398).

All compute runs in the HIP kernels of libgdn_hip.so on torch's current
stream.
"""

from __future__ import annotations

import ctypes
import math
import weakref
from typing import Optional

import torch

from . import _capi

NUM_Q_HEADS = 4
NUM_K_HEADS = 4
NUM_V_HEADS = 8
HEAD_SIZE = 128
CHUNK_SIZE = 64


def _resolve_scale(scale) -> float:
    # PRE:1777-1778
    if scale is None or scale == 0.0:
        return 1.0 / math.sqrt(HEAD_SIZE)
    return float(scale)


# Host copies of cu_seqlens by tensor object: (weak reference, version, copy).
_CU_HOST = {}
# Path choices by (host copy, T, HV, device): (the host copy, slices per
# chain, 0 = fused); holding the copy keeps its id from being reused.
_CHOICE = {}
# Launch plans by (host copy, T, HQ, HV, flags, device): (the host copy, plan).
_PLANS = {}
# Split-path workspaces by (device, stream), reused by later calls on the
# same stream (stream order keeps them from overlapping).
_WORKSPACE = {}


def host_cu_seqlens(cu_seqlens: torch.Tensor) -> torch.Tensor:
    """``cu_seqlens`` in host memory: one device-to-host read per tensor object
    and version, kept while the tensor lives.  Torch advances a tensor's
    version on every in-place write made through torch, so a rewritten
    ``cu_seqlens`` is read again; a write that bypasses torch (a raw kernel
    on its storage) is not seen -- pass a new tensor then."""
    ent = _CU_HOST.get(id(cu_seqlens))
    if ent is not None and ent[0]() is cu_seqlens and ent[1] == cu_seqlens._version:
        return ent[2]
    host = cu_seqlens.detach().to("cpu").contiguous()
    if len(_CU_HOST) >= 64:
        for key in [key for key, e in _CU_HOST.items() if e[0]() is None]:
            del _CU_HOST[key]
        if len(_CU_HOST) >= 64:
            _CU_HOST.clear()
    _CU_HOST[id(cu_seqlens)] = (weakref.ref(cu_seqlens), cu_seqlens._version, host)
    return host


def _split_workspace(nbytes: int, device) -> torch.Tensor:
    key = (device.index, _capi.stream_handle(device))
    ws = _WORKSPACE.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACE[key] = ws
    return ws


def validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens,
                    num_q_heads: int = NUM_Q_HEADS, num_v_heads: int = NUM_V_HEADS,
                    check_total: bool = True) -> Optional[torch.Tensor]:
    """The checks of PRE:1635-1667, raising AssertionError before any launch.

    ``check_total`` keeps the reference's ``cu_seqlens[-1] == T`` check
    (PRE:1665) and returns the host copy of ``cu_seqlens`` it reads for it
    (one device-to-host copy per tensor and version, :func:`host_cu_seqlens`);
    else None.
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda
    assert A_log.is_cuda and a.is_cuda and dt_bias.is_cuda and b.is_cuda and cu_seqlens.is_cuda
    assert q.dtype == torch.bfloat16
    assert k.dtype == torch.bfloat16
    assert v.dtype == torch.bfloat16
    assert A_log.dtype == torch.float32
    assert dt_bias.dtype == torch.float32
    assert a.dtype == torch.bfloat16
    assert b.dtype == torch.bfloat16
    if state is not None:
        assert state.is_cuda and state.dtype == torch.float32
    assert q.shape[1:] == (num_q_heads, HEAD_SIZE)
    assert k.shape[1:] == (num_q_heads, HEAD_SIZE)
    assert v.shape[1:] == (num_v_heads, HEAD_SIZE)
    assert A_log.shape == (num_v_heads,)
    assert dt_bias.shape == (num_v_heads,)
    assert a.shape == (q.shape[0], num_v_heads)
    assert b.shape == (q.shape[0], num_v_heads)
    assert cu_seqlens.dtype in (torch.int64, torch.int32)
    assert cu_seqlens.dim() == 1 and cu_seqlens.numel() >= 1
    if state is not None:
        assert state.shape == (cu_seqlens.numel() - 1, num_v_heads, HEAD_SIZE, HEAD_SIZE)
    if check_total:
        cu_host = host_cu_seqlens(cu_seqlens)
        assert int(cu_host[-1]) == q.shape[0]
        return cu_host
    return None


def workspace_bytes(N: int, T: int, HQ: int, HV: int) -> int:
    """Workspace the automatic path selection uses for this problem on the
    current device (0 when the fused chain kernel runs)."""
    return int(_capi.lib().gdn_prefill_workspace_bytes(N, T, HQ, HV))


def auto_path(N: int, HV: int) -> str:
    """The kernels the library's automatic choice runs for N sequences of HV
    v-heads on the current device: ``"fused"`` or ``"split<slices>"``."""
    s = int(_capi.lib().gdn_prefill_auto_slices(N, HV))
    return f"split{s}" if s > 0 else "fused"


def choose_slices(cu_host: torch.Tensor, T: int, HV: int) -> int:
    """Path choice from the sequence lengths (``cu_host``: ``cu_seqlens`` in
    host memory): 8 or 4 state slices per chain (the split path) or 0 (the
    fused chain kernel), whichever the library's cost model of the launches
    on the current device finishes first (``gdn_prefill_choose_slices``)."""
    cu = cu_host.contiguous()
    assert not cu.is_cuda and cu.dtype in (torch.int64, torch.int32) and cu.dim() == 1
    s = int(_capi.lib().gdn_prefill_choose_slices(
        cu.data_ptr(), 1 if cu.dtype == torch.int32 else 0, cu.numel() - 1, int(T), int(HV), 0))
    assert s in (0, 4, 8), s
    return s


class Plan:
    """A prefill launch plan made on the host from the sequence lengths
    (``gdn_prefill_plan``): the path (``slices`` 4 / 8: the split path, 0:
    the fused kernel), the seams (the fused kernel's: ``seams`` sequences cut
    at chunk ``split_chunk``, ``periods`` the modelled finish in chunk
    periods; the split path's: ``seams`` slots its launch reserves, the cuts
    chosen on the device), the kernels a call launches and the device
    workspace :func:`gdn_prefill` needs with it."""

    __slots__ = ("buf", "slices", "seams", "split_chunk", "periods", "workspace_bytes")

    def __init__(self, cu_host: torch.Tensor, T: int, HQ: int, HV: int, *, seams: bool = True,
                 fused: bool = False, cus: int = 0):
        cu = cu_host.contiguous()
        assert not cu.is_cuda and cu.dtype in (torch.int64, torch.int32) and cu.dim() == 1
        lib = _capi.lib()
        self.buf = ctypes.create_string_buffer(_capi.GDN_PREFILL_PLAN_BYTES)
        ws = ctypes.c_size_t(0)
        flags = (0 if seams else _capi.GDN_NO_SEAMS) | (_capi.GDN_PLAN_FUSED if fused else 0)
        _capi.check(lib.gdn_prefill_plan(cu.data_ptr(), 1 if cu.dtype == torch.int32 else 0,
                                         cu.numel() - 1, int(T), int(HQ), int(HV), int(cus), flags,
                                         self.buf, ctypes.byref(ws)), "gdn_prefill_plan")
        info = [ctypes.c_int(0) for _ in range(4)]
        _capi.check(lib.gdn_prefill_plan_info(self.buf, *[ctypes.byref(i) for i in info]),
                    "gdn_prefill_plan_info")
        self.slices, self.seams, self.split_chunk, self.periods = (int(i.value) for i in info)
        self.workspace_bytes = int(ws.value)

    @property
    def path(self) -> str:
        if self.slices:
            return f"split{self.slices}"
        return f"fused+{self.seams}seams" if self.seams else "fused"

    @property
    def kernels(self) -> list:
        ks = (["gdn_prefill_prep_kernel", "gdn_prefill_slice_kernel"] if self.slices
              else ["gdn_prefill_chain_kernel"])
        return ks + (["gdn_prefill_seam_kernel"] if self.seams else [])


def _plan_for(cu_host: torch.Tensor, T: int, HQ: int, HV: int, seams: bool, fused: bool,
              device) -> Plan:
    """The plan of these lengths, made once per host copy of ``cu_seqlens``."""
    key = (id(cu_host), int(T), int(HQ), int(HV), bool(seams), bool(fused), device.index)
    ent = _PLANS.get(key)
    if ent is not None and ent[0] is cu_host:
        return ent[1]
    plan = Plan(cu_host, T, HQ, HV, seams=seams, fused=fused)
    if len(_PLANS) >= 256:
        _PLANS.clear()
    _PLANS[key] = (cu_host, plan)
    return plan


def split_workspace_bytes(N: int, T: int, HQ: int, HV: int) -> int:
    """Workspace of the split path (chunk preparation + state slices)."""
    return int(_capi.lib().gdn_prefill_split_workspace_bytes(N, T, HQ, HV))


def num_chunks(cu_seqlens: torch.Tensor, T: int) -> int:
    """64-token chunks of the batch, ``sum ceil(len_n / 64)`` (the chunk count
    of PRE:1358-1361): the first dimension of ``h``.  Reads ``cu_seqlens``
    on the host (a device-to-host copy when it lives on the GPU)."""
    cu = cu_seqlens.detach().to("cpu").contiguous()
    assert cu.dtype in (torch.int64, torch.int32) and cu.dim() == 1 and cu.numel() >= 1
    n = _capi.lib().gdn_prefill_chunk_count(cu.data_ptr(), 1 if cu.dtype == torch.int32 else 0,
                                            cu.numel() - 1, int(T))
    assert n >= 0
    return int(n)


@torch.no_grad()
def gdn_prefill(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None, *,
                output=None, final_state=None, workspace=None, validate: bool = True,
                qk_l2norm: bool = False, h=None, path: str = "auto", slices: int = 8,
                seams: bool = True, check_range: bool = False):
    """Chunked GDN prefill over packed varlen sequences, any ``HV % HQ == 0``.

    ``q, k [T, HQ, 128]``, ``v [T, HV, 128]``, ``a, b [T, HV]`` bf16;
    ``state [N, HV, 128, 128]`` fp32 or ``None`` (zeros); ``cu_seqlens [N+1]``
    int64/int32.  Returns ``(output [T, HV, 128] bf16, final_state)``.
    ``validate=False`` skips the host read-back of ``cu_seqlens[-1]``; the
    caller then guarantees ``cu_seqlens[N] == T``.  ``qk_l2norm=True`` uses
    every q and k row L2-normalised, ``x (sum x^2 + 1e-6)^-1/2`` in fp32
    inside the kernel (an option the reference does not have: it expects
    normalised inputs).  ``h``, a ``[NT, HV, 128, 128]`` bf16 buffer
    (``NT = num_chunks(cu_seqlens, T)``), also receives the state entering
    every chunk; the output and final state are the same bit for bit.

    ``path`` selects the kernels: ``"auto"`` (the split path -- a parallel
    chunk-preparation launch and ``HV * N * slices`` state slices -- or the
    fused chain kernel, whichever the library's :class:`Plan` of these
    sequence lengths expects to finish first; with ``validate=False`` the
    lengths are not read and the library decides from N and HV alone),
    ``"fused"`` (one workgroup per chain) or ``"split"`` with ``slices`` in
    (4, 8) state slices per chain.  Without ``qk_l2norm`` the two paths
    perform the state-path operations in the same order: their final states
    agree bit for bit but for rare last-place differences (one or two
    sequences in thousands).  ``seams=False`` keeps that equality where
    either path would otherwise cut its longest sequences in two in time to
    use idle CUs (a zero-state tail and a transition chain beside the head,
    joined by a seam pass; results then agree with the serial chain to the
    rounding of the state path, and the per-chunk states ``h`` never use
    seams).

    Input range: the state path multiplies fp16 operands, so k, v, the state
    and the intermediate X and Vn must stay below 65504 in magnitude (far
    above normalised q / k and states of ordinary size; the reference's bf16
    intermediates reach 3e38).  A value past that range becomes infinite and
    the state, once infinite or NaN, stays so to the final state:
    ``check_range=True`` checks the final states on the device after the
    launch (one reduction and one synchronisation) and raises
    :class:`RangeOverflowError` naming the sequences whose final state is not
    finite.
    """
    cu_host = validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, q.shape[1],
                              v.shape[1], check_total=validate)
    o, s = _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output=output,
                   final_state=final_state, workspace=workspace, qk_l2norm=qk_l2norm, h=h,
                   path=path, slices=slices, cu_host=cu_host, seams=seams)
    if check_range:
        check_final_range(s, state)
    return o, s


class RangeOverflowError(FloatingPointError):
    """A prefill's state path left the fp16 range: some final state is not finite."""


def check_final_range(final_state: torch.Tensor, state: Optional[torch.Tensor] = None) -> None:
    """Raise :class:`RangeOverflowError` when a final state holds an infinite
    or NaN value that its initial state did not (one device reduction per
    tensor and one synchronisation)."""
    bad = ~torch.isfinite(final_state).flatten(1).all(dim=1)
    if state is not None:
        bad &= torch.isfinite(state).flatten(1).all(dim=1)
    idx = bad.nonzero().flatten().tolist()
    if idx:
        raise RangeOverflowError(
            f"prefill state left the fp16 operand range (|x| > 65504) in sequence(s) {idx[:16]}"
            + (" ..." if len(idx) > 16 else "") + "; scale k / v or the initial state down")


def _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None, *, output=None,
            final_state=None, workspace=None, qk_l2norm: bool = False, h=None,
            path: str = "auto", slices: int = 8, cu_host: Optional[torch.Tensor] = None,
            seams: bool = True):
    """Allocation, layout and the C call behind :func:`gdn_prefill` (inputs
    already validated; ``cu_host``, when given, is the host copy of
    ``cu_seqlens`` the automatic path choice reads)."""
    T, nq, d = q.shape
    nv = v.shape[1]
    assert nv % nq == 0
    scale = _resolve_scale(scale)
    N = cu_seqlens.numel() - 1
    if state is not None and not state.is_contiguous():
        state = state.contiguous()
    q, k, v, a, b = (t.contiguous() for t in (q, k, v, a, b))
    cu = cu_seqlens.contiguous()
    A_log = A_log.contiguous()
    dt_bias = dt_bias.contiguous()
    if output is None:
        output = torch.empty(T, nv, HEAD_SIZE, dtype=torch.bfloat16, device=q.device)
    if final_state is None:
        final_state = torch.empty(N, nv, HEAD_SIZE, HEAD_SIZE, dtype=torch.float32,
                                  device=q.device)
    assert output.dtype == torch.bfloat16 and output.is_contiguous()
    assert output.shape == (T, nv, HEAD_SIZE)
    assert final_state.dtype == torch.float32 and final_state.is_contiguous()
    assert final_state.shape == (N, nv, HEAD_SIZE, HEAD_SIZE)
    assert path in ("auto", "fused", "split"), path
    flags = (_capi.GDN_QK_L2NORM if qk_l2norm else 0) | (0 if seams else _capi.GDN_NO_SEAMS)
    if path in ("auto", "fused") and cu_host is not None and h is None:
        plan = _plan_for(cu_host, T, nq, nv, seams, path == "fused", q.device)
        ws_need = plan.workspace_bytes
        if ws_need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < ws_need):
            workspace = _split_workspace(ws_need, q.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        rc = _capi.lib().gdn_prefill_plan_fwd(
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
            _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu),
            1 if cu.dtype == torch.int32 else 0, N, T, nq, nv, float(scale),
            _capi.ptr(output), _capi.ptr(final_state), plan.buf, _capi.ptr(workspace), ws_bytes,
            flags, _capi.stream_handle(q.device))
        _capi.check(rc, "gdn_prefill_plan_fwd")
        return output, final_state
    if path == "auto" and cu_host is not None:
        key = (id(cu_host), T, nv, q.device.index)
        ent = _CHOICE.get(key)
        if ent is not None and ent[0] is cu_host:
            chosen = ent[1]
        else:
            chosen = choose_slices(cu_host, T, nv) if N > 0 else 0
            if len(_CHOICE) >= 256:
                _CHOICE.clear()
            _CHOICE[key] = (cu_host, chosen)
        path, slices = ("split", chosen) if chosen else ("fused", slices)
    if path == "split":
        ws_need = split_workspace_bytes(N, T, nq, nv)
    elif path == "auto" and h is None:
        ws_need = workspace_bytes(N, T, nq, nv)
    else:
        ws_need = 0
        workspace = None
    if ws_need > 0 and (workspace is None or workspace.numel() * workspace.element_size() < ws_need):
        workspace = _split_workspace(ws_need, q.device)
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    if h is not None:
        assert h.dtype == torch.bfloat16 and h.is_contiguous() and h.device == q.device
        assert h.dim() == 4 and h.shape[1:] == (nv, HEAD_SIZE, HEAD_SIZE)
    if path == "split" and h is not None:
        rc = _capi.lib().gdn_prefill_split_h_fwd(
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
            _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu),
            1 if cu.dtype == torch.int32 else 0, N, T, nq, nv, float(scale),
            _capi.ptr(output), _capi.ptr(final_state), _capi.ptr(h), h.shape[0], int(slices),
            _capi.ptr(workspace), ws_bytes, flags, _capi.stream_handle(q.device))
        _capi.check(rc, "gdn_prefill_split_h_fwd")
        return output, final_state
    if path == "split":
        rc = _capi.lib().gdn_prefill_split_fwd(
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
            _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu),
            1 if cu.dtype == torch.int32 else 0, N, T, nq, nv, float(scale),
            _capi.ptr(output), _capi.ptr(final_state), int(slices), _capi.ptr(workspace),
            ws_bytes, flags, _capi.stream_handle(q.device))
        _capi.check(rc, "gdn_prefill_split_fwd")
        return output, final_state
    if h is not None:
        rc = _capi.lib().gdn_prefill_h_fwd(
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
            _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu),
            1 if cu.dtype == torch.int32 else 0, N, T, nq, nv, float(scale),
            _capi.ptr(output), _capi.ptr(final_state), _capi.ptr(h), h.shape[0],
            _capi.ptr(workspace), ws_bytes, flags, _capi.stream_handle(q.device))
        _capi.check(rc, "gdn_prefill_h_fwd")
        return output, final_state
    rc = _capi.lib().gdn_prefill_ex_fwd(
        _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
        _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu),
        1 if cu.dtype == torch.int32 else 0, N, T, nq, nv, float(scale),
        _capi.ptr(output), _capi.ptr(final_state), _capi.ptr(workspace), ws_bytes,
        flags, _capi.stream_handle(q.device))
    _capi.check(rc, "gdn_prefill_ex_fwd")
    return output, final_state


@torch.no_grad()
def gdn_prefill_h(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale=None, *,
                  output=None, final_state=None, h=None, workspace=None, qk_l2norm: bool = False,
                  path: str = "auto", slices: int = 8):
    """:func:`gdn_prefill` that also returns ``h [NT, HV, 128, 128]`` bf16, the
    state entering every 64-token chunk: ``h[chunk_offset(n) + i]`` is the
    state of sequence ``n`` before its chunk ``i`` (the initial state for
    ``i = 0``), as ``chunk_gated_delta_rule_fwd_h`` stores it (PRE:1341-1398,
    1153-1160; round to nearest even).  Returns ``(output, final_state, h)``.
    Reads ``cu_seqlens`` on the host once, for the reference's
    ``cu_seqlens[-1] == T`` check, to size ``h`` (as the reference's chunk
    index preparation does, PRE:175-209) and for the path choice: ``path``
    as for :func:`gdn_prefill` -- with few chains the split path writes ``h``
    from its state slices (the reference writes it from its V-split grid,
    PRE:1365-1393).
    """
    T = q.shape[0]
    nv = v.shape[1]
    cu_host = validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, q.shape[1], nv)
    NT = num_chunks(cu_host, T)
    if h is None:
        h = torch.empty(NT, nv, HEAD_SIZE, HEAD_SIZE, dtype=torch.bfloat16, device=q.device)
    assert h.shape[0] >= NT, (h.shape, NT)
    o, s = _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output=output,
                   final_state=final_state, workspace=workspace, qk_l2norm=qk_l2norm, h=h,
                   path=path, slices=slices, cu_host=cu_host)
    return o, s, h


@torch.no_grad()
def run(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale):
    """Reference-compatible prefill entry (PRE:1762-1802), qk4 / v8 / d128.

    Validates once, as PRE:1635-1667 does (one host read of ``cu_seqlens``,
    which also feeds the path choice), then launches."""
    cu_host = validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens)
    return _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, cu_host=cu_host)


@torch.no_grad()
def run_dps(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output, final_state):
    """Destination-passing prefill: writes ``output`` / ``final_state``, returns None."""
    cu_host = validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens)
    _launch(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output=output,
            final_state=final_state, cu_host=cu_host)


class PreparedPrefill:
    """A prefill call on fixed buffers, validated once and launched by one C call.

    ``cu_seqlens`` is read back once here (the reference's ``cu_seqlens[-1]
    == T`` check, and the library's :class:`Plan` of the lengths: ``path``
    is ``"split4"``, ``"split8"``, ``"fused"`` or ``"fused+<k>seams"``);
    ``__call__`` only enqueues the launches on the stream that was current at
    construction.  ``qk_l2norm`` and ``seams`` as for :func:`gdn_prefill`;
    ``fused=True`` plans the fused kernel whatever the lengths favour.
    """

    def __init__(self, q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, output,
                 final_state, *, qk_l2norm: bool = False, seams: bool = True, fused: bool = False):
        T, nq, _ = q.shape
        nv = v.shape[1]
        cu_host = validate_inputs(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, nq, nv)
        N = cu_seqlens.numel() - 1
        for t in (q, k, v, a, b, cu_seqlens, A_log, dt_bias):
            assert t.is_contiguous()
        assert state is None or state.is_contiguous()
        assert output.dtype == torch.bfloat16 and output.is_contiguous()
        assert output.shape == (T, nv, HEAD_SIZE)
        assert final_state.dtype == torch.float32 and final_state.is_contiguous()
        assert final_state.shape == (N, nv, HEAD_SIZE, HEAD_SIZE)
        # the path and seams the sequence lengths favour
        self.plan = Plan(cu_host, T, nq, nv, seams=seams, fused=fused)
        self.slices = self.plan.slices
        self.path = self.plan.path
        ws = self.plan.workspace_bytes
        self._ws = torch.empty(ws, dtype=torch.uint8, device=q.device) if ws else None
        self._keep = (q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, output, final_state)
        head = (
            _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), _capi.ptr(state), _capi.ptr(A_log),
            _capi.ptr(a), _capi.ptr(dt_bias), _capi.ptr(b), _capi.ptr(cu_seqlens),
            1 if cu_seqlens.dtype == torch.int32 else 0, N, T, nq, nv,
            float(_resolve_scale(scale)), _capi.ptr(output), _capi.ptr(final_state))
        flags = (_capi.GDN_QK_L2NORM if qk_l2norm else 0) | (0 if seams else _capi.GDN_NO_SEAMS)
        self._name = "gdn_prefill_plan_fwd"
        self._args = head + (self.plan.buf, _capi.ptr(self._ws), ws, flags,
                             _capi.stream_handle(q.device))
        self._fn = getattr(_capi.lib(), self._name)

    def __call__(self) -> None:
        rc = self._fn(*self._args)
        if rc:
            _capi.check(rc, self._name)
