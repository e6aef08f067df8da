"""Short causal convolution ahead of GDN (a Qwen3-Next-style layer's
``mixed_qkv`` conv1d + SiLU), written straight into the GDN operators' q / k /
v layout.

The reference operators take q, k and v after this step (they have no
counterpart of it).  In the layer, ``mixed_qkv = cat(q, k, v)`` over
channels (``C = 2 * 128 * HQ + 128 * HV``) passes through a depthwise causal
conv1d of kernel size W (4) and SiLU; decode keeps the last inputs of every
sequence as a conv state.

* :func:`qkv_conv1d` -- packed varlen sequences (prefill); returns q, k, v
  ready for :func:`prefill.gdn_prefill` and each sequence's final conv state.
* :func:`qkv_conv1d_update` -- one token per sequence (decode), the conv
  state updated in place; returns q, k, v shaped for :func:`decode.gdn_decode`.

All compute runs in the HIP kernels of libgdn_hip.so on torch's current
stream.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _capi

D = 128
_ACT = {"silu": _capi.GDN_ACT_SILU, None: _capi.GDN_ACT_NONE}


def _weights(weight, bias, C):
    assert weight.dim() == 2 and weight.shape[0] == C, weight.shape
    weight = weight.float().contiguous()
    if bias is not None:
        assert bias.shape == (C,)
        bias = bias.float().contiguous()
    return weight, bias


@torch.no_grad()
def qkv_conv1d(mixed_qkv, weight, bias, cu_seqlens, conv_state=None, *, num_q_heads: int,
               num_v_heads: int, activation: Optional[str] = "silu", state_len: Optional[int] = None,
               return_state: bool = True):
    """Causal depthwise conv1d + activation over packed sequences.

    ``mixed_qkv [T, C]`` bf16 with ``C = 256 * num_q_heads + 128 * num_v_heads``;
    ``weight [C, W]`` (any float dtype, used in fp32), ``bias [C]`` or ``None``;
    ``cu_seqlens [N+1]`` int64/int32 on the GPU; ``conv_state [N, C, S]`` bf16
    or ``None``.  Returns ``(q [T, HQ, 128], k [T, HQ, 128], v [T, HV, 128],
    final_state [N, C, S] or None)``; ``S`` is the given state's length, else
    ``state_len``, else ``W - 1``.
    """
    assert mixed_qkv.is_cuda and mixed_qkv.dtype == torch.bfloat16 and mixed_qkv.dim() == 2
    T, C = mixed_qkv.shape
    HQ, HV = int(num_q_heads), int(num_v_heads)
    assert C == 2 * D * HQ + D * HV, (C, HQ, HV)
    assert cu_seqlens.is_cuda and cu_seqlens.dtype in (torch.int64, torch.int32)
    N = cu_seqlens.numel() - 1
    weight, bias = _weights(weight, bias, C)
    W = weight.shape[1]
    if conv_state is not None:
        assert conv_state.dtype == torch.bfloat16 and conv_state.dim() == 3
        assert conv_state.shape[:2] == (N, C)
        conv_state = conv_state.contiguous()
        S = conv_state.shape[2]
    else:
        S = int(state_len) if state_len is not None else W - 1
    x = mixed_qkv.contiguous()
    cu = cu_seqlens.contiguous()
    q = torch.empty(T, HQ, D, dtype=torch.bfloat16, device=x.device)
    k = torch.empty(T, HQ, D, dtype=torch.bfloat16, device=x.device)
    v = torch.empty(T, HV, D, dtype=torch.bfloat16, device=x.device)
    final = (torch.empty(N, C, S, dtype=torch.bfloat16, device=x.device) if return_state else None)
    rc = _capi.lib().gdn_qkv_conv1d_fwd(
        _capi.ptr(x), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(cu),
        1 if cu.dtype == torch.int32 else 0, N, T, C, W, _capi.ptr(conv_state), _capi.ptr(final),
        S, _capi.ptr(q), _capi.ptr(k), _capi.ptr(v), D * HQ, D * HQ, _ACT[activation],
        _capi.stream_handle(x.device))
    _capi.check(rc, "gdn_qkv_conv1d_fwd")
    return q, k, v, final


@torch.no_grad()
def qkv_conv1d_update(mixed_qkv, conv_state, weight, bias, *, num_q_heads: int, num_v_heads: int,
                      slot_ids=None, activation: Optional[str] = "silu"):
    """One decode token per sequence: ``mixed_qkv [B, C]`` (or ``[B, 1, C]``)
    bf16, ``conv_state [pool, C, S]`` bf16 updated in place (row
    ``slot_ids[b]`` or ``b``).  Returns ``(q [B, 1, HQ, 128], k [B, 1, HQ, 128],
    v [B, 1, HV, 128])``, the decode operators' input shapes."""
    assert mixed_qkv.is_cuda and mixed_qkv.dtype == torch.bfloat16
    x = mixed_qkv.reshape(mixed_qkv.shape[0], -1).contiguous()
    B, C = x.shape
    HQ, HV = int(num_q_heads), int(num_v_heads)
    assert C == 2 * D * HQ + D * HV, (C, HQ, HV)
    assert conv_state.dtype == torch.bfloat16 and conv_state.is_contiguous()
    assert conv_state.dim() == 3 and conv_state.shape[1] == C
    weight, bias = _weights(weight, bias, C)
    W = weight.shape[1]
    if slot_ids is not None:
        assert slot_ids.dtype == torch.int32 and slot_ids.is_cuda and slot_ids.numel() == B
        slot_ids = slot_ids.contiguous()
    else:
        assert conv_state.shape[0] >= B
    q = torch.empty(B, 1, HQ, D, dtype=torch.bfloat16, device=x.device)
    k = torch.empty(B, 1, HQ, D, dtype=torch.bfloat16, device=x.device)
    v = torch.empty(B, 1, HV, D, dtype=torch.bfloat16, device=x.device)
    rc = _capi.lib().gdn_qkv_conv1d_update(
        _capi.ptr(x), _capi.ptr(weight), _capi.ptr(bias), _capi.ptr(conv_state), conv_state.shape[2],
        _capi.ptr(slot_ids), conv_state.shape[0], B, C, W, _capi.ptr(q), _capi.ptr(k), _capi.ptr(v),
        D * HQ, D * HQ, _ACT[activation], _capi.stream_handle(x.device))
    _capi.check(rc, "gdn_qkv_conv1d_update")
    return q, k, v
