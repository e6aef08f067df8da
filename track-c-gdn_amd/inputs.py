"""Seeded synthetic inputs for the GDN decode / prefill workloads.

All tensors are drawn on the CPU from ``torch.Generator().manual_seed(seed)``
in float32 and then cast, so the CPU checker and the GPU see bit-identical
inputs.  Distributions (the workloads the operators are benchmarked on):

* ``q, k ~ N(0, 1)``, L2-normalised over the head dimension in fp32, then bf16
* ``v ~ N(0, 1)`` bf16
* ``state ~ N(0, 0.02)`` fp32 (std 0.02)
* ``A_log ~ U(-2, 0)`` fp32, ``dt_bias ~ N(0, 0.1)`` fp32
* ``a, b ~ N(0, 1)`` bf16
* ``scale = 1 / sqrt(head_dim)``

Shapes follow the reference entry points: decode ``q, k [B, 1, HQ, D]``,
``v [B, 1, HV, D]``, ``a, b [B, 1, HV]`` (DEC:117-120, 132-134); prefill
``q, k [T, HQ, D]``, ``v [T, HV, D]``, ``a, b [T, HV]``, ``cu_seqlens [N+1]``
(PRE:1657-1667).
"""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import torch

D = 128


def _unit_rows(x: torch.Tensor) -> torch.Tensor:
    return x / x.norm(dim=-1, keepdim=True).clamp_min(1e-12)


def _common_gates(gen: torch.Generator, HV: int):
    A_log = torch.rand(HV, generator=gen) * 2.0 - 2.0
    dt_bias = torch.randn(HV, generator=gen) * 0.1
    return A_log.float(), dt_bias.float()


def decode_inputs(B: int, HQ: int = 4, HV: int = 8, seed: int = 1001,
                  with_state: bool = True, head_dim: int = D) -> Dict[str, torch.Tensor]:
    """Inputs of one decode step at batch ``B`` (CPU tensors)."""
    gen = torch.Generator().manual_seed(seed)
    q = _unit_rows(torch.randn(B, 1, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    k = _unit_rows(torch.randn(B, 1, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, 1, HV, head_dim, generator=gen).to(torch.bfloat16)
    state = (torch.randn(B, HV, head_dim, head_dim, generator=gen) * 0.02) if with_state else None
    A_log, dt_bias = _common_gates(gen, HV)
    a = torch.randn(B, 1, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(B, 1, HV, generator=gen).to(torch.bfloat16)
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                scale=1.0 / math.sqrt(head_dim))


def decode_multi_inputs(B: int, T: int, HQ: int = 4, HV: int = 8, seed: int = 1005,
                        with_state: bool = True, head_dim: int = D) -> Dict[str, torch.Tensor]:
    """Inputs of T consecutive decode steps per sequence at batch ``B`` (CPU tensors)."""
    gen = torch.Generator().manual_seed(seed)
    q = _unit_rows(torch.randn(B, T, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    k = _unit_rows(torch.randn(B, T, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, HV, head_dim, generator=gen).to(torch.bfloat16)
    state = (torch.randn(B, HV, head_dim, head_dim, generator=gen) * 0.02) if with_state else None
    A_log, dt_bias = _common_gates(gen, HV)
    a = torch.randn(B, T, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(B, T, HV, generator=gen).to(torch.bfloat16)
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                scale=1.0 / math.sqrt(head_dim))


def prefill_inputs(lengths: Sequence[int], HQ: int = 4, HV: int = 8, seed: int = 1002,
                   with_state: bool = False, cu_dtype=torch.int64,
                   head_dim: int = D) -> Dict[str, torch.Tensor]:
    """Inputs of one varlen prefill call over sequences of ``lengths`` (CPU tensors)."""
    gen = torch.Generator().manual_seed(seed)
    lengths = [int(x) for x in lengths]
    T = sum(lengths)
    N = len(lengths)
    cu = torch.zeros(N + 1, dtype=torch.int64)
    cu[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0)
    q = _unit_rows(torch.randn(T, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    k = _unit_rows(torch.randn(T, HQ, head_dim, generator=gen)).to(torch.bfloat16)
    v = torch.randn(T, HV, head_dim, generator=gen).to(torch.bfloat16)
    state = (torch.randn(N, HV, head_dim, head_dim, generator=gen) * 0.02) if with_state else None
    A_log, dt_bias = _common_gates(gen, HV)
    a = torch.randn(T, HV, generator=gen).to(torch.bfloat16)
    b = torch.randn(T, HV, generator=gen).to(torch.bfloat16)
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                cu_seqlens=cu.to(cu_dtype), scale=1.0 / math.sqrt(head_dim))


def varlen_lengths_uniform(n: int, lo: int, hi: int, seed: int) -> List[int]:
    """``n`` lengths drawn uniformly from ``[lo, hi]`` (seeded)."""
    gen = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=gen)]


def varlen_lengths_total(n: int, total: int, seed: int, spread: float = 0.5) -> List[int]:
    """``n`` ragged lengths summing to ``total``.

    Each length is ``total/n * (1 + spread * u)`` with ``u ~ U(-1, 1)``
    (seeded), rescaled to the exact total; the rounding residue goes to the
    last sequence.
    """
    gen = torch.Generator().manual_seed(seed)
    w = 1.0 + spread * (torch.rand(n, generator=gen, dtype=torch.float64) * 2.0 - 1.0)
    raw = (w / w.sum() * total).floor().long()
    raw[-1] += total - int(raw.sum())
    return [int(x) for x in raw]


# The benchmark workloads, by name.
WORKLOADS = {
    "decode_b1_qk4_v8": dict(kind="decode", B=1, HQ=4, HV=8, seed=1000),
    "decode_b256_qk4_v8": dict(kind="decode", B=256, HQ=4, HV=8, seed=1001),
    "prefill_t4096_n1_qk4_v8": dict(kind="prefill", lengths=[4096], HQ=4, HV=8, seed=1002,
                                    with_state=False),
    "prefill_varlen16_qk4_v8": dict(kind="prefill", lengths=None, HQ=4, HV=8, seed=1003,
                                    with_state=True, cu_dtype=torch.int32),
    "prefill_varlen8_t32768_qk16_v32": dict(kind="prefill", lengths=None, HQ=16, HV=32,
                                            seed=1004, with_state=True),
    "decode_pool_b1024_qk16_v32": dict(kind="decode_pool", B=1024, HQ=16, HV=32, seed=1004),
}


def workload_lengths(name: str) -> Optional[List[int]]:
    """Sequence lengths of a prefill workload.

    * ``prefill_varlen16_qk4_v8``: 16 lengths ``~ U[128, 8192]`` (seed 1003).
    * ``prefill_varlen8_t32768_qk16_v32``: 8 ragged lengths summing to 32768,
      each within +-50% of the mean before rescaling (seed 1004).
    """
    w = WORKLOADS[name]
    if w["kind"] != "prefill":
        return None
    if w["lengths"] is not None:
        return list(w["lengths"])
    if name == "prefill_varlen16_qk4_v8":
        return varlen_lengths_uniform(16, 128, 8192, seed=w["seed"])
    if name == "prefill_varlen8_t32768_qk16_v32":
        return varlen_lengths_total(8, 32768, seed=w["seed"], spread=0.5)
    raise KeyError(name)
