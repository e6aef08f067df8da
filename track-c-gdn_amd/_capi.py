"""ctypes binding of libgdn_hip.so (declared in include/gdn_hip.h).

torch is imported before the library is opened so that the library binds to
the HIP runtime torch already loaded (one runtime per process).  A missing
library is an error: there is no fallback path.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = Path(__file__).resolve().with_name("libgdn_hip.so")

GDN_OK = 0
GDN_ERR_NULL = -1001
GDN_ERR_SHAPE = -1002
GDN_ERR_WORKSPACE = -1003
GDN_QK_L2NORM = 1
GDN_NO_SEAMS = 2
GDN_PLAN_FUSED = 4
GDN_PREFILL_PLAN_BYTES = 512
GDN_ACT_NONE = 0
GDN_ACT_SILU = 1

# Every symbol include/gdn_hip.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.c_size_t
SIGNATURES = {
    "gdn_abi_version": (_I, []),
    "gdn_error_string": (ctypes.c_char_p, [_I]),
    "gdn_decode_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "gdn_decode_pool_fwd": (_I, [_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P]),
    "gdn_decode_ex_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _I, _P]),
    "gdn_decode_multi_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _P]),
    "gdn_prefill_workspace_bytes": (_S, [_I, _I, _I, _I]),
    "gdn_prefill_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                             _P, _P, _P, _S, _P]),
    "gdn_prefill_ex_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                _P, _P, _P, _S, _I, _P]),
    "gdn_prefill_auto_slices": (_I, [_I, _I]),
    "gdn_prefill_split_workspace_bytes": (_S, [_I, _I, _I, _I]),
    "gdn_prefill_split_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                   _P, _P, _I, _P, _S, _I, _P]),
    "gdn_prefill_split_noalloc_max_bytes": (_S, []),
    "gdn_prefill_split_noalloc_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                           _F, _P, _P, _I, _I, _P]),
    "gdn_prefill_chunk_count": (ctypes.c_longlong, [_P, _I, _I, _I]),
    "gdn_prefill_choose_slices": (_I, [_P, _I, _I, _I, _I, _I]),
    "gdn_prefill_plan": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, ctypes.POINTER(_S)]),
    "gdn_prefill_plan_info": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I),
                                   ctypes.POINTER(_I)]),
    "gdn_prefill_plan_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                  _P, _P, _P, _P, _S, _I, _P]),
    "gdn_qkv_conv1d_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P, _P, _P, _I, _I,
                                _I, _P]),
    "gdn_qkv_conv1d_update": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I, _I,
                                   _P]),
    "gdn_prefill_h_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                               _P, _P, _P, _I, _P, _S, _I, _P]),
    "gdn_prefill_split_h_fwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F,
                                     _P, _P, _P, _I, _I, _P, _S, _I, _P]),
    "gdn_prefill_bwd_workspace_bytes": (_S, [_I, _I, _I, _I]),
    "gdn_prefill_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _I, _P,
                             _P, _P, _P, _P, _P, _P, _P, _P, _S, _P]),
    "gdn_gate_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _P, _P]),
}

_lib = None


class GdnError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """Open libgdn_hip.so once and declare its signatures."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950) first")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != GDN_OK:
        msg = lib().gdn_error_string(rc).decode()
        raise GdnError(f"{what} failed with status {rc}: {msg}")


def ptr(t) -> int:
    """Device address of a tensor (or 0 for None)."""
    return 0 if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device) -> int:
    """The hipStream_t of torch's current stream on ``device`` (torch's raw
    accessor when it has one: a tenth of the cost of building the Stream
    object)."""
    if _raw_stream is not None:
        idx = device.index if isinstance(device, torch.device) else None
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream
