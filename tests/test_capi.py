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
        "gdn_prefill_fwd", "gdn_prefill_ex_fwd"])


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
