"""The C ABI library loads and exports every entry point include/nanokv.h
declares; argument validation fails cleanly without touching a GPU."""
import ctypes
import re
from pathlib import Path

import pytest

from nanokv_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "nanokv.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(nkv_[a-z_0-9]+)\s*\(", text)))


def test_header_matches_binding_list():
    assert declared_functions() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.nkv_abi_version() == _lib.NKV_ABI_VERSION


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _lib.lib()
    # odd rank: cannot pack two codes per byte
    rc = lib.nkv_quant_pack(None, None, 4, 7, 7, 0, 0, None, None)
    assert rc == _lib.NKV_ERR_INVALID
    assert b"multiple of 8" in lib.nkv_last_error()
    rc = lib.nkv_quant_pack(None, None, 4, 64, 32, 5, 0, None, None)
    assert rc == _lib.NKV_ERR_INVALID
    rc = lib.nkv_assign(None, None, None, 10, 300, 64, None, 1)
    assert rc == _lib.NKV_ERR_INVALID and b"uint8 ids" in lib.nkv_last_error()
    # empty work succeeds without pointers
    assert lib.nkv_quant_pack(None, None, 0, 64, 32, 0, 0, None, None) == _lib.NKV_OK
    assert lib.nkv_last_error() == b""


def test_attend_rejects_unsupported_shapes():
    lib = _lib.lib()
    args = _lib.NkvAttendArgs()
    args.B, args.H, args.D, args.Q = 1, 2, 64, 8
    assert lib.nkv_attend_workspace_size(ctypes.byref(args)) == 0
    assert b"D == 128" in lib.nkv_last_error()
    rc = lib.nkv_attend(None, ctypes.byref(args), None, 0)
    assert rc == _lib.NKV_ERR_UNSUPPORTED
    args.D = 128
    args.N = 10
    args.key.r = 96
    args.key.packed = args.key.scales = args.key.w_dec = 1
    rc = lib.nkv_attend(None, ctypes.byref(args), None, 0)
    assert rc == _lib.NKV_ERR_UNSUPPORTED and b"ranks" in lib.nkv_last_error()
