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
    args.B, args.H, args.D, args.Q = 1, 2, 256, 8
    assert lib.nkv_attend_workspace_size(ctypes.byref(args)) == 0
    assert b"D == 128" in lib.nkv_last_error()
    args.D = 60   # narrower heads need D % 8 == 0
    assert lib.nkv_attend_workspace_size(ctypes.byref(args)) == 0
    assert b"D % 8" in lib.nkv_last_error()
    args.D = 256
    rc = lib.nkv_attend(None, ctypes.byref(args), None, 0)
    assert rc == _lib.NKV_ERR_UNSUPPORTED
    args.D = 128
    args.N = 10
    args.key.r = 96
    args.key.packed = args.key.scales = args.key.w_dec = 1
    rc = lib.nkv_attend(None, ctypes.byref(args), None, 0)
    assert rc == _lib.NKV_ERR_UNSUPPORTED and b"ranks" in lib.nkv_last_error()


STRUCTS = {
    "nkv_segment": _lib.NkvSegment, "nkv_codec": _lib.NkvCodec, "nkv_rope": _lib.NkvRope,
    "nkv_camera": _lib.NkvCamera, "nkv_encode_args": _lib.NkvEncodeArgs,
    "nkv_decode_args": _lib.NkvDecodeArgs, "nkv_attend_args": _lib.NkvAttendArgs,
    "nkv_reader_group": _lib.NkvReaderGroup, "nkv_fast_args": _lib.NkvFastArgs,
    "nkv_lift_combine_args": _lib.NkvLiftCombineArgs, "nkv_finish_args": _lib.NkvFinishArgs,
    "nkv_reader_rows_args": _lib.NkvReaderRowsArgs,
}


def test_ctypes_structs_match_the_header_layout(tmp_path):
    """Every ctypes mirror has the size and field offsets gcc gives the C
    structs of include/nanokv.h (a stale mirror would pass fields at the wrong
    offsets)."""
    import shutil
    import subprocess
    gcc = shutil.which("gcc") or shutil.which("cc")
    if gcc is None:
        pytest.skip("no C compiler")
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    for cname, cls in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([gcc, "-std=c99", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        cname, field, value = line.split()
        got[(cname, field)] = int(value)
    for cname, cls in STRUCTS.items():
        assert ctypes.sizeof(cls) == got[(cname, "size")], cname
        for field, _ in cls._fields_:
            assert getattr(cls, field).offset == got[(cname, field)], (cname, field)
