"""ctypes binding of libnanokv_hip.so (the C ABI declared in include/nanokv.h).

The library is loaded lazily on first use.  There is no fallback: if the
shared library is missing or fails to load, every product call raises.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import (POINTER, Structure, c_char_p, c_float, c_int, c_int64, c_size_t,
                    c_uint8, c_uint16, c_void_p)
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnanokv_hip.so"

NKV_ABI_VERSION = 7
NKV_OK = 0
NKV_ERR_INVALID = -1
NKV_ERR_UNSUPPORTED = -2
NKV_ERR_HIP = -3
NKV_ERR_WORKSPACE = -4

NKV_DTYPE_BF16 = 0
NKV_DTYPE_FP16 = 1
NKV_QUANT_FP32 = 0
NKV_QUANT_BF16 = 1
NKV_SCHEDULE_AUTO = 0
NKV_SCHEDULE_QUERY_TILES = 1
NKV_SCHEDULE_KEY_CHUNKS = 2

# Every symbol include/nanokv.h declares (checked by tests/test_abi.py).
EXPORTED = (
    "nkv_abi_version", "nkv_last_error", "nkv_quant_pack", "nkv_unpack", "nkv_assign",
    "nkv_encode", "nkv_encode_batch", "nkv_decode", "nkv_attend_workspace_size", "nkv_attend", "nkv_lse_merge",
    "nkv_fast_attend_workspace_size", "nkv_fast_attend", "nkv_rope_apply", "nkv_int8_pack",
    "nkv_int8_dequant", "nkv_c64_fit_workspace_size", "nkv_c64_fit", "nkv_camera_apply",
    "nkv_attend_static", "nkv_lift_lse_combine", "nkv_finish", "nkv_reader_rows",
)
NKV_STATIC_SCRATCH_BYTES = 64 << 20


class NkvSegment(Structure):
    _fields_ = [
        ("packed", c_void_p), ("scales", c_void_p), ("ids", c_void_p), ("centers", c_void_p),
        ("row_start", c_int64), ("rows", c_int64), ("centers_batch_stride", c_int64),
        ("center_base", c_int64), ("num_centers", c_int), ("id_bytes", c_int),
    ]


class NkvCodec(Structure):
    _fields_ = [
        ("packed", c_void_p), ("scales", c_void_p), ("ids", c_void_p), ("centers", c_void_p),
        ("w_dec", c_void_p), ("mean", c_void_p),
        ("r", c_int), ("group", c_int), ("scale_dtype", c_int), ("id_bytes", c_int),
        ("num_centers", c_int), ("n_segments", c_int),
        ("centers_batch_stride", c_int64),
        ("segments", POINTER(NkvSegment)), ("segments_dev", c_void_p),
    ]


class NkvEncodeArgs(Structure):
    _fields_ = [
        ("rows", c_int64), ("HD", c_int), ("r", c_int), ("group", c_int),
        ("scale_dtype", c_int), ("quant_mode", c_int), ("num_centers", c_int),
        ("id_bytes", c_int), ("ids_in", c_int),
        ("x", c_void_p), ("centers", c_void_p), ("mean", c_void_p), ("w_enc", c_void_p),
        ("ids", c_void_p), ("coeff", c_void_p), ("packed", c_void_p), ("scales", c_void_p),
        ("x_bf16", c_void_p), ("x_stride", c_int64),
    ]


class NkvDecodeArgs(Structure):
    _fields_ = [
        ("B", c_int), ("HD", c_int), ("N", c_int64), ("rows", c_int64),
        ("row_index", c_void_p), ("codec", NkvCodec), ("out", c_void_p),
    ]


class NkvRope(Structure):
    _fields_ = [
        ("cs_t", c_void_p), ("cs_h", c_void_p), ("cs_w", c_void_p), ("frame_pos", c_void_p),
        ("n_frames", c_int64), ("n_t", c_int), ("pt", c_int), ("ph", c_int), ("pw", c_int),
        ("grid_h", c_int), ("grid_w", c_int), ("_pad", c_int),
        ("cs_rows", c_void_p), ("n_rows", c_int64),
    ]


NKV_CAMERA_FULL = 0
NKV_CAMERA_SF13 = 1


class NkvCamera(Structure):
    _fields_ = [
        ("mats", c_void_p), ("mats_bs", c_int64), ("n_mats", c_int), ("layout", c_int),
        ("frame_mat", c_void_p), ("n_frames", c_int64), ("tokens_per_frame", c_int),
        ("n_batches", c_int),
    ]


class NkvAttendArgs(Structure):
    _fields_ = [
        ("B", c_int), ("H", c_int), ("D", c_int), ("splits", c_int),
        ("Q", c_int64), ("N", c_int64), ("Nc", c_int64),
        ("softmax_scale", c_float), ("schedule", c_int),
        ("q", c_void_p), ("q_sb", c_int64), ("q_st", c_int64), ("q_sh", c_int64),
        ("k_cur", c_void_p), ("k_sb", c_int64), ("k_st", c_int64), ("k_sh", c_int64),
        ("v_cur", c_void_p), ("v_sb", c_int64), ("v_st", c_int64), ("v_sh", c_int64),
        ("key", NkvCodec), ("value", NkvCodec),
        ("out", c_void_p), ("o_sb", c_int64), ("o_st", c_int64), ("o_sh", c_int64),
        ("lse", c_void_p), ("ev_kernel_begin", c_void_p), ("ev_kernel_end", c_void_p),
        ("rope", POINTER(NkvRope)), ("camera", POINTER(NkvCamera)),
        ("hist_rows", c_void_p), ("n_hist", c_int64), ("cur_mask", c_void_p),
        ("q_group", c_void_p), ("n_groups", c_int), ("cur_mask_words", c_int),
    ]


class NkvReaderGroup(Structure):
    _fields_ = [
        ("num_heads", c_int), ("d", c_int), ("heads", c_void_p), ("q_reduce", c_void_p),
        ("k_read", c_void_p), ("v_read", c_void_p), ("k_affine", c_void_p),
        ("v_affine", c_void_p), ("rope_pairs", c_void_p), ("cam_blocks", c_void_p),
    ]


class NkvFastArgs(Structure):
    _fields_ = [
        ("attend", NkvAttendArgs), ("protect_rows", c_void_p), ("n_protect", c_int64),
        ("low_rows", c_void_p), ("n_low", c_int64), ("num_groups", c_int), ("_pad", c_int),
        ("groups", POINTER(NkvReaderGroup)),
        ("q_pre", c_void_p), ("qp_sb", c_int64), ("qp_st", c_int64), ("qp_sh", c_int64),
        ("q_rope", POINTER(NkvRope)), ("q_camera", POINTER(NkvCamera)),
        ("low_shift", c_void_p), ("ls_sb", c_int64), ("ls_sh", c_int64),
        ("o_camera", POINTER(NkvCamera)),
    ]


class NkvReaderRowsArgs(Structure):
    _fields_ = [
        ("B", c_int), ("H", c_int), ("D", c_int), ("E", c_int), ("nh", c_int),
        ("out_width", c_int), ("S", c_int64),
        ("x", c_void_p), ("x_sb", c_int64), ("x_st", c_int64), ("x_sh", c_int64),
        ("heads", c_void_p), ("w", c_void_p),
        ("rope", POINTER(NkvRope)), ("pairs", c_void_p),
        ("camera", POINTER(NkvCamera)), ("blocks", c_void_p),
        ("out", c_void_p),
    ]


class NkvLiftCombineArgs(Structure):
    _fields_ = [
        ("B", c_int), ("H", c_int), ("Q", c_int), ("low_dim", c_int),
        ("native", c_void_p), ("n_sb", c_int64), ("n_sh", c_int64), ("n_sq", c_int64),
        ("n_sd", c_int64),
        ("native_lse", c_void_p), ("nl_sb", c_int64), ("nl_sh", c_int64), ("nl_sq", c_int64),
        ("low", c_void_p), ("l_sb", c_int64), ("l_sh", c_int64), ("l_sq", c_int64),
        ("l_sd", c_int64),
        ("main_lift", c_void_p), ("ml_sh", c_int64), ("ml_sk", c_int64), ("ml_so", c_int64),
        ("prope_mix", c_void_p), ("pm_sh", c_int64), ("pm_sk", c_int64), ("pm_so", c_int64),
        ("history_lse", c_void_p), ("hl_sb", c_int64), ("hl_sh", c_int64), ("hl_sq", c_int64),
        ("out", c_void_p),
    ]


class NkvFinishArgs(Structure):
    _fields_ = [
        ("B", c_int), ("H_native", c_int), ("H_group", c_int), ("S", c_int), ("D", c_int),
        ("native", c_void_p), ("a_sb", c_int64), ("a_sh", c_int64), ("a_ss", c_int64),
        ("a_sd", c_int64),
        ("native_lse", c_void_p), ("la_sb", c_int64), ("la_sh", c_int64), ("la_ss", c_int64),
        ("lifted", c_void_p), ("b_sb", c_int64), ("b_sh", c_int64), ("b_ss", c_int64),
        ("b_sd", c_int64),
        ("low_lse", c_void_p), ("lb_sb", c_int64), ("lb_sh", c_int64), ("lb_ss", c_int64),
        ("heads", c_void_p),
        ("mean", c_void_p), ("m_sb", c_int64), ("m_sh", c_int64), ("m_sd", c_int64),
        ("projected", c_void_p), ("p_sb", c_int64), ("p_sh", c_int64), ("p_sd", c_int64),
        ("result", c_void_p), ("y_sb", c_int64), ("y_sh", c_int64), ("y_ss", c_int64),
        ("y_sd", c_int64),
    ]


class NanoKVError(RuntimeError):
    """A libnanokv_hip.so call returned an error code."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed with code {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib = None


def _declare(lib: ctypes.CDLL) -> None:
    lib.nkv_abi_version.restype = c_int
    lib.nkv_abi_version.argtypes = []
    lib.nkv_last_error.restype = c_char_p
    lib.nkv_last_error.argtypes = []
    lib.nkv_quant_pack.restype = c_int
    lib.nkv_quant_pack.argtypes = [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int,
                                   c_void_p, c_void_p]
    lib.nkv_unpack.restype = c_int
    lib.nkv_unpack.argtypes = [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int,
                               c_int, c_void_p]
    lib.nkv_assign.restype = c_int
    lib.nkv_assign.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p,
                               c_int]
    lib.nkv_encode.restype = c_int
    lib.nkv_encode.argtypes = [c_void_p, POINTER(NkvEncodeArgs)]
    lib.nkv_encode_batch.restype = c_int
    lib.nkv_encode_batch.argtypes = [c_void_p, POINTER(NkvEncodeArgs), c_int]
    lib.nkv_decode.restype = c_int
    lib.nkv_decode.argtypes = [c_void_p, POINTER(NkvDecodeArgs)]
    lib.nkv_attend_workspace_size.restype = c_size_t
    lib.nkv_attend_workspace_size.argtypes = [POINTER(NkvAttendArgs)]
    lib.nkv_attend.restype = c_int
    lib.nkv_attend.argtypes = [c_void_p, POINTER(NkvAttendArgs), c_void_p, c_size_t]
    lib.nkv_attend_static.restype = c_int
    lib.nkv_attend_static.argtypes = [c_void_p, POINTER(NkvAttendArgs)]
    lib.nkv_fast_attend_workspace_size.restype = c_size_t
    lib.nkv_fast_attend_workspace_size.argtypes = [POINTER(NkvFastArgs)]
    lib.nkv_fast_attend.restype = c_int
    lib.nkv_fast_attend.argtypes = [c_void_p, POINTER(NkvFastArgs), c_void_p, c_size_t]
    lib.nkv_reader_rows.restype = c_int
    lib.nkv_reader_rows.argtypes = [c_void_p, POINTER(NkvReaderRowsArgs)]
    lib.nkv_c64_fit_workspace_size.restype = c_size_t
    lib.nkv_c64_fit_workspace_size.argtypes = [c_int, c_int64, c_int]
    lib.nkv_c64_fit.restype = c_int
    lib.nkv_c64_fit.argtypes = [c_void_p, c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_size_t]
    lib.nkv_int8_pack.restype = c_int
    lib.nkv_int8_pack.argtypes = [c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p]
    lib.nkv_int8_dequant.restype = c_int
    lib.nkv_int8_dequant.argtypes = [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int,
                                     c_void_p]
    lib.nkv_rope_apply.restype = c_int
    lib.nkv_rope_apply.argtypes = [c_void_p, POINTER(NkvRope), c_int, c_int64, c_int, c_int,
                                   c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                   c_int64, c_int64, c_int64]
    lib.nkv_camera_apply.restype = c_int
    lib.nkv_camera_apply.argtypes = [c_void_p, POINTER(NkvCamera), c_int, c_int64, c_int, c_int,
                                     c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p,
                                     c_int64, c_int64, c_int64]
    lib.nkv_lse_merge.restype = c_int
    lib.nkv_lse_merge.argtypes = [c_void_p, c_int64, c_int, c_void_p, c_int64, c_void_p,
                                  c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p]
    lib.nkv_lift_lse_combine.restype = c_int
    lib.nkv_lift_lse_combine.argtypes = [c_void_p, POINTER(NkvLiftCombineArgs)]
    lib.nkv_finish.restype = c_int
    lib.nkv_finish.argtypes = [c_void_p, POINTER(NkvFinishArgs)]


def lib() -> ctypes.CDLL:
    """Load libnanokv_hip.so once; raise if it is absent or incompatible."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m nanokv_amd.build` "
                    "(there is no CPU fallback for the NanoKV HIP path)")
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            version = handle.nkv_abi_version()
            if version != NKV_ABI_VERSION:
                raise RuntimeError(f"libnanokv_hip ABI {version} != expected {NKV_ABI_VERSION}")
            _lib = handle
    return _lib


def check(func: str, code: int) -> None:
    if code != NKV_OK:
        message = lib().nkv_last_error().decode(errors="replace")
        raise NanoKVError(func, code, message)
