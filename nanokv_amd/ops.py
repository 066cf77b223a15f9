"""Torch-facing wrappers of the NanoKV HIP kernels.

Each function validates shapes, dtypes and devices on the host, allocates its
outputs with torch on the input's device, and enqueues the kernel on the
current HIP stream through the C ABI (include/nanokv.h).  There is no CPU
path: tensors must live on the GPU and the HIP library must be built.
"""
from __future__ import annotations

import ctypes
import math
from ctypes import byref
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import (NKV_DTYPE_BF16, NKV_DTYPE_FP16, NKV_QUANT_BF16, NKV_QUANT_FP32,
                   NKV_SCHEDULE_AUTO, NKV_SCHEDULE_KEY_CHUNKS, NKV_SCHEDULE_QUERY_TILES,
                   NkvAttendArgs, NkvCodec, NkvDecodeArgs, NkvEncodeArgs, NkvFastArgs,
                   NkvCamera, NkvFinishArgs, NkvLiftCombineArgs, NkvReaderGroup,
                   NkvReaderRowsArgs, NkvRope,
                   NkvSegment, check, lib)

_SCALE_CODES = {torch.bfloat16: NKV_DTYPE_BF16, torch.float16: NKV_DTYPE_FP16}
_QUANT_CODES = {"fp32": NKV_QUANT_FP32, "bf16": NKV_QUANT_BF16}
_ID_BYTES = {torch.uint8: 1, torch.int16: 2, torch.int32: 4}
SCHEDULES = {"auto": NKV_SCHEDULE_AUTO, "query_tiles": NKV_SCHEDULE_QUERY_TILES,
             "key_chunks": NKV_SCHEDULE_KEY_CHUNKS}
if hasattr(torch, "uint16"):
    _ID_BYTES[torch.uint16] = 2


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("NanoKV HIP ops require GPU tensors (no CPU fallback)")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} vs {t.device}")
    if device is None:
        raise ValueError("no tensor given")
    return device


def _contig(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def id_dtype_for(num_centers: int) -> torch.dtype:
    """uint8 ids up to 256 centers (the reference's layout), else 16-bit."""
    if num_centers <= 256:
        return torch.uint8
    if num_centers <= 65536:
        return torch.int16
    return torch.int32


# ---------------------------------------------------------------- quantiser
def quant_pack(coeff: torch.Tensor, group: int, scale_dtype: torch.dtype = torch.bfloat16,
               quant_mode: str = "fp32") -> tuple[torch.Tensor, torch.Tensor]:
    """INT4 quantise + pack fp32 coefficients [..., r] (see nkv_quant_pack).

    Returns (packed uint8 [..., r/2], scales [..., r/group] of scale_dtype).
    """
    device = _require_gpu(coeff)
    _contig(coeff, torch.float32, "coeff")
    r = int(coeff.shape[-1])
    rows = coeff.numel() // r if r else 0
    if r % 2:
        raise ValueError("INT4 packing needs an even coefficient width")
    if group <= 0 or r % group:
        raise ValueError(f"group {group} must divide r={r}")
    packed = torch.empty((*coeff.shape[:-1], r // 2), device=device, dtype=torch.uint8)
    scales = torch.empty((*coeff.shape[:-1], r // group), device=device, dtype=scale_dtype)
    check("nkv_quant_pack", lib().nkv_quant_pack(
        _stream(device), coeff.data_ptr(), rows, r, group, _SCALE_CODES[scale_dtype],
        _QUANT_CODES[quant_mode], packed.data_ptr(), scales.data_ptr()))
    return packed, scales


def unpack(packed: torch.Tensor, scales: torch.Tensor, r: int, group: int,
           row_index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """bf16(code * scale) for all rows or the rows in row_index: [rows, r]."""
    device = _require_gpu(packed, scales, row_index)
    _contig(packed, torch.uint8, "packed")
    if scales.dtype not in _SCALE_CODES or not scales.is_contiguous():
        raise TypeError("scales must be a contiguous bf16 or fp16 tensor")
    src_rows = packed.numel() // (r // 2)
    if packed.numel() != src_rows * (r // 2) or scales.numel() != src_rows * (r // group):
        raise ValueError("invalid packed INT4 payload")
    if row_index is not None:
        _contig(row_index, torch.int32, "row_index")
        rows = row_index.numel()
    else:
        rows = src_rows
    out = torch.empty((rows, r), device=device, dtype=torch.bfloat16)
    check("nkv_unpack", lib().nkv_unpack(
        _stream(device), packed.data_ptr(), scales.data_ptr(), _SCALE_CODES[scales.dtype],
        _ptr(row_index), rows, r, group, out.data_ptr()))
    return out


def assign(x: torch.Tensor, centers: torch.Tensor,
           id_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Nearest bf16 center per fp32 row (fp64 decision, first index on ties)."""
    device = _require_gpu(x, centers)
    _contig(x, torch.float32, "x")
    _contig(centers, torch.bfloat16, "centers")
    hd = int(x.shape[-1])
    if centers.dim() != 2 or centers.shape[1] != hd:
        raise ValueError("centers must be [C, HD] with the rows' HD")
    C = int(centers.shape[0])
    id_dtype = id_dtype or id_dtype_for(C)
    rows = x.numel() // hd
    ids = torch.empty(x.shape[:-1], device=device, dtype=id_dtype)
    check("nkv_assign", lib().nkv_assign(_stream(device), x.data_ptr(), centers.data_ptr(), rows,
                                         C, hd, ids.data_ptr(), _ID_BYTES[id_dtype]))
    return ids


def _encode_args(x: torch.Tensor, w_enc: torch.Tensor, centers, mean, group, scale_dtype,
                 quant_mode, id_dtype, out, ids):
    """nkv_encode_args of one encode problem and its output tensors."""
    device = _require_gpu(x, w_enc, centers, mean)
    if x.dtype not in (torch.float32, torch.bfloat16) or x.dim() < 1 or x.stride(-1) != 1:
        raise ValueError("x must be fp32 or bf16 rows [..., HD] with contiguous HD")
    hd = int(x.shape[-1])
    if x.dim() == 2:
        stride = int(x.stride(0)) if x.shape[0] > 1 else hd
    elif x.is_contiguous():
        stride = hd
    else:
        raise ValueError("x must be contiguous, or a 2-D view [rows, HD] with a row stride")
    rows = x.numel() // hd if hd else 0
    _contig(w_enc, torch.bfloat16, "w_enc")
    r = int(w_enc.shape[0])
    if w_enc.shape[1] != hd:
        raise ValueError("w_enc must be [r, HD]")
    args = NkvEncodeArgs()
    args.rows, args.HD, args.r, args.group = rows, hd, r, group
    args.scale_dtype = _SCALE_CODES[scale_dtype]
    args.quant_mode = _QUANT_CODES[quant_mode]
    args.x_stride = stride
    lead = tuple(x.shape[:-1])

    def _out(name, shape, dtype):
        if out is None or out.get(name) is None:
            return torch.empty(shape, device=device, dtype=dtype)
        t = out[name]
        _contig(t, dtype, f"out[{name!r}]")
        if t.numel() != math.prod(shape) or t.device != device:
            raise ValueError(f"out[{name!r}] must hold {tuple(shape)} on {device}")
        return t

    given = ids
    ids = None
    if given is not None and centers is None:
        raise ValueError("ids need centers")
    if centers is not None:
        _contig(centers, torch.bfloat16, "centers")
        C = int(centers.shape[0])
        if given is not None:
            _require_gpu(given)
            if given.dtype not in _ID_BYTES or not given.is_contiguous() \
                    or given.numel() != rows:
                raise ValueError("ids must be a contiguous integer tensor of one id per row")
            ids, id_dtype = given, given.dtype
            args.ids_in = 1
        else:
            id_dtype = id_dtype or id_dtype_for(C)
            ids = _out("ids", lead, id_dtype)
        args.num_centers, args.id_bytes = C, _ID_BYTES[id_dtype]
        args.centers, args.ids = centers.data_ptr(), ids.data_ptr()
    if mean is not None:
        _contig(mean, torch.float32, "mean")
        args.mean = mean.data_ptr()
    coeff = _out("coeff", (*lead, r), torch.float32)
    packed = _out("packed", (*lead, r // 2), torch.uint8)
    scales = _out("scales", (*lead, r // group), scale_dtype)
    if x.dtype == torch.bfloat16:
        args.x_bf16 = x.data_ptr()
    else:
        args.x = x.data_ptr()
    args.w_enc = w_enc.data_ptr()
    args.coeff, args.packed, args.scales = coeff.data_ptr(), packed.data_ptr(), scales.data_ptr()
    return args, {"packed": packed, "scales": scales, "ids": ids, "coeff": coeff}, device


def encode(x: torch.Tensor, w_enc: torch.Tensor, *, centers: Optional[torch.Tensor] = None,
           mean: Optional[torch.Tensor] = None, group: int = 32,
           scale_dtype: torch.dtype = torch.bfloat16, quant_mode: str = "fp32",
           id_dtype: Optional[torch.dtype] = None, out: Optional[dict] = None,
           ids: Optional[torch.Tensor] = None) -> dict:
    """Encode rows [rows, HD] with given centers (see nkv_encode).

    x: fp32, or bf16 (read as value.float(), exact; needs HD % 256 == 0 and
    at most 256 centers to search); a 2-D x may be a view with a row stride.
    out: optional preallocated outputs {"packed", "scales", "ids", "coeff"}
    (contiguous, shaped like the returned ones; "ids" only with centers), so
    that a chunk can be encoded straight into a slot of a larger cache.
    ids: each row's center, given (no nearest-center search), e.g. the
    labels of a C64 fit; returned as the payload's ids."""
    args, res, device = _encode_args(x, w_enc, centers, mean, group, scale_dtype, quant_mode,
                                     id_dtype, out, ids)
    check("nkv_encode", lib().nkv_encode(_stream(device), byref(args)))
    return res


def encode_batch(problems: list, *, group: int = 32, scale_dtype: torch.dtype = torch.bfloat16,
                 quant_mode: str = "fp32") -> list:
    """Up to 8 encodes of one shape in one launch per stage (nkv_encode_batch),
    e.g. the K and V rows of a layer's chunk.  problems: dicts of encode's
    arguments (x, w_enc, and optionally centers, mean, id_dtype, out, ids);
    returns encode's result for each."""
    if not 1 <= len(problems) <= 8:
        raise ValueError("encode_batch takes 1 to 8 problems")
    built = [_encode_args(p["x"], p["w_enc"], p.get("centers"), p.get("mean"), group,
                          scale_dtype, quant_mode, p.get("id_dtype"), p.get("out"), p.get("ids"))
             for p in problems]
    arr = (NkvEncodeArgs * len(built))(*(b[0] for b in built))
    device = built[0][2]
    check("nkv_encode_batch", lib().nkv_encode_batch(_stream(device), arr, len(built)))
    return [b[1] for b in built]


# ---------------------------------------------------------------- codec view
@dataclass
class Segment:
    """Device tensors of one immutable segment of a codec cache (one payload of
    a worldplay_segments_v1 list): packed [B, rows, r/2] uint8, scales
    [B, rows, r/group] bf16/fp16, ids [B, rows] or None, centers [B or 1, C, HD]
    bf16 or None (its own table)."""
    packed: torch.Tensor
    scales: torch.Tensor
    ids: Optional[torch.Tensor] = None
    centers: Optional[torch.Tensor] = None


class SegmentTable:
    """The nkv_segment table of a list of segments: a host ctypes array (the
    library validates and plans from it) and the same bytes in device memory
    (the kernels read it).  Built once per segment list; the segments'
    tensors are kept alive with it."""

    def __init__(self, segments: list, device: torch.device):
        if not segments:
            raise ValueError("a segment table needs at least one segment")
        self.segments = list(segments)
        n = len(self.segments)
        self.host = (NkvSegment * n)()
        row, cbase = 0, 0
        with_centers = self.segments[0].centers is not None
        for i, sg in enumerate(self.segments):
            _contig(sg.packed, torch.uint8, "segment packed")
            if sg.scales.dtype not in _SCALE_CODES or not sg.scales.is_contiguous():
                raise TypeError("segment scales must be contiguous bf16 or fp16")
            if sg.packed.dim() != 3 or sg.scales.dim() != 3 or \
                    sg.scales.shape[:2] != sg.packed.shape[:2]:
                raise ValueError("segment packed/scales must be [B, rows, ...]")
            if (sg.centers is not None) != with_centers:
                raise ValueError("every segment must have a center table, or none")
            e = self.host[i]
            e.packed, e.scales = sg.packed.data_ptr(), sg.scales.data_ptr()
            e.row_start, e.rows = row, int(sg.packed.shape[1])
            if with_centers:
                _contig(sg.centers, torch.bfloat16, "segment centers")
                if sg.ids is None or sg.ids.dtype not in _ID_BYTES or not sg.ids.is_contiguous() \
                        or tuple(sg.ids.shape) != tuple(sg.packed.shape[:2]):
                    raise ValueError("segment ids must be contiguous [B, rows] integers")
                if sg.centers.dim() != 3 or sg.centers.shape[0] not in (1, sg.packed.shape[0]):
                    raise ValueError("segment centers must be [B or 1, C, HD]")
                e.ids, e.centers = sg.ids.data_ptr(), sg.centers.data_ptr()
                e.id_bytes = _ID_BYTES[sg.ids.dtype]
                e.num_centers = int(sg.centers.shape[1])
                e.centers_batch_stride = 0 if sg.centers.shape[0] == 1 else int(sg.centers.stride(0))
                e.center_base = cbase
                cbase += e.num_centers
            row += e.rows
        self.rows = row
        self.batch = int(self.segments[0].packed.shape[0])
        raw = bytes(memoryview(self.host).cast("B"))
        self.device = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(device)

    @property
    def has_centers(self) -> bool:
        return self.segments[0].centers is not None


@dataclass
class Codec:
    """Device tensors of one K or V history codec: either flat arrays of all
    rows, packed [B, N, r/2] uint8, scales [B, N, r/group] bf16/fp16, ids
    [B, N] (uint8/int16/int32) or None, centers [B or 1, C, HD] bf16 or None;
    or a SegmentTable of per-segment arrays (then packed/scales/ids/centers
    are None).  w_dec [HD, r] bf16, mean [HD] fp32 or None apply to all rows.
    """
    packed: Optional[torch.Tensor]
    scales: Optional[torch.Tensor]
    w_dec: torch.Tensor
    group: int
    ids: Optional[torch.Tensor] = None
    centers: Optional[torch.Tensor] = None
    mean: Optional[torch.Tensor] = None
    segments: Optional[SegmentTable] = None

    @property
    def r(self) -> int:
        return int(self.w_dec.shape[1])

    @property
    def batch(self) -> int:
        return self.segments.batch if self.segments is not None else int(self.packed.shape[0])

    @property
    def tokens(self) -> int:
        return self.segments.rows if self.segments is not None else int(self.packed.shape[1])

    @property
    def scale_dtype(self) -> torch.dtype:
        src = self.segments.segments[0].scales if self.segments is not None else self.scales
        return src.dtype

    def validate(self, hd: int) -> None:
        r = self.r
        _contig(self.w_dec, torch.bfloat16, "w_dec")
        if tuple(self.w_dec.shape) != (hd, r):
            raise ValueError(f"w_dec must be [HD={hd}, r={r}]")
        if self.mean is not None:
            _contig(self.mean, torch.float32, "mean")
            if self.mean.numel() != hd:
                raise ValueError("mean must have HD elements")
        if self.segments is not None:
            if self.group <= 0 or r % self.group:
                raise ValueError("group must divide r")
            for sg in self.segments.segments:
                B, rows = int(sg.packed.shape[0]), int(sg.packed.shape[1])
                if tuple(sg.packed.shape) != (B, rows, r // 2) or \
                        tuple(sg.scales.shape) != (B, rows, r // self.group) or \
                        B != self.batch or sg.scales.dtype != self.scale_dtype:
                    raise ValueError("every segment must be [B, rows, r/2] codes with "
                                     "[B, rows, r/group] scales of one dtype")
                if sg.centers is not None and sg.centers.shape[2] != hd:
                    raise ValueError("segment centers must have HD columns")
            return
        _contig(self.packed, torch.uint8, "packed")
        _contig(self.w_dec, torch.bfloat16, "w_dec")
        if self.scales.dtype not in _SCALE_CODES or not self.scales.is_contiguous():
            raise TypeError("scales must be a contiguous bf16 or fp16 tensor")
        B, N = self.batch, self.tokens
        if tuple(self.packed.shape) != (B, N, r // 2):
            raise ValueError(f"packed must be [B, N, r/2], got {tuple(self.packed.shape)}")
        if self.group <= 0 or r % self.group or tuple(self.scales.shape) != (B, N, r // self.group):
            raise ValueError("scales must be [B, N, r/group]")
        if self.centers is not None:
            _contig(self.centers, torch.bfloat16, "centers")
            if self.ids is None or self.ids.dtype not in _ID_BYTES or not self.ids.is_contiguous():
                raise TypeError("ids must be a contiguous uint8/int16/int32 tensor with centers")
            if tuple(self.ids.shape) != (B, N):
                raise ValueError("ids must be [B, N]")
            if self.centers.dim() != 3 or self.centers.shape[0] not in (1, B) or \
                    self.centers.shape[2] != hd:
                raise ValueError("centers must be [B or 1, C, HD]")

    def struct(self) -> NkvCodec:
        c = NkvCodec()
        c.w_dec = self.w_dec.data_ptr()
        c.r, c.group, c.scale_dtype = self.r, self.group, _SCALE_CODES[self.scale_dtype]
        if self.mean is not None:
            c.mean = self.mean.data_ptr()
        if self.segments is not None:
            c.n_segments = len(self.segments.segments)
            c.segments = ctypes.cast(self.segments.host, ctypes.POINTER(NkvSegment))
            c.segments_dev = self.segments.device.data_ptr()
            return c
        c.packed, c.scales = self.packed.data_ptr(), self.scales.data_ptr()
        if self.centers is not None:
            c.centers, c.ids = self.centers.data_ptr(), self.ids.data_ptr()
            c.id_bytes = _ID_BYTES[self.ids.dtype]
            c.num_centers = int(self.centers.shape[1])
            c.centers_batch_stride = (0 if self.centers.shape[0] == 1
                                      else int(self.centers.stride(0)))
        return c


def decode(codec: Codec, hd: int, row_index: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Full-width bf16 decode [B, rows, HD] of all or selected rows (a flat
    codec; the segments of a segment list are decoded one by one)."""
    if codec.segments is not None:
        raise ValueError("decode takes a flat codec; decode segments one at a time")
    device = _require_gpu(codec.packed, row_index)
    codec.validate(hd)
    args = NkvDecodeArgs()
    args.B, args.HD, args.N = codec.batch, hd, codec.tokens
    if row_index is not None:
        _contig(row_index, torch.int32, "row_index")
        args.rows, args.row_index = row_index.numel(), row_index.data_ptr()
    else:
        args.rows = codec.tokens
    args.codec = codec.struct()
    out = torch.empty((codec.batch, int(args.rows), hd), device=device, dtype=torch.bfloat16)
    args.out = out.data_ptr()
    check("nkv_decode", lib().nkv_decode(_stream(device), byref(args)))
    return out


def _strides_bthd(t: torch.Tensor, name: str) -> tuple[int, int, int]:
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError(f"{name} must be [B, T, H, D] with contiguous D")
    if t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:3]):
        raise ValueError(f"{name} must be 16-byte aligned with strides divisible by 8")
    return t.stride(0), t.stride(1), t.stride(2)


def _attend_args(q: torch.Tensor, k_cur: Optional[torch.Tensor], v_cur: Optional[torch.Tensor],
                 key: Optional[Codec], value: Optional[Codec], softmax_scale: Optional[float],
                 out: Optional[torch.Tensor], return_lse: bool):
    """Validated nkv_attend_args for [B, Q, H, D] q and [B, Nc, H, D] current K/V;
    allocates out / lse when not given."""
    device = _require_gpu(q, k_cur, v_cur)
    if q.dtype != torch.bfloat16:
        raise TypeError("q must be bf16")
    B, Qn, H, D = (int(v) for v in q.shape)
    hd = H * D
    args = NkvAttendArgs()
    args.B, args.H, args.D, args.Q = B, H, D, Qn
    args.softmax_scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    args.q = q.data_ptr()
    args.q_sb, args.q_st, args.q_sh = _strides_bthd(q, "q")
    if (key is None) != (value is None):
        raise ValueError("key and value codecs must be given together")
    if key is not None:
        key.validate(hd)
        value.validate(hd)
        if key.tokens != value.tokens or key.batch != B or value.batch != B:
            raise ValueError("key/value codec token counts or batch differ from q")
        args.N = key.tokens
        args.key, args.value = key.struct(), value.struct()
    if (k_cur is None) != (v_cur is None):
        raise ValueError("k_cur and v_cur must be given together")
    if k_cur is not None:
        for name, t in (("k_cur", k_cur), ("v_cur", v_cur)):
            if t.dtype != torch.bfloat16 or t.shape[0] != B or t.shape[2] != H or t.shape[3] != D:
                raise ValueError(f"{name} must be bf16 [B, Nc, H, D]")
        if k_cur.shape[1] != v_cur.shape[1]:
            raise ValueError("k_cur and v_cur lengths differ")
        args.Nc = int(k_cur.shape[1])
        args.k_cur, args.v_cur = k_cur.data_ptr(), v_cur.data_ptr()
        args.k_sb, args.k_st, args.k_sh = _strides_bthd(k_cur, "k_cur")
        args.v_sb, args.v_st, args.v_sh = _strides_bthd(v_cur, "v_cur")
    if out is None:
        out = torch.empty((B, Qn, H, D), device=device, dtype=torch.bfloat16)
    args.out = out.data_ptr()
    args.o_sb, args.o_st, args.o_sh = _strides_bthd(out, "out")
    lse = torch.empty((B, H, Qn), device=device, dtype=torch.float32) if return_lse else None
    args.lse = _ptr(lse)
    return args, out, lse, device


def _set_visibility(args: NkvAttendArgs, visibility: Optional[Visibility], Qn: int) -> None:
    """Point the args at a current-key visibility mask (nkv_attend_args.cur_mask)."""
    if visibility is None:
        return
    _contig(visibility.bits, torch.int32, "visibility bits")
    _contig(visibility.q_group, torch.int32, "visibility q_group")
    if visibility.bits.dim() != 2 or visibility.q_group.numel() != Qn:
        raise ValueError("visibility must be bits [groups, words] and q_group [Q]")
    if visibility.words * 32 < args.Nc:
        raise ValueError("visibility bits cover fewer keys than the current chunk holds")
    args.cur_mask, args.q_group = visibility.bits.data_ptr(), visibility.q_group.data_ptr()
    args.n_groups, args.cur_mask_words = visibility.groups, visibility.words


def _set_hist_rows(args: NkvAttendArgs, hist_rows: Optional[torch.Tensor]):
    """Point the args at a history row list (nkv_attend_args.hist_rows).  An
    empty list still needs a non-NULL pointer (NULL means every row), and an
    empty tensor's data_ptr() is 0, so it gets a one-element stand-in that is
    never read; the caller keeps the returned tensor alive over the call."""
    if hist_rows is None:
        return None
    _contig(hist_rows, torch.int32, "hist_rows")
    if hist_rows.numel() == 0:
        hist_rows = torch.zeros(1, device=hist_rows.device, dtype=torch.int32)
        args.hist_rows, args.n_hist = hist_rows.data_ptr(), 0
        return hist_rows
    args.hist_rows, args.n_hist = hist_rows.data_ptr(), int(hist_rows.numel())
    return hist_rows


def c64_fit(x: torch.Tensor, init_rows: torch.Tensor, iterations: int = 2,
            workspace: Optional[torch.Tensor] = None):
    """Per-chunk C64 center fit (nkv_c64_fit): x [B, S, HD] fp32, init_rows
    int32 [C] (the seeded permutation's first C rows).  Returns (centers
    [B, C, HD] fp32, labels [B, S] int32 of the last round)."""
    device = _require_gpu(x, init_rows)
    _contig(x, torch.float32, "x")
    _contig(init_rows, torch.int32, "init_rows")
    if x.dim() != 3:
        raise ValueError("x must be [B, S, HD]")
    B, S, HD = (int(v) for v in x.shape)
    C = int(init_rows.numel())
    centers = torch.empty((B, C, HD), device=device, dtype=torch.float32)
    labels = torch.empty((B, S), device=device, dtype=torch.int32)
    need = int(lib().nkv_c64_fit_workspace_size(B, S, C))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), device=device, dtype=torch.uint8)
    check("nkv_c64_fit", lib().nkv_c64_fit(_stream(device), x.data_ptr(), B, S, HD, C,
                                           int(iterations), init_rows.data_ptr(),
                                           centers.data_ptr(), labels.data_ptr(),
                                           workspace.data_ptr(), need))
    return centers, labels


def int8_pack(weight: torch.Tensor, group_size: int = 0) -> dict:
    """INT8 operator storage of a weight [rows, cols] (_pack_operator's int8
    mode, MG:108-131, nkv_int8_pack): per row and group of `group_size`
    columns (0: the whole row) s = max(amax, 1e-12) / 127, qweight =
    clamp(round(w / s), -127, 127) int8, scale = bf16(s) [rows, cols/group]."""
    device = _require_gpu(weight)
    if weight.dim() != 2:
        raise ValueError("weight must be [rows, cols]")
    rows, cols = (int(v) for v in weight.shape)
    group = int(group_size) or cols
    if group > cols or cols % group:
        raise ValueError(f"INT8 group size {group} must divide {cols}")
    w = weight.detach().to(torch.float32).contiguous()
    q = torch.empty((rows, cols), device=device, dtype=torch.int8)
    scale = torch.empty((rows, cols // group), device=device, dtype=torch.bfloat16)
    check("nkv_int8_pack", lib().nkv_int8_pack(_stream(device), w.data_ptr(), rows, cols, group,
                                               q.data_ptr(), scale.data_ptr()))
    return {"storage": "int8", "qweight": q, "scale": scale, "group_size": group}


def int8_dequant(packed: dict) -> torch.Tensor:
    """bf16 weight of an INT8 operator dict (qweight, scale, group_size):
    bf16(q * scale), as unpack_int8_weight (nanokv_codec_kernels.py:64-82)."""
    q, scale = packed["qweight"], packed["scale"]
    device = _require_gpu(q, scale)
    _contig(q, torch.int8, "qweight")
    _contig(scale, torch.bfloat16, "scale")
    rows, cols = (int(v) for v in q.shape)
    group = int(packed["group_size"])
    if group <= 0 or cols % group or tuple(scale.shape) != (rows, cols // group):
        raise ValueError("scale must be [rows, cols / group_size]")
    out = torch.empty((rows, cols), device=device, dtype=torch.bfloat16)
    check("nkv_int8_dequant", lib().nkv_int8_dequant(_stream(device), q.data_ptr(),
                                                     scale.data_ptr(), rows, cols, group,
                                                     out.data_ptr()))
    return out


def rope_bands(D: int, end: int = 1024, theta: float = 10000.0):
    """The temporal, row and column RoPE frequency bands of a D-wide head,
    complex128 on the CPU: t [end, pt], h [end, ph], w [end, pw] with
    ph = pw = (D // 3) // 2 and pt = D / 2 - ph - pw.  Entry [n, i] is
    exp(1j * n * theta^(-2i / dim)) for the band's width dim (the tables of
    precompute_freqs_cis_3d, wan_video_dit.py:168-182; the angles are formed
    and rounded as there, so the rotations agree to the last bit)."""
    def band(dim: int) -> torch.Tensor:
        inv = 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].double() / dim))
        angle = torch.outer(torch.arange(end), inv)
        return torch.polar(torch.ones_like(angle), angle)
    third = D // 3
    return band(D - 2 * third), band(third), band(third)


@dataclass
class Rope:
    """Read-time RoPE positions (nkv_rope) on the device: fp64 (cos, sin)
    bands cs_t [n_t, pt, 2], cs_h [grid_h, ph, 2], cs_w [grid_w, pw, 2], and
    frame_pos int32 [n_frames], the cs_t row of each frame of codec rows
    (frame f holds rows f*grid_h*grid_w .. +grid_h*grid_w, row-major)."""
    cs_t: torch.Tensor
    cs_h: torch.Tensor
    cs_w: torch.Tensor
    frame_pos: torch.Tensor
    grid_h: int
    grid_w: int

    @classmethod
    def from_bands(cls, bands, temporal_positions, grid_h: int, grid_w: int,
                   device: torch.device, disable_t: bool = False) -> "Rope":
        """Positions of frames at the given temporal positions (one per frame)
        on a grid_h x grid_w token grid, as _kv_freqs builds them
        (pipelines/wan_video.py:3322-3341).  disable_t: identity temporal band
        (prope_disable_t_rope, wan_video_dit.py:276-283)."""
        t, h, w = bands
        pos = torch.as_tensor(list(temporal_positions), dtype=torch.int64)
        if pos.numel() == 0:
            raise ValueError("RoPE needs at least one frame")
        if int(pos.min()) < 0 or int(pos.max()) >= t.shape[0]:
            raise ValueError("temporal position outside the frequency table")
        if grid_h > h.shape[0] or grid_w > w.shape[0]:
            raise ValueError("token grid larger than the frequency tables")
        used, frame_pos = torch.unique(pos, return_inverse=True)
        cs_t = torch.view_as_real(t[used]).contiguous()
        if disable_t:
            cs_t = torch.zeros_like(cs_t)
            cs_t[..., 0] = 1.0
        return cls(cs_t=cs_t.to(device), cs_h=torch.view_as_real(h[:grid_h]).contiguous().to(device),
                   cs_w=torch.view_as_real(w[:grid_w]).contiguous().to(device),
                   frame_pos=frame_pos.to(torch.int32).to(device), grid_h=int(grid_h),
                   grid_w=int(grid_w))

    @property
    def pairs(self) -> int:
        return int(self.cs_t.shape[1] + self.cs_h.shape[1] + self.cs_w.shape[1])

    @property
    def rows(self) -> int:
        """Codec rows the frames cover."""
        return int(self.frame_pos.numel()) * self.grid_h * self.grid_w

    def struct(self) -> NkvRope:
        for name in ("cs_t", "cs_h", "cs_w"):
            t = getattr(self, name)
            _contig(t, torch.float64, name)
            if t.dim() != 3 or t.shape[2] != 2:
                raise ValueError(f"{name} must be [n, pairs, 2] float64")
        _contig(self.frame_pos, torch.int32, "frame_pos")
        _require_gpu(self.cs_t, self.cs_h, self.cs_w, self.frame_pos)
        if self.cs_h.shape[0] < self.grid_h or self.cs_w.shape[0] < self.grid_w:
            raise ValueError("cs_h / cs_w have fewer rows than the token grid")
        r = NkvRope()
        r.cs_t, r.cs_h, r.cs_w = (self.cs_t.data_ptr(), self.cs_h.data_ptr(),
                                  self.cs_w.data_ptr())
        r.frame_pos, r.n_frames = self.frame_pos.data_ptr(), int(self.frame_pos.numel())
        r.n_t = int(self.cs_t.shape[0])
        r.pt, r.ph, r.pw = (int(self.cs_t.shape[1]), int(self.cs_h.shape[1]),
                            int(self.cs_w.shape[1]))
        r.grid_h, r.grid_w = self.grid_h, self.grid_w
        return r


@dataclass
class RopeTable:
    """Read-time RoPE from a per-row frequency table (nkv_rope.cs_rows): the
    reference's own per-token form, cache_freqs [rows, 1, D/2] or [rows, D/2]
    complex128 (_kv_freqs, pipelines/wan_video.py:3322-3341), stored on the
    device as fp64 (cos, sin) pairs [rows, D/2, 2]; row n of the codec (or
    query t) rotates by entry n."""
    cs_rows: torch.Tensor

    @classmethod
    def from_freqs(cls, freqs: torch.Tensor, device: torch.device) -> "RopeTable":
        f = torch.as_tensor(freqs)
        if not torch.is_complex(f):
            raise ValueError("freqs must be a complex per-row table")
        if f.dim() == 3:
            if f.shape[1] != 1:
                raise ValueError("freqs must be [rows, 1, D/2] or [rows, D/2]")
            f = f[:, 0]
        if f.dim() != 2 or f.shape[0] == 0:
            raise ValueError("freqs must be a non-empty [rows, D/2] table")
        return cls(torch.view_as_real(f.to(torch.complex128)).contiguous().to(device))

    @property
    def pairs(self) -> int:
        return int(self.cs_rows.shape[1])

    @property
    def rows(self) -> int:
        return int(self.cs_rows.shape[0])

    def struct(self) -> NkvRope:
        _contig(self.cs_rows, torch.float64, "cs_rows")
        _require_gpu(self.cs_rows)
        if self.cs_rows.dim() != 3 or self.cs_rows.shape[2] != 2:
            raise ValueError("cs_rows must be [rows, D/2, 2] float64")
        r = NkvRope()
        r.cs_rows, r.n_rows = self.cs_rows.data_ptr(), self.rows
        r.pt = self.pairs
        return r


@dataclass
class Visibility:
    """Visibility of the current keys per query group (nkv_attend_args.cur_mask):
    bits [groups, words] int32 (bit k % 32 of word k / 32: current key k is
    seen), q_group [Q] int32 (each query's group).  from_bool builds it from
    a boolean mask [Q, Nc] (True = visible, the reference's attention_lse
    mask convention, CN/core.py:45-72) by grouping identical rows, as
    attention_grouped_mask groups queries of equal visibility
    (CN/core.py:94-103)."""
    bits: torch.Tensor
    q_group: torch.Tensor

    @classmethod
    def from_bool(cls, mask: torch.Tensor, device: torch.device) -> "Visibility":
        m = torch.as_tensor(mask)
        if m.dtype != torch.bool:
            raise ValueError("Only boolean visibility masks are supported")
        if m.dim() != 2:
            raise ValueError("mask must be [Q, Nc]")
        rows, inverse = torch.unique(m.to(torch.uint8), dim=0, return_inverse=True)
        nc = int(m.shape[1])
        words = max(1, (nc + 31) // 32)
        padded = torch.zeros((rows.shape[0], words * 32), dtype=torch.int64, device=rows.device)
        padded[:, :nc] = rows.to(torch.int64)
        weights = torch.bitwise_left_shift(torch.ones(32, dtype=torch.int64, device=rows.device),
                                           torch.arange(32, device=rows.device))
        packed = (padded.view(rows.shape[0], words, 32) * weights).sum(-1)
        # two's-complement int32 view of the unsigned 32-bit words
        packed = torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)
        return cls(packed.contiguous().to(device),
                   inverse.reshape(-1).to(torch.int32).contiguous().to(device))

    @property
    def groups(self) -> int:
        return int(self.bits.shape[0])

    @property
    def words(self) -> int:
        return int(self.bits.shape[1])


def rope_apply(x: torch.Tensor, rope: Rope, rows: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RoPE of x [B, S, H, D] bf16 at the positions of codec rows rows[s]
    (int32 [S]; None: row s), as rope_apply (wan_video_dit.py:185-192) with
    the frequencies of rope (nkv_rope_apply).  out may be x."""
    device = _require_gpu(x, rows, out)
    if x.dtype != torch.bfloat16 or x.dim() != 4 or x.stride(3) != 1:
        raise ValueError("x must be bf16 [B, S, H, D] with contiguous D")
    B, S, H, D = (int(v) for v in x.shape)
    if rows is not None:
        _contig(rows, torch.int32, "rows")
        if rows.numel() != S:
            raise ValueError("rows must hold one codec row per position s")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != torch.bfloat16 or out.stride(3) != 1:
        raise ValueError("out must match x")
    r = rope.struct()
    check("nkv_rope_apply", lib().nkv_rope_apply(
        _stream(device), byref(r), B, S, H, D, x.data_ptr(), x.stride(0), x.stride(1),
        x.stride(2), _ptr(rows), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)))
    return out


CAMERA_LAYOUTS = {"full": _lib.NKV_CAMERA_FULL, "sf13": _lib.NKV_CAMERA_SF13}


@dataclass
class Camera:
    """Camera PRoPE matrices (nkv_camera) on the device: mats fp32
    [batches, n_mats, 4 sub-frames, 4, 4] (one of P, P_T, P_inv, as the role
    needs: keys and values take P_inv), frame_mat int32 [n_frames], the
    matrix set of each frame of codec rows, tokens_per_frame codec rows per
    frame; layout "full" or "sf13" (PROPE_CAMERA_LAYOUTS,
    prope_attention.py:21-24)."""
    mats: torch.Tensor
    frame_mat: torch.Tensor
    tokens_per_frame: int
    layout: str = "full"

    def struct(self) -> NkvCamera:
        _contig(self.mats, torch.float32, "mats")
        _contig(self.frame_mat, torch.int32, "frame_mat")
        _require_gpu(self.mats, self.frame_mat)
        if self.mats.dim() != 5 or tuple(self.mats.shape[2:]) != (4, 4, 4):
            raise ValueError("mats must be [batches, n_mats, 4, 4, 4] float32")
        if self.layout not in CAMERA_LAYOUTS:
            raise ValueError(f"camera layout must be one of {sorted(CAMERA_LAYOUTS)}")
        c = NkvCamera()
        c.mats = self.mats.data_ptr()
        c.mats_bs = self.mats.stride(0) if self.mats.shape[0] > 1 else 0
        c.n_mats, c.layout = int(self.mats.shape[1]), CAMERA_LAYOUTS[self.layout]
        c.frame_mat, c.n_frames = self.frame_mat.data_ptr(), int(self.frame_mat.numel())
        c.tokens_per_frame = int(self.tokens_per_frame)
        c.n_batches = int(self.mats.shape[0])
        return c


def camera_apply(x: torch.Tensor, camera: Camera, rows: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Camera transform of x [B, S, H, D] bf16 at codec rows rows[s] (int32
    [S]; None: row s) by the frame matrices of camera (nkv_camera_apply), the
    per-frame 4x4 products of _apply_tiled_projmat / _apply_contiguous_projmat
    (prope_attention.py:120-176).  out may be x."""
    device = _require_gpu(x, rows, out)
    if x.dtype != torch.bfloat16 or x.dim() != 4 or x.stride(3) != 1:
        raise ValueError("x must be bf16 [B, S, H, D] with contiguous D")
    B, S, H, D = (int(v) for v in x.shape)
    if camera.mats.shape[0] not in (1, B):
        raise ValueError("camera batch must match x or broadcast")
    if rows is not None:
        _contig(rows, torch.int32, "rows")
        if rows.numel() != S:
            raise ValueError("rows must hold one codec row per position s")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != torch.bfloat16 or out.stride(3) != 1:
        raise ValueError("out must match x")
    c = camera.struct()
    check("nkv_camera_apply", lib().nkv_camera_apply(
        _stream(device), byref(c), B, S, H, D, x.data_ptr(), x.stride(0), x.stride(1),
        x.stride(2), _ptr(rows), out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)))
    return out


def reader_rows(x: torch.Tensor, heads: torch.Tensor, w: Optional[torch.Tensor] = None, *,
                rope=None, pairs: Optional[torch.Tensor] = None,
                camera: Optional[Camera] = None, blocks: Optional[torch.Tensor] = None,
                out_width: Optional[int] = None) -> torch.Tensor:
    """Rows of x [B, S, H, D] bf16 read through a reader group
    (nkv_reader_rows): bf16(x[:, :, heads[i]] . w[i]) (w [nh, D, E] bf16;
    None: the rows themselves), rotated on the retained pairs (pairs [nh,
    E/2] int32) at row s of rope, multiplied on the 8-dim blocks (blocks
    [nh, E/8] int32 sub-frames) by row s's camera; returns [B, S, nh,
    out_width] bf16 whose columns past E are zero.  MG's low_native segment
    (mg35.py:241-249, 324-336) and the group query of that segment."""
    device = _require_gpu(x, heads, w, pairs, blocks)
    if x.dtype != torch.bfloat16 or x.dim() != 4 or x.stride(3) != 1:
        raise ValueError("x must be bf16 [B, S, H, D] with contiguous D")
    B, S, H, D = (int(v) for v in x.shape)
    _contig(heads, torch.int32, "heads")
    nh = int(heads.numel())
    E = D
    if w is not None:
        _contig(w, torch.bfloat16, "w")
        if w.dim() != 3 or tuple(w.shape[:2]) != (nh, D):
            raise ValueError("w must be bf16 [nh, D, E]")
        E = int(w.shape[2])
    W = E if out_width is None else int(out_width)
    out = torch.empty((B, S, nh, W), device=device, dtype=torch.bfloat16)
    a = NkvReaderRowsArgs()
    a.B, a.H, a.D, a.E, a.nh, a.out_width, a.S = B, H, D, E, nh, W, S
    a.x, a.x_sb, a.x_st, a.x_sh = x.data_ptr(), x.stride(0), x.stride(1), x.stride(2)
    a.heads, a.w, a.out = heads.data_ptr(), _ptr(w), out.data_ptr()
    keep = []
    if rope is not None:
        rs = rope.struct()
        keep.append(rs)
        a.rope = ctypes.pointer(rs)
        if pairs is not None:
            _contig(pairs, torch.int32, "pairs")
            if tuple(pairs.shape) != (nh, E // 2):
                raise ValueError("pairs must be int32 [nh, E/2]")
            a.pairs = pairs.data_ptr()
    if camera is not None:
        cs = camera.struct()
        keep.append(cs)
        a.camera = ctypes.pointer(cs)
        if blocks is not None:
            _contig(blocks, torch.int32, "blocks")
            if tuple(blocks.shape) != (nh, E // 8):
                raise ValueError("blocks must be int32 [nh, E/8]")
            a.blocks = blocks.data_ptr()
    check("nkv_reader_rows", lib().nkv_reader_rows(_stream(device), byref(a)))
    return out


def attend(q: torch.Tensor, k_cur: Optional[torch.Tensor], v_cur: Optional[torch.Tensor],
           key: Optional[Codec] = None, value: Optional[Codec] = None, *,
           softmax_scale: Optional[float] = None, return_lse: bool = True,
           splits: int = 0, out: Optional[torch.Tensor] = None,
           kernel_events: Optional[tuple[int, int]] = None,
           workspace: Optional[torch.Tensor] = None, schedule: str = "auto",
           rope=None, camera: Optional[Camera] = None,
           hist_rows: Optional[torch.Tensor] = None, visibility: Optional[Visibility] = None):
    """Fused decode+attention (see nkv_attend).

    q [B, Q, H, D] bf16; k_cur/v_cur [B, Nc, H, D] bf16 or None; key/value
    history codecs (both or neither).  Returns (out [B, Q, H, D] bf16,
    lse [B, H, Q] fp32 or None).  kernel_events: optional (begin, end) raw
    hipEvent_t handles recorded around the fused kernel.  workspace: optional
    preallocated uint8 buffer of at least nkv_attend_workspace_size bytes.
    schedule: "auto", "query_tiles" or "key_chunks" (nkv_schedule).
    rope: read-time RoPE of the history keys at their codec rows (q and
    k_cur are taken as already rotated); runs on the key-chunk schedule.
    camera: camera P^-1 of the decoded history keys (after rope) and values
    at their codec rows (q, k_cur and v_cur are taken as already
    transformed; the caller applies P to the output); key-chunk schedule.
    rope may be a Rope (frame bands) or a RopeTable (per-row table).
    hist_rows: int32 codec rows attended (None: all, in order).
    visibility: which current keys each query sees (None: all).
    """
    if schedule not in SCHEDULES:
        raise ValueError(f"schedule must be one of {sorted(SCHEDULES)}")
    args, out, lse, device = _attend_args(q, k_cur, v_cur, key, value, softmax_scale, out,
                                          return_lse)
    if hist_rows is not None or visibility is not None:
        _require_gpu(q, hist_rows, *(() if visibility is None else (visibility.bits,)))
    hold = _set_hist_rows(args, hist_rows)
    _set_visibility(args, visibility, int(q.shape[1]))
    args.splits = int(splits)
    args.schedule = SCHEDULES[schedule]
    rope_struct = None
    if rope is not None:
        rope_struct = rope.struct()
        args.rope = ctypes.pointer(rope_struct)
    cam_struct = None
    if camera is not None:
        if camera.mats.shape[0] not in (1, q.shape[0]):
            raise ValueError("camera batch must match q or broadcast")
        cam_struct = camera.struct()
        args.camera = ctypes.pointer(cam_struct)
    if kernel_events is not None:
        args.ev_kernel_begin, args.ev_kernel_end = kernel_events
    need = lib().nkv_attend_workspace_size(byref(args))
    err = lib().nkv_last_error().decode()
    if need == 0 and err:
        raise _lib.NanoKVError("nkv_attend_workspace_size", _lib.NKV_ERR_INVALID, err)
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, device=device, dtype=torch.uint8)
    check("nkv_attend", lib().nkv_attend(_stream(device), byref(args),
                                         _ptr(workspace) if need else None, need))
    del hold
    return out, lse


def attend_static(q: torch.Tensor, k_cur: Optional[torch.Tensor], v_cur: Optional[torch.Tensor],
                  key: Optional[Codec] = None, value: Optional[Codec] = None, *,
                  softmax_scale: Optional[float] = None, return_lse: bool = True,
                  out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                  schedule: str = "auto", hist_rows: Optional[torch.Tensor] = None,
                  visibility: Optional[Visibility] = None):
    """nkv_attend_static: attend() without any device allocation by the
    library (its scratch is a static per-GPU array of
    NKV_STATIC_SCRATCH_BYTES).  Pass out (and lse) to allocate nothing here
    either, e.g. under graph capture.  Calls that overlap on one GPU race."""
    if schedule not in SCHEDULES:
        raise ValueError(f"schedule must be one of {sorted(SCHEDULES)}")
    args, out, lse_new, device = _attend_args(q, k_cur, v_cur, key, value, softmax_scale, out,
                                              return_lse and lse is None)
    if lse is not None:
        _contig(lse, torch.float32, "lse")
        if tuple(lse.shape) != (q.shape[0], q.shape[2], q.shape[1]) or lse.device != device:
            raise ValueError("lse must be float32 [B, H, Q] on q's device")
        args.lse = lse.data_ptr()
    else:
        lse = lse_new
    args.schedule = SCHEDULES[schedule]
    if hist_rows is not None and hist_rows.numel() == 0:
        raise ValueError("an empty history row list needs attend() (it allocates a stand-in)")
    hold = _set_hist_rows(args, hist_rows)
    _set_visibility(args, visibility, int(q.shape[1]))
    check("nkv_attend_static", lib().nkv_attend_static(_stream(device), byref(args)))
    del hold
    return out, lse


@dataclass
class ReaderTensors:
    """Device tensors of one NanoKV-Fast reader group (nkv_reader_group):
    heads int32 [nh]; k_read bf16 [nh, d, rK]; v_read bf16 [nh, D, rV];
    q_reduce / k_affine bf16 [nh, D, d] and v_affine bf16 [nh, D, D], each
    None for the identity; rope_pairs int32 [nh, d/2], the original RoPE
    pair of each reader pair (None: pair j, d == D); cam_blocks int32
    [nh, d/8], the camera sub-frame of each 8-dim reader block (None: j % 4,
    d == D)."""
    heads: torch.Tensor
    d: int
    k_read: torch.Tensor
    v_read: torch.Tensor
    q_reduce: Optional[torch.Tensor] = None
    k_affine: Optional[torch.Tensor] = None
    v_affine: Optional[torch.Tensor] = None
    rope_pairs: Optional[torch.Tensor] = None
    cam_blocks: Optional[torch.Tensor] = None

    def struct(self, D: int, rK: int, rV: int) -> NkvReaderGroup:
        nh, d = int(self.heads.numel()), int(self.d)
        _contig(self.heads, torch.int32, "heads")
        expect = {"k_read": (nh, d, rK), "v_read": (nh, D, rV), "q_reduce": (nh, D, d),
                  "k_affine": (nh, D, d), "v_affine": (nh, D, D)}
        for name, shape in expect.items():
            t = getattr(self, name)
            if t is None:
                if name in ("k_read", "v_read"):
                    raise ValueError(f"{name} is required")
                continue
            _contig(t, torch.bfloat16, name)
            if tuple(t.shape) != shape:
                raise ValueError(f"bad {name} shape {tuple(t.shape)}; expected {shape}")
        g = NkvReaderGroup()
        g.num_heads, g.d, g.heads = nh, d, self.heads.data_ptr()
        g.k_read, g.v_read = self.k_read.data_ptr(), self.v_read.data_ptr()
        g.q_reduce, g.k_affine, g.v_affine = (_ptr(self.q_reduce), _ptr(self.k_affine),
                                              _ptr(self.v_affine))
        if self.rope_pairs is not None:
            _contig(self.rope_pairs, torch.int32, "rope_pairs")
            if tuple(self.rope_pairs.shape) != (nh, d // 2):
                raise ValueError(f"rope_pairs must be [{nh}, {d // 2}]")
            g.rope_pairs = self.rope_pairs.data_ptr()
        if self.cam_blocks is not None:
            _contig(self.cam_blocks, torch.int32, "cam_blocks")
            if tuple(self.cam_blocks.shape) != (nh, d // 8):
                raise ValueError(f"cam_blocks must be [{nh}, {d // 8}]")
            g.cam_blocks = self.cam_blocks.data_ptr()
        return g


def _fast_args(q, k_cur, v_cur, key, value, protect_rows, low_rows, groups, softmax_scale, out,
               return_lse, rope=None, q_pre=None, q_rope=None, camera=None, q_camera=None,
               visibility=None, low_shift=None, out_camera=None):
    args, out, lse, device = _attend_args(q, k_cur, v_cur, key, value, softmax_scale, out,
                                          return_lse)
    keep = []  # ctypes structs the call points to
    if rope is not None:
        r = rope.struct()
        keep.append(r)
        args.rope = ctypes.pointer(r)
    if camera is not None:
        if camera.mats.shape[0] not in (1, q.shape[0]):
            raise ValueError("camera batch must match q or broadcast")
        c = camera.struct()
        keep.append(c)
        args.camera = ctypes.pointer(c)
    if visibility is not None:
        _require_gpu(visibility.bits)
        _set_visibility(args, visibility, int(q.shape[1]))
    _require_gpu(protect_rows, low_rows, *[g.heads for g in groups])
    _contig(protect_rows, torch.int32, "protect_rows")
    _contig(low_rows, torch.int32, "low_rows")
    f = NkvFastArgs()
    f.attend = args
    f.protect_rows, f.n_protect = protect_rows.data_ptr(), protect_rows.numel()
    f.low_rows, f.n_low = low_rows.data_ptr(), low_rows.numel()
    D = int(q.shape[3])
    structs = (NkvReaderGroup * max(1, len(groups)))()
    for i, g in enumerate(groups):
        structs[i] = g.struct(D, key.r, value.r)
    f.num_groups = len(groups)
    f.groups = structs
    if q_pre is not None:
        _require_gpu(q_pre)
        if q_pre.dtype != torch.bfloat16 or tuple(q_pre.shape) != tuple(q.shape):
            raise ValueError("q_pre must be bf16 with q's shape [B, Q, H, D]")
        f.q_pre = q_pre.data_ptr()
        f.qp_sb, f.qp_st, f.qp_sh = _strides_bthd(q_pre, "q_pre")
    if rope is not None and q_rope is not None:
        qr = q_rope.struct()
        keep.append(qr)
        f.q_rope = ctypes.pointer(qr)
    if camera is not None and q_camera is not None:
        qc = q_camera.struct()
        keep.append(qc)
        f.q_camera = ctypes.pointer(qc)
    if out_camera is not None:
        if out_camera.mats.shape[0] not in (1, q.shape[0]):
            raise ValueError("out_camera batch must match q or broadcast")
        oc = out_camera.struct()
        keep.append(oc)
        f.o_camera = ctypes.pointer(oc)
    if low_shift is not None:
        _require_gpu(low_shift)
        B, _, H, D = (int(x) for x in q.shape)
        if low_shift.dtype != torch.float32 or tuple(low_shift.shape) != (B, H, D) or \
                low_shift.stride(2) != 1:
            raise ValueError("low_shift must be float32 [B, H, D] with unit stride in d")
        f.low_shift = low_shift.data_ptr()
        f.ls_sb, f.ls_sh = low_shift.stride(0), low_shift.stride(1)
    need = lib().nkv_fast_attend_workspace_size(byref(f))
    err = lib().nkv_last_error().decode()
    if need == 0 and err:
        raise _lib.NanoKVError("nkv_fast_attend_workspace_size", _lib.NKV_ERR_INVALID, err)
    # structs must stay alive while f points at them
    return f, (structs, keep), need, out, lse, device


def fast_attend_workspace_size(q: torch.Tensor, k_cur: Optional[torch.Tensor],
                               v_cur: Optional[torch.Tensor], key: Codec, value: Codec,
                               protect_rows: torch.Tensor, low_rows: torch.Tensor,
                               groups: list, **kw) -> int:
    """Workspace bytes nkv_fast_attend needs for this problem; kw: the
    transforms fast_attend takes (rope, q_pre, q_rope, camera, q_camera,
    visibility, low_shift, out_camera), which the workspace depends on."""
    return int(_fast_args(q, k_cur, v_cur, key, value, protect_rows, low_rows, groups, None,
                          None, False, **kw)[2])


def fast_attend(q: torch.Tensor, k_cur: Optional[torch.Tensor], v_cur: Optional[torch.Tensor],
                key: Codec, value: Codec, protect_rows: torch.Tensor, low_rows: torch.Tensor,
                groups: list, *, softmax_scale: Optional[float] = None,
                return_lse: bool = True, out: Optional[torch.Tensor] = None,
                kernel_events: Optional[tuple[int, int]] = None,
                workspace: Optional[torch.Tensor] = None, rope=None,
                q_pre: Optional[torch.Tensor] = None, q_rope=None,
                camera: Optional[Camera] = None, q_camera: Optional[Camera] = None,
                visibility: Optional[Visibility] = None,
                low_shift: Optional[torch.Tensor] = None,
                out_camera: Optional[Camera] = None):
    """NanoKV-Fast mixed-dimensional attention (see nkv_fast_attend).

    protect_rows / low_rows: int32 codec rows of the native and low
    partitions; groups: ReaderTensors covering every head once.  Returns
    (out [B, Q, H, D] bf16, lse [B, H, Q] fp32 or None).  kernel_events
    bracket the native partition's attention kernel (the one attention launch
    of every partition when they run as one staged launch).  rope: positions of the
    codec rows (history keys rotated at read); then q is the rotated query,
    q_pre [B, Q, H, D] the pre-RoPE query the reader groups project and
    q_rope the queries' positions (query t at row t).  camera: P^-1 of the
    history rows (q, k_cur, v_cur already transformed), q_camera: P^T of the
    query rows for the reader queries (then q_pre is the untransformed
    query), out_camera: P of the query rows, applied to out after the merge
    (None: the caller applies it).  visibility: which current keys each query
    sees in the native partition.  low_shift [B, H, D] fp32: the value-mean
    correction added to each head's low-partition values before the merge.
    """
    f, structs, need, out, lse, device = _fast_args(q, k_cur, v_cur, key, value, protect_rows,
                                                    low_rows, groups, softmax_scale, out,
                                                    return_lse, rope, q_pre, q_rope, camera,
                                                    q_camera, visibility, low_shift, out_camera)
    if kernel_events is not None:
        f.attend.ev_kernel_begin, f.attend.ev_kernel_end = kernel_events
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 1), device=device, dtype=torch.uint8)
    check("nkv_fast_attend", lib().nkv_fast_attend(_stream(device), byref(f), _ptr(workspace),
                                                   need))
    return out, lse


def attend_workspace_size(q: torch.Tensor, n_hist: int, n_cur: int, key: Optional[Codec],
                          value: Optional[Codec], splits: int = 0, schedule: str = "auto") -> int:
    """Workspace bytes nkv_attend needs for this problem (0 if none)."""
    B, Qn, H, D = (int(v) for v in q.shape)
    args = NkvAttendArgs()
    args.B, args.H, args.D, args.splits, args.Q, args.N, args.Nc = B, H, D, splits, Qn, n_hist, n_cur
    args.schedule = SCHEDULES[schedule]
    if key is not None:
        args.key, args.value = key.struct(), value.struct()
    args.q, args.out = q.data_ptr(), q.data_ptr()
    args.k_cur = args.v_cur = q.data_ptr()
    return int(lib().nkv_attend_workspace_size(byref(args)))


def lse_merge(a: torch.Tensor, lse_a: torch.Tensor, b: torch.Tensor, lse_b: torch.Tensor,
              out: Optional[torch.Tensor] = None):
    """Merge two attention partitions [..., D] with their LSE [...] (nkv_lse_merge)."""
    device = _require_gpu(a, lse_a, b, lse_b)
    for name, t in (("a", a), ("b", b)):
        _contig(t, torch.bfloat16, name)
    for name, t in (("lse_a", lse_a), ("lse_b", lse_b)):
        _contig(t, torch.float32, name)
    D = int(a.shape[-1])
    rows = a.numel() // D
    if b.shape != a.shape or lse_a.numel() != rows or lse_b.numel() != rows:
        raise ValueError("merge operands have mismatched shapes")
    out = torch.empty_like(a) if out is None else out
    lse = torch.empty_like(lse_a)
    check("nkv_lse_merge", lib().nkv_lse_merge(
        _stream(device), rows, D, a.data_ptr(), D, lse_a.data_ptr(), b.data_ptr(), D,
        lse_b.data_ptr(), out.data_ptr(), D, lse.data_ptr()))
    return out, lse


def lift_lse_combine(native: torch.Tensor, native_lse: torch.Tensor, low: torch.Tensor,
                     main_lift: torch.Tensor, prope_mix: torch.Tensor,
                     history_lse: torch.Tensor) -> torch.Tensor:
    """HY's two history branches lifted to D = 128 and merged into the native
    output by LSE in one write (nkv_lift_lse_combine; the reference's
    lift_lse_combine, HYP:1807-1867, with the same arguments and checks).
    native [2B, H, Q, 128], low [2B, H, Q, Dlow] (Dlow in 32/64/96): items
    0..B the Main branch (lifted by main_lift [H, Dlow, 128]), items B..2B the
    PRoPE branch (coordinate c of quartet k mixed by prope_mix [H, Dlow/4, 32]
    into output dims 4j + c); LSEs [2B, H, Q].  Returns a new contiguous
    [2B, H, Q, 128] bf16 tensor."""
    device = _require_gpu(native, native_lse, low, main_lift, prope_mix, history_lse)
    if native.ndim != 4 or native.shape[0] % 2:
        raise ValueError("native output must be [2B,H,Q,128]")
    batch, heads, queries, width = (native.shape[0] // 2, native.shape[1], native.shape[2],
                                    native.shape[3])
    if width != 128 or low.ndim != 4 or tuple(low.shape[:3]) != (2 * batch, heads, queries):
        raise ValueError("fused lift expects [2B,H,Q,Dlow] and D128 native")
    low_dim = int(low.shape[-1])
    if low_dim not in (32, 64, 96):
        raise ValueError("fused lift supports D32/D64/D96")
    if tuple(main_lift.shape) != (heads, low_dim, 128):
        raise ValueError("main lift must be [H,Dlow,128]")
    if tuple(prope_mix.shape) != (heads, low_dim // 4, 32):
        raise ValueError("PRoPE lift must be [H,Dlow/4,32]")
    if tuple(native_lse.shape) != tuple(native.shape[:-1]) or \
            tuple(history_lse.shape) != tuple(native_lse.shape):
        raise ValueError("segment LSE tensors must match [2B,H,Q]")
    for name, t in (("native", native), ("low", low)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16")
    main_lift = main_lift.to(torch.bfloat16)
    prope_mix = prope_mix.to(torch.bfloat16)
    native_lse = native_lse.float()
    history_lse = history_lse.float()
    out = torch.empty(native.shape, device=device, dtype=torch.bfloat16)
    a = NkvLiftCombineArgs()
    a.B, a.H, a.Q, a.low_dim = batch, heads, queries, low_dim
    a.native = native.data_ptr()
    a.n_sb, a.n_sh, a.n_sq, a.n_sd = native.stride()
    a.native_lse = native_lse.data_ptr()
    a.nl_sb, a.nl_sh, a.nl_sq = native_lse.stride()
    a.low = low.data_ptr()
    a.l_sb, a.l_sh, a.l_sq, a.l_sd = low.stride()
    a.main_lift = main_lift.data_ptr()
    a.ml_sh, a.ml_sk, a.ml_so = main_lift.stride()
    a.prope_mix = prope_mix.data_ptr()
    a.pm_sh, a.pm_sk, a.pm_so = prope_mix.stride()
    a.history_lse = history_lse.data_ptr()
    a.hl_sb, a.hl_sh, a.hl_sq = history_lse.stride()
    a.out = out.data_ptr()
    check("nkv_lift_lse_combine", lib().nkv_lift_lse_combine(_stream(device), byref(a)))
    return out


def lse_combine_split(native: torch.Tensor, native_lse: torch.Tensor, main: torch.Tensor,
                      prope: torch.Tensor, history_lse: torch.Tensor) -> torch.Tensor:
    """HY's merge of already lifted history halves (the reference's
    lse_combine_split, HYP:1768-1804): items 0..B of native merge with main
    [B, H, Q, D], items B..2B with prope, by their LSEs [2B, H, Q]
    (nkv_lse_merge over each half).  Returns a new contiguous tensor."""
    _require_gpu(native, native_lse, main, prope, history_lse)
    if native.ndim != 4 or native.shape[0] % 2:
        raise ValueError("native output must be [2B,H,Q,D]")
    batch = native.shape[0] // 2
    expected = (batch, *native.shape[1:])
    if tuple(main.shape) != expected or tuple(prope.shape) != expected:
        raise ValueError("split history outputs must each be [B,H,Q,D]")
    if tuple(native_lse.shape) != tuple(native.shape[:-1]) or \
            tuple(history_lse.shape) != tuple(native_lse.shape):
        raise ValueError("segment LSE tensors must match [2B,H,Q]")
    out = torch.empty(native.shape, device=native.device, dtype=torch.bfloat16)
    for half, hist in ((slice(0, batch), main), (slice(batch, 2 * batch), prope)):
        lse_merge(native[half].to(torch.bfloat16).contiguous(),
                  native_lse[half].float().contiguous(),
                  hist.to(torch.bfloat16).contiguous(), history_lse[half].float().contiguous(),
                  out=out[half])
    return out


def finish(native: torch.Tensor, native_lse: torch.Tensor, lifted: torch.Tensor,
           low_lse: torch.Tensor, heads: torch.Tensor, result: torch.Tensor,
           mean: Optional[torch.Tensor] = None, projected: Optional[torch.Tensor] = None):
    """LingBot's finish of one reader group (nkv_finish; the reference's
    finish, LBF:36-46, with the same arguments): merge lifted [B, h, S, D]
    (LSE low_lse [B, h, S]) into native [B, Hn, S, D] (native_lse [B, Hn, S])
    at native heads heads[g] and write the rows to result [B, Hn, S, D]; with
    mean [B, Hn, 1, D] and projected [B, h, 1, D] (fp32) the lifted values are
    first corrected by + mean - projected.  Returns result."""
    device = _require_gpu(native, native_lse, lifted, low_lse, heads, result)
    correct = mean is not None
    if correct != (projected is not None):
        raise ValueError("mean and projected come together")
    if native.ndim != 4 or lifted.ndim != 4 or result.shape != native.shape:
        raise ValueError("native, lifted and result must be [B,H,S,D]")
    b, h, s, d = (int(x) for x in lifted.shape)
    if native.shape[0] != b or native.shape[2] != s or native.shape[3] != d:
        raise ValueError("lifted must match native in batch, rows and width")
    if tuple(low_lse.shape) != (b, h, s) or tuple(native_lse.shape) != tuple(native.shape[:3]):
        raise ValueError("LSE shapes must be [B,H,S]")
    if heads.numel() != h:
        raise ValueError("one native head per group head")
    for name, t in (("native", native), ("result", result)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16")
    lifted = lifted.to(torch.bfloat16)
    native_lse = native_lse.float()
    low_lse = low_lse.float()
    heads32 = heads.to(device=device, dtype=torch.int32).contiguous()
    a = NkvFinishArgs()
    a.B, a.H_native, a.H_group, a.S, a.D = b, int(native.shape[1]), h, s, d
    a.native = native.data_ptr()
    a.a_sb, a.a_sh, a.a_ss, a.a_sd = native.stride()
    a.native_lse = native_lse.data_ptr()
    a.la_sb, a.la_sh, a.la_ss = native_lse.stride()
    a.lifted = lifted.data_ptr()
    a.b_sb, a.b_sh, a.b_ss, a.b_sd = lifted.stride()
    a.low_lse = low_lse.data_ptr()
    a.lb_sb, a.lb_sh, a.lb_ss = low_lse.stride()
    a.heads = heads32.data_ptr()
    if correct:
        mean = mean.float()
        projected = projected.float()
        if mean.ndim != 4 or projected.ndim != 4 or mean.shape[3] != d or projected.shape[3] != d:
            raise ValueError("mean and projected must be [B,H,1,D]")
        a.mean = mean.data_ptr()
        a.m_sb, a.m_sh, a.m_sd = mean.stride(0), mean.stride(1), mean.stride(3)
        a.projected = projected.data_ptr()
        a.p_sb, a.p_sh, a.p_sd = projected.stride(0), projected.stride(1), projected.stride(3)
    a.result = result.data_ptr()
    a.y_sb, a.y_sh, a.y_ss, a.y_sd = result.stride()
    check("nkv_finish", lib().nkv_finish(_stream(device), byref(a)))
    return result
