"""CPU oracle for NanoKV's codec-native historical attention.

TEST INFRASTRUCTURE ONLY.  This module is the checker the HIP product path is
compared against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py import it; the product package never imports it and has no
CPU fallback.

It restates the reference algorithm (paths relative to the NanoKV tree;
MG = models/Matrix-Game-3.5/fast/diffsynth/models/nanokv_codec.py,
CN = models/Matrix-Game-3.5/fast/codec_native) in plain C (nkv_oracle.c, for
the integer/byte and rounding-sensitive steps) and numpy float64 (GEMMs and
softmax attention).

Pinning (the independent check that fixes each function; see tests/):
  f32<->bf16/fp16 conversion  exhaustive comparison against torch's own
                               .to(bfloat16/float16) and numpy float16 over
                               all bf16 bit patterns and random/edge floats
                               (tests/test_oracle.py::test_conversions_*)
  quant_pack                  hand-computed known answers incl. RNE half
                               ties, zero rows, fp16 overflow/underflow;
                               brute-force search of the nearest code
                               (argmin over all 15 codes, ties to even) on
                               random data; committed golden fixtures
  pack / unpack_codes         hand-computed bytes; round trip over all codes
  c64_fit                     labels against exact rational distances on
                               small inputs; the update against the closed-form
                               mean of each cluster; 0 rounds = the drawn rows;
                               the reference's torch loop (fp32 bmm, one-hot
                               mean) on the CPU agrees (labels equal, centers
                               to fp32 rounding)
  int8_pack / int8_dequant    brute-force nearest code per weight (ties to
                               even); hand KATs (zero rows, exact multiples,
                               the 1e-12 floor); torch's tensor ops of
                               _pack_operator and of the bf16 dequant product
  unpack_latent               torch: codes.float() * scale.float() -> bf16
                               (MG:429-434) computed by torch, not by the oracle
  assign                      brute force with exact rational arithmetic
                               (fractions.Fraction) on small inputs; exact
                               tie cases; golden fixtures
  residual_bf16 / project     torch float64 reference of x - c - mean and
                               the matmul (independent library routine)
  decode (epilogue)           torch bf16 tensor ops reproducing MG:438-454
                               (F.linear with bf16 bias, add_ of fp32 gather)
  attention                   torch.nn.functional.scaled_dot_product_attention
                               in float64 (library routine), plus the LSE
                               closed form on tiny inputs
  merge                       invariant merge(attend(K1), attend(K2)) ==
                               attend(K1 u K2); closed forms for empty (-inf)
                               partitions (CN/core.py:33-42)
  protected_frames            hand-computed policy tables and an exhaustive
                               comparison with an independent set-based
                               statement (CN/metadata_cache.py:48-72) for all
                               small (count, recent, stride, sink)
  hybrid_attention            identity readers reduce it exactly to the full
                               decode-then-attend path (CN/reader_tools.py:7-35)
  rope_bands / kv_freqs       the closed form exp(1j * n * theta^(-2i/dim))
                               element by element against torch.polar; band
                               widths for several D; position 0 = identity;
                               the layout against a hand-built token
  rope_apply                  the RoPE identities in fp64: every pair keeps its
                               norm, rotations compose (angle addition), the
                               score q(m) . k(n) depends only on n - m; torch's
                               view_as_complex product (the reference's form)
                               agrees after rounding to bf16
  camera_vectors / camera_apply  the reference's rearrange + einsum of both
                               layouts (prope_attention.py:120-176) in fp64
                               on bf16-rounded matrices, element for element;
                               identity matrices leave x unchanged; a
                               permutation matrix moves dims exactly; P then
                               P^-1 returns x to bf16 rounding
  camera_blocks_apply         camera_selected's einsum "bhfgij,bhftgjr->
                               bhftgir" (CN/core.py:134-137) in fp64 on
                               bf16-rounded matrices; block sub-frames j % 4
                               at width 128 equal camera_apply's full layout
  attention (mask)            torch SDPA with a boolean attn_mask in fp64 for
                               rows that see a key; the closed form (0, -inf)
                               of the reference's blockwise path for rows that
                               see none (CN/core.py:57-72); an all-True mask
                               equals no mask
  lift_lse_combine            the union invariant in fp64: merging the native
                               partition with a lifted low partition equals one
                               softmax over both key sets with the low values
                               lifted (V_low L); the PRoPE mix equals the Main
                               lift by the matrix L[4k+c, 4j+c] = mix[k, j]
  finish                      equals merge() of the native and lifted rows at
                               the group's heads (other heads untouched); the
                               correction equals merging lifted + mean -
                               projected; mean = projected changes nothing
"""
from __future__ import annotations

import ctypes
import math
import subprocess
from ctypes import c_int, c_int64, c_void_p
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libnkv_oracle.so"

_lib = None


def build() -> Path:
    """Compile nkv_oracle.c with the Makefile next to this file."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        l.nkvo_quant_pack.argtypes = [c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p,
                                      c_void_p, c_void_p]
        l.nkvo_unpack_codes.argtypes = [c_void_p, c_int64, c_void_p]
        l.nkvo_unpack_latent.argtypes = [c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int,
                                         c_int, c_void_p]
        l.nkvo_assign.argtypes = [c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p]
        l.nkvo_residual_bf16.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int,
                                         c_void_p]
        l.nkvo_decode_epilogue.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                           c_int, c_void_p]
        for name in ("nkvo_round_bf16", "nkvo_round_f16"):
            getattr(l, name).argtypes = [c_void_p, c_int64, c_void_p]
        for name in ("nkvo_widen_bf16", "nkvo_widen_f16"):
            getattr(l, name).argtypes = [c_void_p, c_int64, c_void_p]
        l.nkvo_int8_pack.argtypes = [c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p]
        l.nkvo_int8_dequant.argtypes = [c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p]
        _lib = l
    return _lib


def _p(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


SCALE_DTYPES = {"bf16": 0, "fp16": 1}
QUANT_MODES = {"fp32": 0, "bf16": 1}


# ----------------------------------------------------------------- numbers
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().nkvo_round_bf16(_p(x), x.size, _p(out))
    return out


def bf16_to_f32(b) -> np.ndarray:
    b = _c(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().nkvo_round_f16(_p(x), x.size, _p(out))
    return out


def f16_to_f32(b) -> np.ndarray:
    b = _c(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().nkvo_widen_f16(_p(b), b.size, _p(out))
    return out


def scale_to_f32(bits, scale_dtype: str) -> np.ndarray:
    return f16_to_f32(bits) if scale_dtype == "fp16" else bf16_to_f32(bits)


# ----------------------------------------------------------------- a4/a5
def c64_fit(x, init_rows, iterations: int = 2):
    """The C64 center fit of semantic_residual (MG:301-330): centers start as
    rows init_rows of each batch item; each round labels every row with the
    center minimising ||c||^2 - 2 x.c in fp64 (first index on ties) and sets
    every center that has rows to fp32(fp64 sum in row order) / count
    (fp32); a center without rows keeps its value.  x [B, S, HD] float32.
    Returns (centers [B, C, HD] float32, labels [B, S] int64 of the last
    round; zeros for 0 rounds)."""
    x = _c(x, np.float32)
    B, S, HD = x.shape
    init = np.asarray(init_rows, np.int64)
    centers = x[:, init].copy()
    C = centers.shape[1]
    labels = np.zeros((B, S), np.int64)
    x64 = x.astype(np.float64)
    for _ in range(iterations):
        for b in range(B):
            c64 = centers[b].astype(np.float64)
            d = (c64 * c64).sum(1)[None, :] - 2.0 * (x64[b] @ c64.T)
            labels[b] = np.argmin(d, axis=1)
        for b in range(B):
            for c in range(C):
                rows = np.nonzero(labels[b] == c)[0]
                if rows.size:
                    total = np.cumsum(x64[b][rows], axis=0)[-1].astype(np.float32)
                    centers[b, c] = total / np.float32(rows.size)
    return centers, labels


def int8_pack(w, group: int = 0):
    """INT8 operator storage (_pack_operator, MG:108-131): w [rows, cols]
    float32 in groups of `group` columns (0: the whole row).  Returns
    (qweight int8 [rows, cols], scale uint16 bf16 bits [rows, cols/group])."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    group = group or cols
    if cols % group:
        raise ValueError("group must divide cols")
    q = np.zeros((rows, cols), np.int8)
    scale = np.zeros((rows, cols // group), np.uint16)
    lib().nkvo_int8_pack(_p(w), rows, cols, group, _p(q), _p(scale))
    return q, scale


def int8_dequant(q, scale, group: int) -> np.ndarray:
    """bf16(q * scale) (unpack_int8_weight, nanokv_codec_kernels.py:64-82) ->
    bf16 bits [rows, cols]."""
    q = _c(q, np.int8)
    scale = _c(scale, np.uint16)
    out = np.zeros(q.shape, np.uint16)
    lib().nkvo_int8_dequant(_p(q), _p(scale), q.shape[0], q.shape[1], group, _p(out))
    return out


def quant_pack(coeff, group: int, scale_dtype: str = "bf16", quant_mode: str = "fp32"):
    """INT4 quantise + pack (MG:349-351, 282-292; HY kv_codecs.py:237-255).

    Returns (packed uint8 [rows, r/2], scales uint16 bits [rows, r/group],
    codes int8 [rows, r]).
    """
    coeff = _c(coeff, np.float32)
    r = coeff.shape[-1]
    rows = coeff.size // r
    if r % 2 or r % group:
        raise ValueError("r must be even and divisible by group")
    packed = np.zeros((rows, r // 2), np.uint8)
    scales = np.zeros((rows, r // group), np.uint16)
    codes = np.zeros((rows, r), np.int8)
    lib().nkvo_quant_pack(_p(coeff), rows, r, group, SCALE_DTYPES[scale_dtype],
                          QUANT_MODES[quant_mode], _p(packed), _p(scales), _p(codes))
    lead = coeff.shape[:-1]
    return (packed.reshape(*lead, r // 2), scales.reshape(*lead, r // group),
            codes.reshape(*lead, r))


def pack_codes(codes) -> np.ndarray:
    """_pack_int4 (MG:282-292): (c[2j]+7) | (c[2j+1]+7) << 4 over the flat codes."""
    flat = _c(codes, np.int8).reshape(-1).astype(np.int16) + 7
    if flat.min(initial=0) < 0 or flat.max(initial=0) >= 16:
        raise RuntimeError("INT4 codes outside frozen symmetric range [-7,7]")
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, np.int16)])
    pairs = flat.reshape(-1, 2)
    return (pairs[:, 0] | (pairs[:, 1] << 4)).astype(np.uint8)


def unpack_codes(packed, count: int) -> np.ndarray:
    """_unpack_int4 (MG:295-298)."""
    packed = _c(packed, np.uint8).reshape(-1)
    out = np.empty(count, np.int8)
    lib().nkvo_unpack_codes(_p(packed), count, _p(out))
    return out


def unpack_latent(packed, scales, r: int, group: int, scale_dtype: str = "bf16",
                  row_index=None) -> np.ndarray:
    """bf16(code * stored scale) (MG:426-434; nanokv_codec_kernels.py:11-27)."""
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint16)
    idx = None if row_index is None else _c(row_index, np.int32)
    rows = (packed.size // (r // 2)) if idx is None else idx.size
    out = np.empty((rows, r), np.uint16)
    lib().nkvo_unpack_latent(_p(packed), _p(scales), SCALE_DTYPES[scale_dtype], _p(idx), rows,
                             r, group, _p(out))
    return out


# ----------------------------------------------------------------- a1
def assign(x, centers_bf16) -> np.ndarray:
    """argmin_c ||x - c||^2 decided in fp64, first index on ties (MG:315-321)."""
    x = _c(x, np.float32)
    centers_bf16 = _c(centers_bf16, np.uint16)
    hd = x.shape[-1]
    rows = x.size // hd
    C = centers_bf16.shape[0]
    ids = np.empty(rows, np.int32)
    lib().nkvo_assign(_p(x), _p(centers_bf16), rows, C, hd, _p(ids))
    return ids.reshape(x.shape[:-1])


def residual_bf16(x, centers_bf16, ids, mean) -> np.ndarray:
    """bf16(x - fp32(center[id]) - mean) (MG:326-330, 346, 138-141)."""
    x = _c(x, np.float32)
    hd = x.shape[-1]
    rows = x.size // hd
    out = np.empty(x.shape, np.uint16)
    c = None if centers_bf16 is None else _c(centers_bf16, np.uint16)
    i = None if ids is None else _c(ids, np.int32)
    m = None if mean is None else _c(mean, np.float32)
    lib().nkvo_residual_bf16(_p(x), _p(c), _p(i), _p(m), rows, hd, _p(out))
    return out


def project(rows_bf16, w_bf16, dtype=np.float64) -> np.ndarray:
    """rows @ w^T with bf16 operands, accumulated in `dtype` (fp64 by default),
    returned as fp32."""
    a = bf16_to_f32(rows_bf16).astype(dtype, copy=False)
    w = bf16_to_f32(w_bf16).astype(dtype, copy=False)
    return np.matmul(a, w.T).astype(np.float32, copy=False)


def encode(x, w_enc_bf16, centers_bf16=None, mean=None, group: int = 32,
           scale_dtype: str = "bf16", quant_mode: str = "fp32") -> dict:
    """encode_tensor (MG:333-365) with given shared centers."""
    x = _c(x, np.float32)
    ids = None if centers_bf16 is None else assign(x, centers_bf16)
    res = residual_bf16(x, centers_bf16, ids, mean)
    coeff = project(res, w_enc_bf16)
    packed, scales, codes = quant_pack(coeff, group, scale_dtype, quant_mode)
    return {"packed": packed, "scales": scales, "codes": codes, "ids": ids, "coeff": coeff}


# ----------------------------------------------------------------- a7/a8
def decode(packed, scales, w_dec_bf16, group: int, scale_dtype: str = "bf16", ids=None,
           centers_bf16=None, mean=None, row_index=None, columns=None,
           dtype=np.float64) -> np.ndarray:
    """Full-width decode of one batch item's rows (MG:393-455) -> bf16 bits.

    rows = bf16(bf16(latent @ W^T + bf16(mean)) + center[id]).  The GEMM is
    accumulated in `dtype` (fp64 by default) and rounded once to fp32.
    `columns` (optional index array) restricts the output to those HD columns.
    """
    w = _c(w_dec_bf16, np.uint16)
    r = w.shape[1]
    latent = unpack_latent(packed, scales, r, group, scale_dtype, row_index)
    if columns is not None:
        w = w[np.asarray(columns)]
    acc = np.ascontiguousarray(project(latent, w, dtype))
    hd = w.shape[0]
    cent = None
    if centers_bf16 is not None:
        cent = _c(centers_bf16, np.uint16)
        if columns is not None:
            cent = np.ascontiguousarray(cent[:, np.asarray(columns)])
    src_ids = None
    if ids is not None:
        src_ids = np.asarray(ids, np.int64)
        if row_index is not None:
            src_ids = src_ids[np.asarray(row_index)]
        src_ids = _c(src_ids, np.int32)
    m = None
    if mean is not None:
        m = _c(mean, np.float32)
        if columns is not None:
            m = np.ascontiguousarray(m[np.asarray(columns)])
    out = np.empty((acc.shape[0], hd), np.uint16)
    lib().nkvo_decode_epilogue(_p(acc), _p(m), _p(cent), _p(src_ids), acc.shape[0], hd, _p(out))
    return out


# ----------------------------------------------------------------- a10-a12
def attention(q, k, v, scale: float, dtype=np.float64, mask=None):
    """softmax(q k^T * scale) v per head (wan_video_dit.py:42-82), computed in
    `dtype` (float64 by default).

    q [H, Q, D], k/v [H, N, D] (float arrays).  Returns (out [H, Q, D],
    lse [H, Q] natural log).  An empty key set gives (0, -inf) as
    attention_lse does (CN/core.py:48-49).  mask [Q, N] bool (True =
    visible, CN/core.py:45-72, shared by the heads): hidden keys get logit
    -inf; a row that sees no key gives (0, -inf), as the reference's
    blockwise path does (its origin is 0 and every probability 0).
    """
    q = np.asarray(q, dtype)
    k = np.asarray(k, dtype)
    v = np.asarray(v, dtype)
    H, Qn, _ = q.shape
    if k.shape[1] == 0:
        return np.zeros((H, Qn, v.shape[2]), dtype), np.full((H, Qn), -np.inf, dtype)
    s = np.matmul(q, k.transpose(0, 2, 1))
    s *= dtype(scale)
    if mask is not None:
        s = np.where(np.asarray(mask, bool)[None], s, -np.inf)
    m = s.max(-1, keepdims=True)
    empty = ~np.isfinite(m)
    m = np.where(empty, 0.0, m)
    s -= m
    np.exp(s, out=s)
    l = s.sum(-1, keepdims=True)
    s /= np.where(empty, 1.0, l)
    out = np.matmul(s, v)
    with np.errstate(divide="ignore"):
        lse = np.where(empty, -np.inf, m + np.log(np.where(empty, 1.0, l)))
    return out, lse[..., 0]


def merge(out_a, lse_a, out_b, lse_b):
    """LSE merge (CN/core.py:33-42)."""
    lse_a = np.asarray(lse_a, np.float64)
    lse_b = np.asarray(lse_b, np.float64)
    lse = np.logaddexp(lse_a, lse_b)
    origin = np.where(np.isfinite(lse), lse, 0.0)
    wa = np.exp(lse_a - origin)
    wb = np.exp(lse_b - origin)
    out = np.asarray(out_a, np.float64) * wa[..., None] + np.asarray(out_b, np.float64) * wb[..., None]
    return out, lse


def lift_lse_combine(native, native_lse, low, main_lift, prope_mix, history_lse):
    """HY's value lift of its two history branches fused with the LSE merge
    (models/HY-WorldPlay/fast/hyvideo/models/transformers/modules/
    codec_native_position_triton.py:883-1014, wrapper :1807-1867), in fp64.
    native [2B, H, Q, 128] and low [2B, H, Q, Dlow] as floats (the bf16
    values), lifts [H, Dlow, 128] / [H, Dlow/4, 32], LSEs [2B, H, Q].  Items
    0..B lift by main_lift, items B..2B by the quartet mix (output dim 4j + c
    takes coordinate c of every quartet k of the low row)."""
    native = np.asarray(native, np.float64)
    low = np.asarray(low, np.float64)
    main_lift = np.asarray(main_lift, np.float64)
    prope_mix = np.asarray(prope_mix, np.float64)
    B = native.shape[0] // 2
    H, Q, K = low.shape[1], low.shape[2], low.shape[3]
    hist = np.empty(native.shape, np.float64)
    hist[:B] = np.einsum("bhqk,hko->bhqo", low[:B], main_lift)
    quart = low[B:].reshape(B, H, Q, K // 4, 4)               # [..., k, c]
    mixed = np.einsum("bhqkc,hkj->bhqjc", quart, prope_mix)   # [..., j, c]
    hist[B:] = mixed.reshape(B, H, Q, 128)                    # dim 4j + c
    a = np.asarray(native_lse, np.float64)
    b = np.asarray(history_lse, np.float64)
    m = np.maximum(a, b)
    wa, wb = np.exp(a - m)[..., None], np.exp(b - m)[..., None]
    return (native * wa + hist * wb) / (wa + wb)


def finish(native, native_lse, lifted, low_lse, heads, result, mean=None, projected=None):
    """LingBot's finish of one reader group (models/LingBot-World-2.0/fast/wan/
    modules/codec_native_finish_triton.py:10-46), in fp64: result (a copy, as
    floats) with the rows of native head heads[g] replaced by the LSE merge of
    native and lifted[:, g] (+ mean[:, heads[g]] - projected[:, g] when given)."""
    native = np.asarray(native, np.float64)
    lifted = np.asarray(lifted, np.float64)
    out = np.array(result, np.float64)
    x_all = np.asarray(native_lse, np.float64)
    z_all = np.asarray(low_lse, np.float64)
    for g, hd in enumerate(np.asarray(heads).tolist()):
        x, z = x_all[:, hd], z_all[:, g]
        with np.errstate(invalid="ignore"):
            l = np.maximum(x, z) + np.log1p(np.exp(-np.abs(x - z)))
        l = np.where((x == z) & np.isinf(x), x, l)
        origin = np.where(np.isinf(l), 0.0, l)
        v = lifted[:, g]
        if mean is not None:
            v = (v + np.asarray(mean, np.float64)[:, hd]) - np.asarray(projected, np.float64)[:, g]
        out[:, hd] = native[:, hd] * np.exp(x - origin)[..., None] + v * np.exp(z - origin)[..., None]
    return out


def decode_attend(q_bf16, k_cur_bf16, v_cur_bf16, key: Optional[dict], value: Optional[dict],
                  scale: float, heads: Optional[Sequence[int]] = None, D: int = 128,
                  dtype=np.float64, key_freqs: Optional[np.ndarray] = None,
                  key_cam: Optional[tuple] = None, hist_rows=None, cur_mask=None):
    """Reference decode-then-SDPA path for one batch item.

    q [Q, H, D] bf16 bits; k_cur/v_cur [Nc, H, D] bf16 bits or None; key/value
    are dicts with the decode() keyword arguments (packed, scales, w_dec_bf16,
    group, scale_dtype, ids, centers_bf16, mean) or None.  Returns
    (out [Q, H', D], lse [H', Q]) for the selected heads, computed in `dtype`
    (float64 for parity checks; float32 is the reference's CPU arithmetic).
    key_freqs [N, D/2] complex128: read-time RoPE of the decoded history keys
    (wan_video_dit.py:538-546), applied before attention.
    key_cam (mats [N, 4, 4, 4] fp32, layout): camera P^-1 of the decoded
    history keys (after RoPE) and values at their rows (camera_apply).
    hist_rows: the codec rows attended (the history filter of
    wan_video_dit.py:509-530), in order; key_freqs and key_cam stay indexed
    by codec row.  cur_mask [Q, Nc] bool: which current keys each query sees
    (the history is visible to every query).
    """
    q = bf16_to_f32(q_bf16)
    Qn, H = q.shape[0], q.shape[1]
    heads = list(range(H)) if heads is None else list(heads)
    cols = np.concatenate([np.arange(h * D, (h + 1) * D) for h in heads])
    ks, vs = [], []
    n_hist = 0
    if key is not None:
        rows = None if hist_rows is None else np.asarray(hist_rows, np.int64)
        kbits = decode(**key, row_index=rows, columns=cols, dtype=dtype)
        if key_freqs is not None:
            kf = key_freqs if rows is None else key_freqs[rows]
            kbits = rope_apply(kbits.reshape(-1, len(heads), D), kf)
        vbits = decode(**value, row_index=rows, columns=cols, dtype=dtype)
        if key_cam is not None:
            mats = key_cam[0] if rows is None else np.asarray(key_cam[0])[rows]
            kbits = camera_apply(kbits.reshape(-1, len(heads), D), mats, *key_cam[1:])
            vbits = camera_apply(vbits.reshape(-1, len(heads), D), mats, *key_cam[1:])
        kd = bf16_to_f32(kbits)
        vd = bf16_to_f32(vbits)
        ks.append(kd.reshape(-1, len(heads), D))
        vs.append(vd.reshape(-1, len(heads), D))
        n_hist = ks[0].shape[0]
    n_cur = 0
    if k_cur_bf16 is not None:
        ks.append(bf16_to_f32(k_cur_bf16)[:, heads])
        vs.append(bf16_to_f32(v_cur_bf16)[:, heads])
        n_cur = ks[-1].shape[0]
    if ks:
        k = np.concatenate(ks, 0).transpose(1, 0, 2)
        v = np.concatenate(vs, 0).transpose(1, 0, 2)
    else:
        k = np.zeros((len(heads), 0, D))
        v = np.zeros((len(heads), 0, D))
    mask = None
    if cur_mask is not None and n_cur:
        mask = np.concatenate([np.ones((Qn, n_hist), bool), np.asarray(cur_mask, bool)], 1)
    out, lse = attention(q[:, heads].transpose(1, 0, 2), k, v, scale, dtype, mask=mask)
    return out.transpose(1, 0, 2), lse


# ------------------------------------------------------------------- RoPE
def rope_bands(D: int, end: int, theta: float = 10000.0):
    """precompute_freqs_cis_3d (wan_video_dit.py:168-182): the temporal, row
    and column bands of a D-wide head as complex128 [end, pairs]; row n of a
    band of width dim is exp(1j * n * theta^(-2i/dim)), i < dim / 2
    (precompute_freqs_cis, wan_video_dit.py:177-182)."""
    def band(dim):
        inv = 1.0 / (theta ** (np.arange(0, dim, 2)[: dim // 2].astype(np.float64) / dim))
        ang = np.outer(np.arange(end, dtype=np.float64), inv)
        return np.cos(ang) + 1j * np.sin(ang)
    third = D // 3
    return band(D - 2 * third), band(third), band(third)


def kv_freqs(bands, temporal_positions, grid_h: int, grid_w: int) -> np.ndarray:
    """_kv_freqs (pipelines/wan_video.py:3322-3341): per-token frequencies
    [frames * grid_h * grid_w, pairs] complex128, frame-major, then row, then
    column: [t[p], h[row], w[col]] concatenated over the pair axis."""
    t, h, w = bands
    parts = []
    for p in temporal_positions:
        tt = np.broadcast_to(t[int(p)], (grid_h, grid_w, t.shape[1]))
        hh = np.broadcast_to(h[:grid_h, None, :], (grid_h, grid_w, h.shape[1]))
        ww = np.broadcast_to(w[None, :grid_w, :], (grid_h, grid_w, w.shape[1]))
        parts.append(np.concatenate([tt, hh, ww], axis=-1).reshape(grid_h * grid_w, -1))
    return np.concatenate(parts, 0)


def rope_rotate(x, freqs) -> np.ndarray:
    """The fp64 rotation of rope_apply (wan_video_dit.py:185-192) before the
    cast: x [S, H, D] (bf16 bits or float) times freqs [S, D/2] per complex
    pair (2i, 2i+1), each product and sum rounded separately."""
    x = np.asarray(x)
    xf = bf16_to_f32(x).astype(np.float64) if x.dtype == np.uint16 else x.astype(np.float64)
    a, b = xf[..., 0::2], xf[..., 1::2]
    c = np.real(freqs)[:, None, :]
    s = np.imag(freqs)[:, None, :]
    y = np.empty_like(xf)
    y[..., 0::2] = a * c - b * s
    y[..., 1::2] = a * s + b * c
    return y


def rope_apply(x_bf16, freqs) -> np.ndarray:
    """rope_apply (wan_video_dit.py:185-192): bf16 bits [S, H, D] rotated in
    fp64 and cast back (float64 -> float32 -> bfloat16, torch's cast)."""
    return f32_to_bf16(rope_rotate(x_bf16, freqs).astype(np.float32))


# ------------------------------------------------------------ camera PRoPE
def camera_vectors(layout: str, D: int):
    """(dims [4], sub-frame) of every 4-vector of a D-dim head the camera
    transforms.  "full" (_apply_tiled_projmat, prope_attention.py:120-130):
    dims ((p*4 + c)*4 + j)*(D/64) + r over j, sub-frame c; "sf13"
    (_apply_contiguous_projmat :133-176, PROPE_CAMERA_LAYOUTS :21-24):
    sub-frame 1 on dims [0, 16), 3 on [16, 32), contiguous 4-vectors."""
    out = []
    if layout == "full":
        if D % 64:
            raise ValueError("full camera layout needs D % 64 == 0")
        rn = D // 64
        for p in range(4):
            for c in range(4):
                for r in range(rn):
                    out.append(([((p * 4 + c) * 4 + j) * rn + r for j in range(4)], c))
    elif layout == "sf13":
        if D < 32:
            raise ValueError("sf13 camera layout needs D >= 32")
        for k, sub in enumerate((1, 3)):
            for f in range(4):
                out.append(([16 * k + 4 * f + j for j in range(4)], sub))
    else:
        raise ValueError(layout)
    return out


def camera_apply(x_bf16, mats, layout: str = "full") -> np.ndarray:
    """Camera transform of bf16 bits x [S, H, D] by the 4x4 sub-frame
    matrices of each row, mats [S, 4, 4, 4] fp32: the matrix entries rounded
    to bf16 (camera_kernel.py:21-24, 34), y_i = sum_j M_ij x_j summed in fp64
    (exact for four bf16 x bf16 products), then fp64 -> fp32 -> bf16; dims
    the layout leaves alone are copied."""
    x = bf16_to_f32(np.asarray(x_bf16)).astype(np.float64)
    m = bf16_to_f32(f32_to_bf16(np.asarray(mats, np.float32))).astype(np.float64)
    y = x.copy()
    for dims, sub in camera_vectors(layout, x.shape[-1]):
        y[:, :, dims] = np.einsum("sij,shj->shi", m[:, sub], x[:, :, dims])
    return f32_to_bf16(y.astype(np.float32))


def camera_blocks_apply(x_bf16, mats, cams) -> np.ndarray:
    """camera_selected (CN/core.py:110-137) of bf16 bits x [S, W] (one head's
    W reader dims, whole 8-dim blocks) by mats [S, 4, 4, 4] fp32 of each row:
    block j uses sub-frame cams[j]; its dims 8j + 2e + r form vector r over
    e (the (j, r) order of the full layout).  Matrix entries rounded to bf16,
    sums exact in fp64, then fp64 -> fp32 -> bf16 (as camera_apply)."""
    x = bf16_to_f32(np.asarray(x_bf16)).astype(np.float64)
    m = bf16_to_f32(f32_to_bf16(np.asarray(mats, np.float32))).astype(np.float64)
    y = x.copy()
    for j, c in enumerate(np.asarray(cams, np.int64).tolist()):
        for r in range(2):
            dims = [8 * j + 2 * e + r for e in range(4)]
            y[:, dims] = np.einsum("sij,sj->si", m[:, c % 4], x[:, dims])
    return f32_to_bf16(y.astype(np.float32))


# ----------------------------------------------------------------- a13
def protected_frames(count: int, recent: int, stride: int, sink: int = 0) -> np.ndarray:
    """Frame-level protection mask (CN/core.py:140-152, metadata_cache.py:64-68).

    Last `recent` frames, the first `sink` frames and every `stride`-th frame
    counting back from the newest unprotected one are kept at full width.
    """
    if min(recent, stride, sink) < 0:
        raise ValueError("Negative protection policy")
    keep = np.zeros(count, bool)
    old = max(0, count - recent)
    keep[old:] = True
    keep[:min(sink, count)] = True
    if stride and old:
        keep[np.arange(old - 1, -1, -stride)] = True
    return keep


# ----------------------------------------------------------------- a14-a16
def reader_tables(centers_bf16, mean, h: int, affine_bf16, D: int = 128, dtype=np.float64):
    """Projected center rows and bias of one reader head (CN/core.py:179-199):
    table = bf16(C_h . affine), bias = bf16(bf16(mean_h) . affine); an affine
    of None is the identity (table = C_h, bias = bf16(mean_h)).  Returns
    (table [C, e] bf16 bits or None, bias [e] float32 or None)."""
    table = bias = None
    if centers_bf16 is not None:
        ch = _c(centers_bf16, np.uint16)[:, h * D:(h + 1) * D]
        if affine_bf16 is None:
            table = np.ascontiguousarray(ch)
        else:
            a = bf16_to_f32(affine_bf16).astype(dtype)
            table = f32_to_bf16((bf16_to_f32(ch).astype(dtype) @ a).astype(np.float32))
    if mean is not None:
        mh = bf16_to_f32(f32_to_bf16(np.asarray(mean, np.float32)[h * D:(h + 1) * D]))
        if affine_bf16 is None:
            bias = mh.astype(np.float32)
        else:
            a = bf16_to_f32(affine_bf16).astype(dtype)
            bias = bf16_to_f32(f32_to_bf16((mh.astype(dtype) @ a).astype(np.float32)))
    return table, bias


def reader_read(codec: dict, rows, read_bf16, table_bf16, bias, dtype=np.float64):
    """ReaderGroup.read for one head (CN/core.py:168-200): the latent rows
    (unpacked codes of `rows`) through F.linear with the bias before the
    bf16 rounding, plus the projected center of each row:
      out = bf16(bf16(latent . read^T + bias) + table[id]).
    codec: decode() keyword dict; read_bf16 [e, r].  Returns [rows, e] bf16
    bits (nkvo_decode_epilogue does both roundings)."""
    return decode(codec["packed"], codec["scales"], read_bf16, codec["group"],
                  codec.get("scale_dtype", "bf16"),
                  codec.get("ids") if table_bf16 is not None else None,
                  table_bf16, bias, row_index=np.asarray(rows), dtype=dtype)


def fast_attend(q_bf16, k_cur_bf16, v_cur_bf16, key: dict, value: dict, protect_rows, low_rows,
                groups: Sequence[dict], scale: float, heads: Optional[Sequence[int]] = None,
                D: int = 128, dtype=np.float64, key_freqs: Optional[np.ndarray] = None,
                q_pre_bf16=None, q_freqs: Optional[np.ndarray] = None, cur_mask=None,
                key_cam=None, q_cam=None, out_cam=None, low_shift=None, native_low=None):
    """NanoKV-Fast for one batch item: hybrid_attention (CN/core.py:278-310)
    with maybe_attention's partitions (CN/mg35.py:192-348), identity lift.

    native partition per head: [full decode of protect_rows; current chunk]
    with q (bf16 output, CN/core.py:45-72); low partition for the head's
    group: q_low = bf16(q_h . q_reduce) (CN:164-166), k_low / v_low =
    reader_read of low_rows; merged by LSE (CN:33-42) into bf16.
    groups: dicts with heads, q_reduce, k_read, v_read, k_affine, v_affine
    and lift (bf16 bits per head, None = identity; v_read [vd, r], v_affine
    [D, vd], lift [vd, D]).  Returns (out [Q, H', D] float32
    of the bf16 result, lse [H', Q]).

    RoPE (key_freqs [N, D/2] of the codec rows, CN/mg35.py:207-214, 305-336):
    the protected keys are rotated after decode (rope_apply); a group's
    query is q_pre_bf16 [Q, H, D] projected, and it and k_low are rotated on
    the retained pairs (rope_selected, CN/core.py:75-91) with original pair
    rope_pairs[i][j] (group key; None: pair j), the query at q_freqs [Q, D/2].
    q_bf16 is then the already rotated query of the native partition.
    cur_mask [Q, Nc] bool: which current keys each query sees (native
    partition, CN/mg35.py:258-300).
    Camera (CN/mg35.py:253-257, 310-347), mats [rows, 4, 4, 4] fp32 per row:
    key_cam (P^-1 of the codec rows) transforms the protected keys (after
    RoPE) and values in the full layout and the low keys / values on their
    8-dim blocks (camera_selected, group keys cam_blocks / v_cam_blocks,
    None: block j % 4); q_cam (P^T of the queries) the group query after its
    RoPE; out_cam (P of the queries) the native output before the merge and
    each low output before its lift.  q_bf16, k_cur and v_cur are taken as
    already transformed; a group's query comes from q_pre_bf16 when given.
    low_shift [H, D]: LingBot's value-mean correction (codec_native_attention.py
    :779-785), added to each head's lifted low output before the merge.
    native_low: MG's low_native segment (CN/mg35.py:241-249, 324-347), a
    dict of k_pre_bf16 / v_pre_bf16 [n, H, D] (the pre-RoPE keys and the
    values of the mosaic / current tokens moved into the low partition),
    freqs [n, D/2] (their RoPE, used when key_freqs is given), cam [n, 4, 4,
    4] (their P^-1, used when key_cam is given) and mask [Q, n] bool or
    None; each group head reads them through k_affine / v_affine (bf16
    einsums), rotates and transforms them as the codec low rows, attends them
    with its group query and merges the result last, after the codec low
    rows.  The caller removes these tokens from the native partition
    (cur_mask)."""
    q = bf16_to_f32(q_bf16)
    Qn, H = q.shape[0], q.shape[1]
    heads = list(range(H)) if heads is None else list(heads)
    prot = np.asarray(protect_rows, np.int64)
    low = np.asarray(low_rows, np.int64)
    outs, lses = [], []
    for h in heads:
        cols = np.arange(h * D, (h + 1) * D)
        ks, vs = [], []
        n_prot = 0
        if prot.size:
            kd = decode(**key, row_index=prot, columns=cols, dtype=dtype)
            vd = decode(**value, row_index=prot, columns=cols, dtype=dtype)
            if key_freqs is not None:
                kd = rope_apply(kd[:, None, :], key_freqs[prot])[:, 0]
            if key_cam is not None:
                kd = camera_apply(kd[:, None, :], np.asarray(key_cam)[prot], "full")[:, 0]
                vd = camera_apply(vd[:, None, :], np.asarray(key_cam)[prot], "full")[:, 0]
            ks.append(bf16_to_f32(kd))
            vs.append(bf16_to_f32(vd))
            n_prot = prot.size
        n_cur = 0
        if k_cur_bf16 is not None:
            ks.append(bf16_to_f32(k_cur_bf16)[:, h])
            vs.append(bf16_to_f32(v_cur_bf16)[:, h])
            n_cur = ks[-1].shape[0]
        k = np.concatenate(ks, 0) if ks else np.zeros((0, D))
        v = np.concatenate(vs, 0) if vs else np.zeros((0, D))
        mask = None
        if cur_mask is not None and n_cur:
            mask = np.concatenate([np.ones((Qn, n_prot), bool), np.asarray(cur_mask, bool)], 1)
        on, ln = attention(q[None, :, h], k[None], v[None], scale, dtype, mask=mask)
        on, ln = bf16_to_f32(f32_to_bf16(on[0].astype(np.float32))), ln[0]
        if out_cam is not None:
            on = bf16_to_f32(camera_apply(f32_to_bf16(on)[:, None, :], out_cam, "full")[:, 0])
        grp = [(g, list(g["heads"]).index(h)) for g in groups if h in list(g["heads"])]
        if grp and (low.size or native_low is not None):
            g, i = grp[0]
            qh = q[:, h] if q_pre_bf16 is None else bf16_to_f32(q_pre_bf16)[:, h]
            if g.get("q_reduce") is not None:
                qr = bf16_to_f32(g["q_reduce"][i]).astype(dtype)
                qh = bf16_to_f32(f32_to_bf16((qh.astype(dtype) @ qr).astype(np.float32)))
            if key_freqs is not None:
                rp = g.get("rope_pairs")
                pairs = np.arange(qh.shape[1] // 2) if rp is None else np.asarray(rp[i])
                qh = bf16_to_f32(rope_apply(f32_to_bf16(qh)[:, None, :], q_freqs[:, pairs])[:, 0])
            cb = g.get("cam_blocks")
            kcams = np.arange(qh.shape[1] // 8) % 4 if cb is None else np.asarray(cb[i])
            vcb = g.get("v_cam_blocks")
            if q_cam is not None:
                qh = bf16_to_f32(camera_blocks_apply(f32_to_bf16(qh), q_cam, kcams))
            vd = int(np.asarray(g["v_read"][i]).shape[0])
            vcams = np.arange(vd // 8) % 4 if vcb is None else np.asarray(vcb[i])
            pairs = None
            if key_freqs is not None:
                rp = g.get("rope_pairs")
                pairs = np.arange(qh.shape[1] // 2) if rp is None else np.asarray(rp[i])

            def finish_segment(on, ln, ol, ll):
                # P, the lift and the merge of one low segment (mg35.py:343-347)
                ol = bf16_to_f32(f32_to_bf16(ol[0].astype(np.float32)))
                if out_cam is not None:
                    ol = bf16_to_f32(camera_blocks_apply(f32_to_bf16(ol), out_cam, vcams))
                if g.get("lift") is not None:
                    # lift_output (CN/core.py:202-204), applied before the merge (mg35.py:347)
                    lf = bf16_to_f32(g["lift"][i]).astype(dtype)
                    ol = bf16_to_f32(f32_to_bf16((ol.astype(dtype) @ lf).astype(np.float32)))
                if low_shift is not None:
                    ol = ol + np.asarray(low_shift, np.float64)[h]
                mo, ml = merge(on, ln, ol, ll[0])
                return bf16_to_f32(f32_to_bf16(np.asarray(mo, np.float32))), ml

        if grp and low.size:
            kt, kb = reader_tables(key.get("centers_bf16"), key.get("mean"), h,
                                   None if g.get("k_affine") is None else g["k_affine"][i], D, dtype)
            vt, vb = reader_tables(value.get("centers_bf16"), value.get("mean"), h,
                                   None if g.get("v_affine") is None else g["v_affine"][i], D, dtype)
            kl = reader_read(key, low, g["k_read"][i], kt, kb, dtype)
            if key_freqs is not None:
                kl = rope_apply(kl[:, None, :], key_freqs[low][:, pairs])[:, 0]
            vl = reader_read(value, low, g["v_read"][i], vt, vb, dtype)
            vcams = np.arange(vl.shape[1] // 8) % 4 if vcb is None else np.asarray(vcb[i])
            if key_cam is not None:
                kl = camera_blocks_apply(kl, np.asarray(key_cam)[low], kcams)
                vl = camera_blocks_apply(vl, np.asarray(key_cam)[low], vcams)
            kl = bf16_to_f32(kl)
            vl = bf16_to_f32(vl)
            ol, ll = attention(qh[None], kl[None], vl[None], scale, dtype)
            on, ln = finish_segment(on, ln, ol, ll)
        if grp and native_low is not None:
            # the mosaic / current tokens read through the group's affine maps
            # (mg35.py:324-328), then RoPE and the camera as the low rows
            nl = native_low
            kp = bf16_to_f32(np.asarray(nl["k_pre_bf16"]))[:, h].astype(dtype)
            vp = bf16_to_f32(np.asarray(nl["v_pre_bf16"]))[:, h].astype(dtype)
            ka, va = g.get("k_affine"), g.get("v_affine")
            kk = f32_to_bf16((kp @ bf16_to_f32(ka[i]).astype(dtype)).astype(np.float32)) \
                if ka is not None else f32_to_bf16(kp.astype(np.float32))
            vv = f32_to_bf16((vp @ bf16_to_f32(va[i]).astype(dtype)).astype(np.float32)) \
                if va is not None else f32_to_bf16(vp.astype(np.float32))
            if key_freqs is not None:
                kk = rope_apply(kk[:, None, :], np.asarray(nl["freqs"])[:, pairs])[:, 0]
            if key_cam is not None:
                kk = camera_blocks_apply(kk, np.asarray(nl["cam"]), kcams)
                vv = camera_blocks_apply(vv, np.asarray(nl["cam"]), vcams)
            ol, ll = attention(qh[None], bf16_to_f32(kk)[None], bf16_to_f32(vv)[None], scale,
                               dtype, mask=nl.get("mask"))
            on, ln = finish_segment(on, ln, ol, ll)
        outs.append(on)
        lses.append(ln)
    return np.stack(outs, 1), np.stack(lses, 0)
