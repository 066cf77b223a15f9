"""NanoKV codec API on the gfx950 kernels.

Mirrors the function names, payload dicts and error behaviour of the
reference codec module models/Matrix-Game-3.5/fast/diffsynth/models/
nanokv_codec.py (cited below as MG:line), so a caller of encode_tensor /
decode_value / concat_values / select_value / decode_pair_selected /
direct_latent_pair_segments can switch to this module unchanged.

Differences from the reference, all additive:
  * payload keys "scale_group", "scale_dtype" and "id_dtype" record the scale
    layout (group width, bf16/fp16) and the id width; "scale" is
    [B, S, r/group] (group == r is the reference's one-scale-per-row [B,S,1]);
  * shared center tables can be registered per (kind, layer) with
    register_centers(); encode_tensor then assigns rows to them (nkv_assign)
    instead of fitting per-chunk C64 centers.

Operators (encoder [r, HD], decoder [HD, r], mean [HD]) are registered with
register_operator() or loaded from the reference's prepacked operator file
with preload_operator_weights().  All compute goes through libnanokv_hip.so
(nanokv_amd.ops); there is no CPU path.
"""
from __future__ import annotations

import os
import weakref
from collections import OrderedDict
from pathlib import Path
from typing import Any, Optional

import torch

from . import ops

CODEC = "worldplay_c64_pca_int4_v1"
RAW = "worldplay_raw_v1"
SEGMENTS = "worldplay_segments_v1"
PREPACKED_FORMAT = "mg35_worldplay_operator_int8_v1"

_OPERATORS: dict = {}
_CENTERS: dict = {}


# ---------------------------------------------------------------- settings
def enabled() -> bool:
    """MG:17-18."""
    return os.environ.get("MG35_KVCODEC_MODE", "").strip().lower() == "worldplay_method"


def _rung() -> str:
    """The operator rung of this deployment, MG35_WORLDPLAY_RUNG (MG:21-25):
    pca (no centers), c64, c64_vqat or full (semantic C64 centers)."""
    value = os.environ.get("MG35_WORLDPLAY_RUNG", "full").strip().lower()
    if value not in {"pca", "c64", "c64_vqat", "full"}:
        raise ValueError(f"unsupported MG35_WORLDPLAY_RUNG={value!r}")
    return value


def _center_storage_mode() -> str:
    """Storage of the per-chunk centers, MG35_KVCODEC_CENTER_STORAGE (MG:35-46):
    bf16 (the WorldPlay method) or int8_block (an MG-only experiment)."""
    mode = os.environ.get("MG35_KVCODEC_CENTER_STORAGE", "bf16").strip().lower()
    if mode not in {"bf16", "int8_block"}:
        raise ValueError(f"unsupported MG35 center storage mode={mode!r}")
    return mode


def _expected_center_provenance() -> tuple[str, int]:
    """MG:49-54."""
    if _rung() == "pca":
        return "none", 0
    return _center_storage_mode(), int(os.environ.get("MG35_KVCODEC_CENTER_BLOCK_SIZE", "64"))


def _check_center_provenance(payload: dict, *, context: str) -> None:
    """An operator artifact must record the center storage this runtime uses
    (MG:56-66)."""
    expected_storage, expected_block = _expected_center_provenance()
    if payload.get("center_storage") != expected_storage or int(
            payload.get("center_block_size", -1)) != expected_block:
        raise RuntimeError(
            f"{context} center provenance mismatch: "
            f"artifact={payload.get('center_storage')}/{payload.get('center_block_size')} "
            f"runtime={expected_storage}/{expected_block}")


def _portable_codec_verified(path: str) -> bool:
    """A prepacked operator vouched for by NANOKV_PORTABLE_CODEC_SHA256 may
    carry training-machine paths (nanokv/artifacts.py:8-23)."""
    expected = os.environ.get("NANOKV_PORTABLE_CODEC_SHA256", "").lower()
    if not expected:
        return False
    if len(expected) != 64 or any(c not in "0123456789abcdef" for c in expected):
        raise ValueError("NANOKV_PORTABLE_CODEC_SHA256 must be a SHA256 digest")
    from .codec_native import file_sha256
    if file_sha256(str(Path(path).resolve())) != expected:
        raise ValueError(f"Packed codec checksum mismatch: {path}")
    return True


def _same_artifact_dir(recorded, expected, portable: bool) -> bool:
    """MG:191-198: recorded and expected artifact directories agree (after
    resolving links), or the packed codec is a verified portable one."""
    if portable:
        return True
    recorded, expected = str(recorded or ""), str(expected or "")
    if not recorded or not expected:
        return recorded == expected
    return Path(recorded).resolve() == Path(expected).resolve()


def _check_entry_provenance(kind: str, layer: int, entry: dict, portable: bool) -> None:
    """The basis / decoder / QAT directories an operator entry was built from
    must be this deployment's (MG:186-212)."""
    basis = os.environ.get("MG35_KVCODEC_BASIS_DIR")
    if basis is None and not portable:
        raise RuntimeError("MG35_KVCODEC_BASIS_DIR is required to check operator provenance")
    expected_basis = str(Path(basis).resolve()) if basis else ""
    rung = _rung()
    if kind == "k":
        expected = ""
        if rung == "full":
            expected = str(Path(os.environ["MG35_KVCODEC_DECODER_DIR_K"]).resolve()) \
                if not portable else ""
        if not _same_artifact_dir(entry.get("basis_dir"), expected_basis, portable) or \
                not _same_artifact_dir(entry.get("decoder_dir"), expected, portable):
            raise RuntimeError(f"prepacked K operator provenance mismatch L{layer}")
    else:
        expected = ""
        if rung in {"c64_vqat", "full"}:
            expected = str(Path(os.environ["MG35_KVCODEC_DECODER_DIR_V"]).resolve()) \
                if not portable else ""
        if not _same_artifact_dir(entry.get("basis_dir"), expected_basis, portable) or \
                not _same_artifact_dir(entry.get("qat_dir"), expected, portable):
            raise RuntimeError(f"prepacked V operator provenance mismatch L{layer}")


def _target_enabled(kind: str) -> bool:
    """MG:28-32."""
    target = os.environ.get("MG35_KVCODEC_TARGET", "both").strip().lower()
    if target not in {"k", "v", "both"}:
        raise ValueError(f"unsupported MG35_KVCODEC_TARGET={target!r}")
    return target == "both" or target == kind


def _scale_group(r: int) -> int:
    """NANOKV_SCALE_GROUP: 0 (default) = one scale per row as the reference."""
    g = int(os.environ.get("NANOKV_SCALE_GROUP", "0") or 0)
    return r if g <= 0 else g


def _scale_dtype() -> torch.dtype:
    v = os.environ.get("NANOKV_SCALE_DTYPE", "bf16").strip().lower()
    if v in {"bf16", "bfloat16"}:
        return torch.bfloat16
    if v in {"fp16", "float16", "half"}:
        return torch.float16
    raise ValueError(f"unsupported NANOKV_SCALE_DTYPE={v!r}")


def _quant_mode() -> str:
    """bf16 (default) reproduces MG's bf16 quantiser arithmetic (MG:349-351);
    fp32 is HY's (kv_codecs.py:244-255)."""
    v = os.environ.get("NANOKV_QUANT_MODE", "bf16").strip().lower()
    if v not in {"bf16", "fp32"}:
        raise ValueError(f"unsupported NANOKV_QUANT_MODE={v!r}")
    return v


# ---------------------------------------------------------------- operators
def pack_operator(weight: torch.Tensor, device: torch.device,
                  group_size: Optional[int] = None) -> dict:
    """The int8 operator storage of _pack_operator (MG:108-131) on `device`
    (nkv_int8_pack): {"storage": "int8", "qweight", "scale", "group_size"};
    group_size defaults to MG35_KVCODEC_INT8_WEIGHT_GROUP_SIZE (0: whole row)."""
    if group_size is None:
        group_size = int(os.environ.get("MG35_KVCODEC_INT8_WEIGHT_GROUP_SIZE", "0") or 0)
    return ops.int8_pack(weight.detach().float().to(device), group_size)


def _operator_weight(w) -> torch.Tensor:
    """bf16 weight of a registered operator: a tensor, or an int8 operator dict
    dequantized on its device (nkv_int8_dequant) as _operator_linear does
    per call (MG:145-152); the operator weights are static, so once here."""
    if isinstance(w, dict):
        if w.get("storage", "int8") != "int8":
            return w["weight"].detach().to(torch.bfloat16).contiguous()
        return ops.int8_dequant(w)
    return w.detach().to(torch.bfloat16).contiguous()


def register_operator(kind: str, layer: int, *, encoder, decoder,
                      mean: Optional[torch.Tensor] = None) -> None:
    """Register the codec operator of (kind, layer): encoder [r, HD] and decoder
    [HD, r] (F.linear weight layouts, MG:134-153) as bf16 tensors or int8
    operator dicts (pack_operator / the prepacked file), mean [HD] fp32."""
    if kind not in {"k", "v"}:
        raise ValueError(kind)
    enc = _operator_weight(encoder)
    dec = _operator_weight(decoder)
    if enc.dim() != 2 or dec.dim() != 2 or enc.shape[0] != dec.shape[1] or enc.shape[1] != dec.shape[0]:
        raise ValueError("encoder must be [r, HD] and decoder [HD, r]")
    m = None if mean is None else mean.detach().float().reshape(-1).contiguous()
    _OPERATORS[(kind, int(layer))] = {"encoder": enc, "decoder": dec, "mean": m}


def register_centers(kind: str, layer: int, centers: Optional[torch.Tensor]) -> None:
    """Shared center table [C, HD] (bf16) for (kind, layer); None removes it."""
    if centers is None:
        _CENTERS.pop((kind, int(layer)), None)
        return
    _CENTERS[(kind, int(layer))] = centers.detach().to(torch.bfloat16).contiguous()


def preload_operator_weights(device: torch.device, path: Optional[str] = None) -> None:
    """Load every operator of the reference's prepacked file (format
    mg35_worldplay_operator_int8_v1, MG:257-279) onto `device`, after its
    checks: the file's center provenance and rung must be this runtime's
    (MG:272-274), and every entry's basis / decoder directories
    (MG:186-212)."""
    path = path or os.environ.get("MG35_KVCODEC_PREPACKED_OPERATOR_PATH", "").strip()
    if not path:
        raise RuntimeError("formal worldplay_method requires MG35_KVCODEC_PREPACKED_OPERATOR_PATH")
    payload = torch.load(path, map_location="cpu", weights_only=True)
    if payload.get("format") != PREPACKED_FORMAT:
        raise RuntimeError(f"bad prepacked WorldPlay operator: {path}")
    _check_center_provenance(payload, context="prepacked operator")
    if payload.get("rung") != _rung():
        raise RuntimeError(f"operator rung={payload.get('rung')} runtime={_rung()}")
    portable = _portable_codec_verified(path)
    for name in sorted(payload["entries"]):
        kind, layer = name.split(":", 1)
        _check_entry_provenance(kind, int(layer), payload["entries"][name], portable)

    def move(packed):
        return {"storage": "int8", "group_size": int(packed["group_size"]),
                "qweight": packed["qweight"].to(device=device, dtype=torch.int8).contiguous(),
                "scale": packed["scale"].to(device=device, dtype=torch.bfloat16).contiguous()}

    for name in sorted(payload["entries"]):
        kind, layer = name.split(":", 1)
        entry = payload["entries"][name]
        register_operator(kind, int(layer), encoder=move(entry["encoder"]),
                          decoder=move(entry["decoder"]), mean=entry["mean"].float().to(device))


def _operator(kind: str, layer: int, device: torch.device) -> dict:
    key = (kind, int(layer))
    if key not in _OPERATORS:
        raise RuntimeError(f"no codec operator registered for {kind}:{int(layer):02d}")
    op = _OPERATORS[key]
    if op["encoder"].device != device:
        op = {k: (None if v is None else v.to(device)) for k, v in op.items()}
        _OPERATORS[key] = op
    return op


# ---------------------------------------------------------------- centers
@torch.no_grad()
def semantic_residual_centers(value: torch.Tensor, layer: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-chunk joint-head C64 centers (MG:301-330) on the GPU (nkv_c64_fit):
    the initial centers are the rows randperm(S) draws from a CPU generator
    seeded with 20260804 + layer (so they match the reference's draw), then
    MG35_KVCODEC_C64_ITERS rounds of nearest-center labels and mean updates.
    Returns (bf16 centers [B, C, HD], labels [B, S] int32 of the last round),
    the stored centers of store_centers (MG:69-90)."""
    batch, sequence, dim = value.shape
    clusters = int(os.environ.get("MG35_KVCODEC_C64_CLUSTERS", "64"))
    iterations = int(os.environ.get("MG35_KVCODEC_C64_ITERS", "2"))
    if clusters <= 0 or clusters > sequence or clusters > 256:
        raise ValueError(f"C64 clusters must be in [1,min(S,256)], got {clusters}")
    draw = torch.Generator(device="cpu").manual_seed(20260804 + int(layer))
    init = torch.randperm(sequence, generator=draw)[:clusters].to(torch.int32)
    centers, labels = ops.c64_fit(value.detach().float().contiguous(),
                                  init.to(value.device), iterations)
    return centers.to(torch.bfloat16), labels


# ---------------------------------------------------------------- encode
@torch.no_grad()
def encode_tensor(kind: str, layer: int, value: torch.Tensor) -> dict:
    """Encode one chunk [B, S, HD] into an immutable payload (MG:333-365).

    With a registered shared center table every row is assigned to its
    nearest center (nkv_assign); otherwise per-chunk C64 centers are fitted
    as the reference does.  Projection and INT4 quantisation run in
    nkv_encode."""
    if kind not in {"k", "v"}:
        raise ValueError(kind)
    if not _target_enabled(kind):
        return {"codec": RAW, "tensor": value.detach()}
    if value.dim() != 3:
        raise ValueError("encode_tensor expects [B, S, HD]")
    semantic = _rung() != "pca"
    if semantic and _center_storage_mode() != "bf16":
        raise NotImplementedError("MG35_KVCODEC_CENTER_STORAGE=int8_block (an MG-only "
                                  "experiment, not WorldPlay parity) is not built")
    batch, seq, dim = (int(v) for v in value.shape)
    op = _operator(kind, layer, value.device)
    r = int(op["encoder"].shape[0])
    group = _scale_group(r)
    sdt = _scale_dtype()
    qmode = _quant_mode()
    rows = value.detach().float().contiguous()
    shared = _CENTERS.get((kind, int(layer)))
    packed, scales, ids_out, tables = [], [], [], []
    centers = ids_t = None
    id_dtype = torch.uint8
    center_batch_shared = False
    if not semantic:
        # the pca rung: the rows themselves are projected (MG:338-342)
        for b in range(batch):
            e = ops.encode(rows[b], op["encoder"], mean=op["mean"], group=group,
                           scale_dtype=sdt, quant_mode=qmode)
            packed.append(e["packed"])
            scales.append(e["scales"])
    elif shared is not None:
        shared = shared.to(value.device)
        id_dtype = ops.id_dtype_for(int(shared.shape[0]))
        for b in range(batch):
            e = ops.encode(rows[b], op["encoder"], centers=shared, mean=op["mean"], group=group,
                           scale_dtype=sdt, quant_mode=qmode, id_dtype=id_dtype)
            packed.append(e["packed"])
            scales.append(e["scales"])
            ids_out.append(e["ids"])
        centers = shared[None]
        center_batch_shared = True
    else:
        fitted, labels = semantic_residual_centers(value, layer)
        id_dtype = torch.uint8
        for b in range(batch):
            # the fit's labels are kept (MG:326-330): the encoder subtracts each
            # row's stored center without searching again
            ids = labels[b].to(torch.uint8)
            e = ops.encode(rows[b], op["encoder"], centers=fitted[b], mean=op["mean"],
                           group=group, scale_dtype=sdt, quant_mode=qmode, ids=ids)
            packed.append(e["packed"])
            scales.append(e["scales"])
            ids_out.append(ids)
        centers = fitted
        center_batch_shared = False
    if ids_out:
        ids_t = torch.stack(ids_out)
    return {
        "codec": CODEC,
        "kind": kind,
        "layer": int(layer),
        "shape": (batch, seq, dim),
        "latent_shape": (batch, seq, r),
        "latent_numel": batch * seq * r,
        "packed_codes": torch.stack(packed).reshape(-1),
        "scale": torch.stack(scales),
        "centers": centers,
        "ids": ids_t,
        "semantic": semantic,
        "source_dtype": str(value.dtype).replace("torch.", ""),
        "scale_group": group,
        "scale_dtype": "fp16" if sdt == torch.float16 else "bf16",
        "id_dtype": str(id_dtype).replace("torch.", ""),
        "shared_centers": center_batch_shared,
    }


def encode_raw_tensor(value: torch.Tensor) -> dict:
    """Cache-owned bf16 copy of a raw segment (MG:458-469)."""
    return {"codec": RAW, "tensor": value.detach().clone(memory_format=torch.contiguous_format)}


# ---------------------------------------------------------------- views
def is_payload(value: Any) -> bool:
    """MG:472-486 (the payload kinds this module produces)."""
    return isinstance(value, dict) and value.get("codec") in {RAW, CODEC, SEGMENTS}


def segments_of(value: Any) -> list:
    if value is None:
        return []
    if isinstance(value, dict) and value.get("codec") == SEGMENTS:
        return list(value["segments"])
    return [value]


def value_shape(value: Any) -> tuple[int, int, int] | None:
    """MG:489-513."""
    if value is None:
        return None
    if torch.is_tensor(value):
        return tuple(int(v) for v in value.shape)
    codec = value.get("codec")
    if codec == RAW:
        return tuple(int(v) for v in value["tensor"].shape)
    if codec == CODEC:
        return tuple(int(v) for v in value["shape"])
    if codec == SEGMENTS:
        shapes = [value_shape(item) for item in value["segments"]]
        if not shapes:
            return None
        return (shapes[0][0], sum(s[1] for s in shapes), shapes[0][2])
    raise RuntimeError(f"unsupported cache value {codec}")


def payload_bytes(value: Any) -> int:
    """Resident bytes of a payload tree (MG:697-704)."""
    if torch.is_tensor(value):
        return value.numel() * value.element_size()
    if isinstance(value, dict):
        return sum(payload_bytes(v) for k, v in value.items() if not str(k).startswith("_"))
    if isinstance(value, (list, tuple)):
        return sum(payload_bytes(v) for v in value)
    return 0


class SegmentList(dict):
    """A worldplay_segments_v1 list, {"codec": SEGMENTS, "segments": [...]}:
    a plain dict to every caller (same keys, same behaviour), which can also be
    weakly referenced, so that history_codecs can remember its segment tables
    exactly as long as the caller keeps the list."""


def concat_values(left: Any, right: Any) -> Any:
    """Append immutable segments (MG:600-609)."""
    if left is None:
        return right
    if right is None:
        return left
    if not is_payload(left) or not is_payload(right):
        raise RuntimeError("WorldPlay packed-cache concat received a raw/payload mixture")
    return SegmentList(codec=SEGMENTS, segments=segments_of(left) + segments_of(right))


def codec_view(part: dict, device: torch.device) -> ops.Codec:
    """Device tensors of one encoded segment as an ops.Codec."""
    if part.get("codec") != CODEC:
        raise RuntimeError(f"unsupported WorldPlay payload {part.get('codec')}")
    batch, seq, _ = (int(v) for v in part["shape"])
    r = int(part["latent_shape"][-1])
    op = _operator(str(part["kind"]), int(part["layer"]), device)
    group = int(part.get("scale_group", r))
    scale = part["scale"].to(device)
    if scale.dtype not in (torch.bfloat16, torch.float16):
        scale = scale.to(torch.bfloat16)
    scale = scale.reshape(batch, seq, r // group).contiguous()
    centers = ids = None
    if part.get("semantic", True) and part.get("centers") is not None:
        centers = part["centers"].to(device)
        if centers.dim() == 2:
            centers = centers[None]
        centers = centers.to(torch.bfloat16).contiguous()
        ids = part["ids"].to(device).reshape(batch, seq)
        if ids.dtype not in (torch.uint8, torch.int16, torch.int32):
            ids = ids.to(ops.id_dtype_for(int(centers.shape[1])))
        ids = ids.contiguous()
    return ops.Codec(packed=part["packed_codes"].to(device).reshape(batch, seq, r // 2),
                     scales=scale, w_dec=op["decoder"], group=group, ids=ids,
                     centers=centers, mean=op["mean"])


# ---------------------------------------------------------------- decode
@torch.no_grad()
def decode_tensor(payload: dict, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """Full-width decode of one payload (MG:368-390) on nkv_decode."""
    if payload.get("codec") == RAW:
        return payload["tensor"].to(device=device, dtype=dtype)
    view = codec_view(payload, torch.device(device))
    out = ops.decode(view, int(payload["shape"][2]))
    return out.to(dtype)


def decode_value(value: Any, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor | None:
    """MG:516-539: raw tensors pass through; segment lists decode per segment
    (each with its own center table) and concatenate along tokens."""
    if value is None:
        return None
    if torch.is_tensor(value):
        return value.to(device=device, dtype=dtype)
    if value.get("codec") == SEGMENTS:
        parts = [decode_value(item, dtype=dtype, device=device) for item in value["segments"]]
        return torch.cat(parts, dim=1) if parts else None
    return decode_tensor(value, dtype=dtype, device=device)


def decode_pair_values(key: Any, value: Any, *, dtype: torch.dtype, device: torch.device):
    """MG:542-597."""
    return (decode_value(key, dtype=dtype, device=device),
            decode_value(value, dtype=dtype, device=device))


def select_value(value: Any, token_idx: torch.Tensor, *, kind: str, layer: int,
                 dtype: torch.dtype, device: torch.device) -> Any:
    """Select tokens keeping whole immutable segments (MG:612-694): fully
    selected segments are reused, a cut segment is decoded, sliced and
    re-encoded."""
    if torch.is_tensor(value):
        return value.index_select(1, token_idx).contiguous()
    parts = segments_of(value)
    wanted = token_idx.detach().cpu().tolist()
    if wanted != sorted(wanted):
        raise RuntimeError("segmented cache selection expects sorted in-range token indices")
    out, offset, cursor = [], 0, 0
    for part in parts:
        length = int(value_shape(part)[1])
        local = []
        while cursor < len(wanted) and wanted[cursor] < offset + length:
            local.append(wanted[cursor] - offset)
            cursor += 1
        if local:
            if local == list(range(length)):
                out.append(part)
            else:
                tensor = decode_value(part, dtype=dtype, device=device)
                sel = tensor.index_select(1, torch.as_tensor(local, device=tensor.device))
                if part.get("codec") == RAW:
                    out.append(encode_raw_tensor(sel))
                else:
                    out.append(encode_tensor(kind, layer, sel.contiguous()))
        offset += length
    if cursor != len(wanted):
        raise RuntimeError("segmented cache selection expects sorted in-range token indices")
    if not out:
        return None
    if len(out) == 1:
        return out[0]
    return SegmentList(codec=SEGMENTS, segments=out)


def _pairs(key: Any, value: Any) -> list:
    kp, vp = segments_of(key), segments_of(value)
    if len(kp) != len(vp):
        raise ValueError("paired codec segment count mismatch")
    for k, v in zip(kp, vp):
        if (k.get("codec") != CODEC or v.get("codec") != CODEC or k.get("kind") != "k"
                or v.get("kind") != "v" or tuple(k["shape"]) != tuple(v["shape"])
                or int(k["layer"]) != int(v["layer"])):
            raise RuntimeError("codec-native attention requires paired formal method payloads")
    return list(zip(kp, vp))


@torch.no_grad()
def decode_pair_selected(key: Any, value: Any, token_keep: torch.Tensor, *, dtype: torch.dtype,
                         device: torch.device):
    """Decode only the kept rows (MG:801-861) with nkv_decode's row index."""
    pairs = _pairs(key, value)
    keep = token_keep.to(device="cpu", dtype=torch.bool).reshape(-1)
    if keep.numel() != sum(int(k["shape"][1]) for k, _ in pairs):
        raise ValueError("selected decode mask/cache length mismatch")
    outs = {"k": [], "v": []}
    offset = 0
    dev = torch.device(device)
    for kpart, vpart in pairs:
        length = int(kpart["shape"][1])
        local = keep[offset:offset + length]
        offset += length
        if not bool(local.any()):
            continue
        index = torch.nonzero(local, as_tuple=False).flatten().to(torch.int32).to(dev)
        for target, part in (("k", kpart), ("v", vpart)):
            view = codec_view(part, dev)
            outs[target].append(ops.decode(view, int(part["shape"][2]), row_index=index).to(dtype))
    if not outs["k"]:
        shape = value_shape(key)
        empty = torch.empty((shape[0], 0, shape[2]), device=device, dtype=dtype)
        return empty, empty.clone()
    return torch.cat(outs["k"], 1), torch.cat(outs["v"], 1)


@torch.no_grad()
def direct_latent_pair_segments(key: Any, value: Any, *, device: torch.device,
                                token_keep: Optional[torch.Tensor] = None) -> list:
    """Expose the bf16 latent rows, center tables/ids and mean of each paired
    segment without reconstructing K/V (MG:707-798); latents come from
    nkv_unpack."""
    pairs = _pairs(key, value)
    wanted = None
    if token_keep is not None:
        wanted = token_keep.to(device="cpu", dtype=torch.bool).reshape(-1)
        if wanted.numel() != sum(int(k["shape"][1]) for k, _ in pairs):
            raise ValueError("direct latent token mask/cache length mismatch")
    dev = torch.device(device)
    result, offset = [], 0
    for kpart, vpart in pairs:
        length = int(kpart["shape"][1])
        local = None if wanted is None else wanted[offset:offset + length]
        offset += length
        if local is not None and not bool(local.any()):
            continue
        index = None if local is None else torch.nonzero(local, as_tuple=False).flatten()

        def expose(part):
            view = codec_view(part, dev)
            B, S = view.batch, view.tokens
            r = view.r
            rows = []
            for b in range(B):
                idx = None if index is None else index.to(torch.int32).to(dev)
                rows.append(ops.unpack(view.packed[b], view.scales[b], r, view.group, idx))
            latent = torch.stack(rows)
            ids = None if view.ids is None else view.ids.long()
            if ids is not None and index is not None:
                ids = ids.index_select(1, index.to(dev))
            centers = None if view.centers is None else view.centers.float()
            return latent, (centers, ids), view.mean

        logical = torch.arange(offset - length, offset, device=dev)
        if index is not None:
            logical = logical.index_select(0, index.to(dev))
        result.append({"k": expose(kpart), "v": expose(vpart), "length": int(logical.numel()),
                       "logical_indices": logical})
    return result


_HISTORY_TABLES: "OrderedDict[tuple, tuple]" = OrderedDict()
_HISTORY_TABLES_MAX = 256


def _evict_history_table(ident: tuple, ref: "weakref.ref") -> None:
    entry = _HISTORY_TABLES.get(ident)
    if entry is not None and any(r is ref for r in entry[0]):
        del _HISTORY_TABLES[ident]


def history_codecs(key: Any, value: Any, device: torch.device):
    """One (K, V) ops.Codec pair covering every segment of a paired cache.

    A single segment is passed as its own flat arrays.  A segment list is
    passed as an nkv_segment table over the segments' own tensors (each with
    its own center table, as the reference decodes them, MG:393-455): no
    codes, scales, ids or tables are copied.  The tables of a K/V pair of
    SegmentLists (what concat_values and select_value return) are remembered
    while both lists live, so the per-layer reads of one denoise step and the
    next reuse them: an entry holds weak references to the two lists and is
    dropped with them (select_value evicting frames, a cache reset), and with
    it the device views it kept.  Other segment lists are not remembered."""
    pairs = _pairs(key, value)
    dev = torch.device(device)
    if len(pairs) == 1:
        return codec_view(pairs[0][0], dev), codec_view(pairs[0][1], dev)
    remember = isinstance(key, SegmentList) and isinstance(value, SegmentList)
    ident = (str(dev), id(key), id(value))
    hit = _HISTORY_TABLES.get(ident) if remember else None
    if hit is not None and hit[0][0]() is key and hit[0][1]() is value:
        _HISTORY_TABLES.move_to_end(ident)
        return hit[1]
    out = []
    for which in (0, 1):
        views = [codec_view(p[which], dev) for p in pairs]
        if len({(v.r, v.group, v.scales.dtype, v.w_dec.data_ptr()) for v in views}) != 1:
            raise RuntimeError("history segments must share rank, scale group, scale dtype "
                               "and codec operator")
        if len({v.centers is None for v in views}) != 1:
            raise RuntimeError("history segments mix semantic and pca payloads")
        table = ops.SegmentTable([ops.Segment(v.packed, v.scales, v.ids, v.centers)
                                  for v in views], dev)
        out.append(ops.Codec(packed=None, scales=None, w_dec=views[0].w_dec,
                             group=views[0].group, mean=views[0].mean, segments=table))
    if remember:
        refs = tuple(weakref.ref(x, lambda ref, ident=ident: _evict_history_table(ident, ref))
                     for x in (key, value))
        _HISTORY_TABLES[ident] = (refs, (out[0], out[1]))
        while len(_HISTORY_TABLES) > _HISTORY_TABLES_MAX:
            _HISTORY_TABLES.popitem(last=False)
    return out[0], out[1]
