"""Codec-native attention on the gfx950 kernels.

Mirrors the partition attention and merge helpers of the reference's
models/Matrix-Game-3.5/fast/codec_native/core.py (cited as CN:line) and the
history read of the NanoKV hook (wan_video_dit.py:488-627, decode_pair_values
followed by attention), with the decode fused into the attention kernel:

  attention_lse(q, k, v)           CN:45-72   uncompressed partition, (O, lse)
  merge(out_a, lse_a, out_b, lse_b) CN:33-42  exact LSE merge of partitions
  protected_tokens(frame_ids, ...) CN:140-152 frame-level protection policy
  codec_history_attention(q, cache, k_cur, v_cur, rope=None)
                                   decode-then-attend of a paired K/V codec
                                   cache plus the current chunk in one library
                                   call (nkv_attend): each history tile is
                                   decoded once, into the call's workspace in
                                   the flash kernel's layout; no K/V tensor;
                                   rope: read-time RoPE of the cached keys
                                   (wan_video_dit.py:538-546)
  kv_rope(freqs, positions, h, w)  the positions of cached frames, as
                                   _kv_freqs (pipelines/wan_video.py:3322-3341)
                                   builds them, for the fused kernel
  ReaderGroup / ReaderLayer        CN:155-224 reader parameters, bound to
                                   the kernels (identity flags CN:256-262)
  enabled(prefix), file_sha256(path), get_layer(prefix, model, layer, ...)
                                   CN:20-30, 229-275: reader checkpoints bound
                                   by a manifest to the deployed codec operator
  fast_history_attention(q, cache, k_cur, v_cur, reader, protect)
                                   NanoKV-Fast: maybe_attention's native /
                                   low partitions (mg35.py:192-348) and
                                   hybrid_attention's merge (CN:278-310),
                                   fused (nkv_fast_attend)

Tensors follow the reference's [B, H, S, D] layout; nothing here runs on the
CPU.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
from pathlib import Path
from typing import Any, Optional

import torch

from . import nanokv_codec, ops


def _attend_bhsd(q, k, v, scale, visibility=None):
    """nkv_attend of [B, H, S, D] tensors with k/v as uncompressed keys."""
    qq = q.to(torch.bfloat16).permute(0, 2, 1, 3)
    if k.shape[-2] == 0:
        out, lse = ops.attend(qq.contiguous(), None, None, softmax_scale=scale)
    else:
        out, lse = ops.attend(qq.contiguous(), k.to(torch.bfloat16).permute(0, 2, 1, 3),
                              v.to(torch.bfloat16).permute(0, 2, 1, 3), softmax_scale=scale,
                              visibility=visibility)
    return out.permute(0, 2, 1, 3).to(q.dtype), lse


def attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  mask: Optional[torch.Tensor] = None, *, scale: Optional[float] = None):
    """softmax(q k^T * scale) v with its natural-log LSE for [B, H, S, D]
    inputs (CN:45-72).  An empty key set gives (0, -inf) (CN:48-49).
    mask (True = visible) broadcasts as [..., Q or 1, N] over [B, H]; the
    kernel takes one visibility per query group (rows of equal visibility), so
    a mask that differs across batch items or heads runs one call per
    (b, h).  A query that sees no key gets (0, -inf)."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if mask is None or k.shape[-2] == 0:
        return _attend_bhsd(q, k, v, scale)
    if mask.dtype != torch.bool:
        raise ValueError("Only boolean visibility masks are supported")
    B, H, Qn, _ = q.shape
    N = int(k.shape[-2])
    if mask.dim() < 2 or mask.shape[-1] != N or mask.shape[-2] not in (1, Qn):
        raise ValueError("mask must broadcast as [..., Q or 1, N]")
    lead = mask.reshape(-1, *mask.shape[-2:]) if mask.dim() > 2 else mask[None]
    if lead.shape[0] == 1:
        vis = ops.Visibility.from_bool(lead[0].expand(Qn, N), q.device)
        return _attend_bhsd(q, k, v, scale, vis)
    full = mask.expand(B, H, Qn, N)
    out = torch.empty((B, H, Qn, v.shape[-1]), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, Qn), device=q.device, dtype=torch.float32)
    for b in range(B):
        for h in range(H):
            vis = ops.Visibility.from_bool(full[b, h], q.device)
            o, l = _attend_bhsd(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                                scale, vis)
            out[b, h], lse[b, h] = o[0, 0], l[0, 0]
    return out, lse


def attention_grouped_mask(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           mask: torch.Tensor, query_groups: torch.Tensor, *, scale: float):
    """Attention where the queries of each group share one visibility row,
    mask[0, 0, first query of the group] (CN:94-103), in one fused call: the
    groups become the kernel's query groups."""
    if k.shape[-2] == 0:
        return _attend_bhsd(q, k, v, scale)
    groups, inverse = torch.unique(query_groups.to(q.device), return_inverse=True)
    first = torch.full((groups.numel(),), query_groups.numel(), device=q.device, dtype=torch.long)
    first.scatter_reduce_(0, inverse, torch.arange(query_groups.numel(), device=q.device),
                          reduce="amin")
    rows = mask[0, 0].index_select(0, first)
    vis = ops.Visibility.from_bool(rows, q.device)
    # from_bool regroups equal rows; map each query's group through it
    vis = ops.Visibility(vis.bits, vis.q_group.long().index_select(0, inverse).to(torch.int32)
                         .contiguous())
    return _attend_bhsd(q, k, v, scale, vis)


def merge(out_a: torch.Tensor, lse_a: torch.Tensor, out_b: torch.Tensor, lse_b: torch.Tensor):
    """Exact global-softmax merge of two partitions; empty rows give zero (CN:33-42)."""
    out, lse = ops.lse_merge(out_a.to(torch.bfloat16).contiguous(), lse_a.float().contiguous(),
                             out_b.to(torch.bfloat16).contiguous(), lse_b.float().contiguous())
    return out.to(out_a.dtype), lse


def protected_tokens(frame_ids: torch.Tensor, recent: int, stride: int, sink: int = 0):
    """Frame-run protection mask (CN:140-152): the last `recent` runs, the
    first `sink` runs and every `stride`-th run back from the newest
    unprotected one; consecutive equal frame ids form one run."""
    if min(recent, stride, sink) < 0:
        raise ValueError("Negative protection policy")
    _, inverse = torch.unique_consecutive(frame_ids, return_inverse=True)
    count = int(inverse.max()) + 1 if inverse.numel() else 0
    old = max(0, count - recent)
    keep = torch.arange(count, device=frame_ids.device) >= old
    keep[:min(sink, count)] = True
    if stride and old:
        keep[torch.arange(old - 1, -1, -stride, device=frame_ids.device)] = True
    return keep[inverse]


def kv_camera(P_inv: torch.Tensor, frames, tokens_per_frame: int, device, *,
              layout: str = "full") -> ops.Camera:
    """Camera of cached frames for the history keys and values: P_inv
    [batches, cameras, 4, 4, 4] (camera_info[1][2]), frames the camera index
    of each cached frame (the runs _viewmats collapses, CN/mg35.py:38-51),
    each frame tokens_per_frame codec rows; layout "full" or "sf13"."""
    mats = P_inv.to(device=device, dtype=torch.float32).contiguous()
    frame_mat = torch.as_tensor(list(frames), dtype=torch.int32)
    if frame_mat.numel() == 0:
        raise ValueError("camera needs at least one frame")
    if int(frame_mat.min()) < 0 or int(frame_mat.max()) >= mats.shape[1]:
        raise ValueError("frame camera index outside P_inv")
    return ops.Camera(mats, frame_mat.to(device), int(tokens_per_frame), layout)


def kv_rope(freqs, temporal_positions, h: int, w: int, device, *,
            disable_t: bool = False) -> ops.Rope:
    """Read-time RoPE positions of cached frames: `freqs` is the model's
    frequency tuple (precompute_freqs_cis_3d: temporal, row, column bands
    first), one temporal position per cached frame, frames of h x w tokens.
    The same arguments as _kv_freqs (pipelines/wan_video.py:3322-3341), which
    returns the per-token complex table instead.  disable_t: identity
    temporal band (prope_disable_t_rope, wan_video_dit.py:542-545)."""
    bands = tuple(torch.as_tensor(b) for b in freqs[:3])
    for b in bands:
        if not torch.is_complex(b) or b.dim() != 2:
            raise ValueError("freqs bands must be complex [positions, pairs] tensors")
    bands = tuple(b.to(torch.complex128).cpu() for b in bands)
    return ops.Rope.from_bands(bands, temporal_positions, h, w, torch.device(device),
                               disable_t=disable_t)


def codec_history_attention(q: torch.Tensor, cache_k: Any, cache_v: Any,
                            k_cur: Optional[torch.Tensor] = None,
                            v_cur: Optional[torch.Tensor] = None, *,
                            scale: Optional[float] = None, return_lse: bool = False,
                            rope=None, camera: Optional[ops.Camera] = None,
                            hist_rows: Optional[torch.Tensor] = None,
                            visibility: Optional[ops.Visibility] = None):
    """Attention of q [B, H, Q, D] over [decoded history; current chunk] where
    the history is the paired codec cache (nanokv_codec payloads or segment
    lists) and k_cur/v_cur [B, H, Nc, D] are uncompressed.  Equivalent to the
    reference's decode_pair_values + attention (wan_video_dit.py:497-627)
    with the decode fused into nkv_attend.  rope (kv_rope): the cached keys
    are rotated after decode at their positions, as the reference's
    rope_apply(cache_k_pre, cache_freqs) (wan_video_dit.py:538-546); q and
    k_cur are taken as already rotated.  camera (kv_camera): the cached keys
    (after RoPE) and values are multiplied by their frames' P^-1 inside the
    kernel, as _native_prope does to the decoded history (CN/mg35.py:54-71);
    q, k_cur and v_cur are taken as already transformed and the caller
    applies P to the output.  hist_rows: int32 cache rows attended (the
    frames a chunk id selects, wan_video_dit.py:509-530); visibility: which
    current keys each query sees (the hole and chunk-id keep masks,
    wan_video_dit.py:454-520)."""
    device = q.device
    B, H, Qn, D = (int(x) for x in q.shape)
    key = value = None
    shape = None if cache_k is None else nanokv_codec.value_shape(cache_k)
    if shape is not None and shape[1] > 0:
        if camera is not None and camera.frame_mat.numel() * camera.tokens_per_frame != shape[1]:
            raise ValueError("the camera's frames must cover exactly the cached rows "
                             "(complete equal-sized frames)")
        key, value = nanokv_codec.history_codecs(cache_k, cache_v, device)
    qq = q.to(torch.bfloat16).permute(0, 2, 1, 3)
    kc = None if k_cur is None else k_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    vc = None if v_cur is None else v_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    if key is None:
        hist_rows = None
    elif hist_rows is not None:
        hist_rows = hist_rows.to(device=device, dtype=torch.int32).contiguous()
    out, lse = ops.attend(qq, kc, vc, key, value,
                          softmax_scale=D ** -0.5 if scale is None else scale,
                          return_lse=return_lse, rope=rope if key is not None else None,
                          camera=camera if key is not None else None, hist_rows=hist_rows,
                          visibility=visibility if kc is not None else None)
    out = out.permute(0, 2, 1, 3)
    return (out, lse) if return_lse else out


def _whole_blocks(indices: torch.Tensor) -> bool:
    """Reader dims made of whole, aligned 8-dim original blocks (CN:118-123)."""
    ind = indices.long().cpu()
    if ind.shape[-1] % 8:
        return False
    blocks = ind.reshape(ind.shape[0], -1, 8)
    return bool(torch.equal(blocks, blocks[..., :1] + torch.arange(8))) and \
        not bool((blocks[..., 0] % 8).any())


def _is_selection(lift: torch.Tensor, v_indices: torch.Tensor) -> bool:
    """lift[h] [vd, D] scatters reader dim e to original dim v_indices[h, e]
    (reader_tools.initialize_reader_state's lift) and nothing else."""
    lf = lift.float().cpu()
    sel = torch.zeros_like(lf)
    sel.scatter_(2, v_indices.long().cpu()[..., None], 1.0)
    return bool(torch.equal(lf, sel))


def _is_identity(w: torch.Tensor) -> bool:
    """The reference's identity test for reader matrices (CN:259-262)."""
    return w.shape[-2] == w.shape[-1] and torch.equal(
        w.float().cpu(), torch.eye(w.shape[-1]).expand_as(w))


class ReaderGroup:
    """One reader group (CN:155-204) on the device: heads that read the low
    history rows through q_reduce / k_read / v_read / k_affine / v_affine.
    Matrices equal to the identity are flagged as such (CN:256-262) and
    skipped, as the reference's fast runtime does.  A value lift [vd, D]
    other than the identity is folded into the value reader once: attention
    is linear in V, so lifting each low partition's output (CN:202-204,
    mg35.py:347) equals reading V' = v_low . lift, i.e. v_read' = lift^T .
    v_read [D, r] and v_affine' = v_affine . lift [D, D] (composed in fp32,
    rounded to bf16 once); only where the bf16 roundings fall differs."""

    def __init__(self, state: dict, device=None):
        self.heads = state["heads"].long()
        self.indices = state["indices"].long()
        self.v_indices = state.get("v_indices", state["indices"]).long()
        h, d = len(self.heads), int(self.indices.shape[1])
        native = int(state["q_reduce"].shape[1])
        rank = int(state["k_read"].shape[2])
        vd = int(self.v_indices.shape[1])
        expected = {"q_reduce": (h, native, d), "k_read": (h, d, rank),
                    "v_read": (h, vd, int(state["v_read"].shape[2])),
                    "k_affine": (h, native, d), "v_affine": (h, native, vd),
                    "lift": (h, vd, native)}
        for name, shape in expected.items():
            if tuple(state[name].shape) != shape:
                raise ValueError(f"Bad {name} shape; expected {shape}")
        self.native_dim, self.d, self.vd = native, d, vd
        self.identity_query = _is_identity(state["q_reduce"])
        self.identity_k = _is_identity(state["k_affine"])
        self.identity_lift = vd == native and _is_identity(state["lift"])
        device = device if device is not None else state["k_read"].device

        def dev(t):
            return t.to(device=device, dtype=torch.bfloat16).contiguous()

        v_read, v_affine = state["v_read"], state["v_affine"]
        if not self.identity_lift:
            lift = state["lift"].to(device=device, dtype=torch.float32)       # [h, vd, D]
            v_read = torch.matmul(lift.transpose(1, 2),
                                  v_read.to(device=device, dtype=torch.float32))   # [h, D, r]
            v_affine = torch.matmul(v_affine.to(device=device, dtype=torch.float32),
                                    lift)                                      # [h, D, D]
        self.identity_v = _is_identity(v_affine)
        self.q_reduce = None if self.identity_query else dev(state["q_reduce"])
        self.k_affine = None if self.identity_k else dev(state["k_affine"])
        self.v_affine = None if self.identity_v else dev(v_affine)
        self.k_read = dev(state["k_read"])
        self.v_read = dev(v_read)
        self.heads_dev = self.heads.to(device=device, dtype=torch.int32).contiguous()
        # RoPE acts on complete original pairs only (rope_selected, CN:75-91):
        # reader dims (2j, 2j+1) must be original dims (2p, 2p+1); pair j then
        # rotates with original pair p
        ind = self.indices
        self.rope_complete = bool(torch.equal(ind[:, 1::2], ind[:, ::2] + 1)
                                  and not bool((ind[:, ::2] % 2).any()))
        self.rope_pairs = (ind[:, ::2] // 2).to(device=device, dtype=torch.int32).contiguous() \
            if self.rope_complete else None
        # camera_selected keeps whole 8-dim blocks (CN:117-127): reader block
        # j is original block indices[8j] / 8, whose camera sub-frame is that
        # block's index mod 4
        self.camera_blocks = _whole_blocks(ind) and (d % 8 == 0)
        self.cam_blocks = ((ind[:, ::8] // 8) % 4).to(device=device, dtype=torch.int32) \
            .contiguous() if self.camera_blocks else None
        # the camera of the values and output commutes with the value lift
        # folded into v_read only for an identity or block-selection lift
        self.camera_lift = self.identity_lift or (
            _whole_blocks(self.v_indices) and _is_selection(state["lift"], self.v_indices))

    def tensors(self, rope: bool = False, camera: bool = False) -> ops.ReaderTensors:
        if rope and not self.rope_complete:
            raise ValueError("RoPE mapping must retain complete original pairs")
        if camera and not self.camera_blocks:
            raise ValueError("Invalid MG camera blocks")
        if camera and not self.camera_lift:
            raise ValueError("the camera of a reader group needs an identity or block-selection "
                             "value lift (a learned lift does not commute with P)")
        return ops.ReaderTensors(heads=self.heads_dev, d=self.d, k_read=self.k_read,
                                 v_read=self.v_read, q_reduce=self.q_reduce,
                                 k_affine=self.k_affine, v_affine=self.v_affine,
                                 rope_pairs=self.rope_pairs if rope else None,
                                 cam_blocks=self.cam_blocks if camera else None)


def enabled(prefix: str) -> bool:
    """Whether the codec-native path of `prefix` is switched on (CN:20-21)."""
    return os.environ.get(prefix + "_ENABLE", "0").lower() in {"1", "true", "yes"}


_DIGESTS: dict = {}


def file_sha256(path: str) -> str:
    """SHA-256 hex digest of a file, streamed in 8 MiB blocks and remembered
    per (path, size, mtime) (CN:24-30)."""
    st = os.stat(path)
    key = (str(path), st.st_size, st.st_mtime_ns)
    if key not in _DIGESTS:
        h = hashlib.sha256()
        with open(path, "rb") as f:
            while True:
                block = f.read(8 << 20)
                if not block:
                    break
                h.update(block)
        _DIGESTS[key] = h.hexdigest()
    return _DIGESTS[key]


_READER_BANKS: dict = {}


def get_layer(prefix: str, model: str, layer: int, *, device, heads: int, native_dim: int,
              operator_path: str, sp_rank: int = 0):
    """The reader layer of (sp_rank, layer) from the manifest named by
    `<prefix>_MANIFEST` (format codec_native_manifest_v1, CN:229-275): the
    manifest must be for `model` and bound to the deployed codec operator
    file by SHA-256; each reader checkpoint is checked against its recorded
    SHA-256 and loaded with weights_only=True; uncalibrated readers are
    refused unless `<prefix>_ALLOW_UNCALIBRATED=1`.  Returns (ReaderLayer or
    None for a layer the manifest does not list, manifest); (None, None) when
    the prefix is not enabled."""
    if not enabled(prefix):
        return None, None
    path = Path(os.environ[prefix + "_MANIFEST"]).resolve()
    op_path = str(Path(operator_path).resolve())
    bank_key = (str(path), model, str(device), op_path)
    if bank_key not in _READER_BANKS:
        manifest = json.loads(path.read_text())
        if manifest.get("format") != "codec_native_manifest_v1" or manifest.get("model") != model:
            raise ValueError("Wrong codec-native manifest/model")
        if manifest.get("codec_operator_sha256") != file_sha256(op_path):
            raise ValueError("Reader is not bound to the deployed frozen codec operator")
        _READER_BANKS[bank_key] = (manifest, {})
    manifest, loaded = _READER_BANKS[bank_key]
    entry = manifest["layers"].get(f"{int(sp_rank)}:{int(layer)}")
    if entry is None:
        return None, manifest
    if not entry.get("calibrated", False) and os.environ.get(prefix + "_ALLOW_UNCALIBRATED") != "1":
        raise RuntimeError("Reader is initialization-only; fit and validate before deployment")
    ident = (int(sp_rank), int(layer))
    if ident not in loaded:
        artifact = (path.parent / entry["path"]).resolve()
        if file_sha256(str(artifact)) != entry["sha256"]:
            raise ValueError("Reader checkpoint checksum mismatch")
        payload = torch.load(artifact, map_location="cpu", weights_only=True)
        loaded[ident] = ReaderLayer(payload, device)
    reader = loaded[ident]
    if reader.heads != heads or reader.native_dim != native_dim:
        raise ValueError("Reader head/shard layout mismatch")
    return reader, manifest


class ReaderLayer:
    """The reader groups of one layer (CN:207-224); they must partition the
    heads exactly once (CN:213-215)."""

    def __init__(self, payload: dict, device=None):
        self.groups = [ReaderGroup(g, device) for g in payload["groups"]]
        self.heads = int(payload["heads"])
        self.native_dim = int(payload["native_dim"])
        self.rank = int(payload["rank"])
        all_heads = torch.cat([g.heads for g in self.groups]).tolist()
        if sorted(all_heads) != list(range(self.heads)):
            raise ValueError("Reader groups must partition heads exactly once")


def _low_value_sums(cache_k: Any, cache_v: Any, low: torch.Tensor, device: torch.device):
    """The sufficient statistics of the low value rows (LingBot
    codec_native_attention.py:478-489): the fp32 sum of their bf16 latents
    [B, r], the center sum from the center counts [B, HD] (None without
    centers), the row count and the value operator; None when no row is
    low."""
    items = nanokv_codec.direct_latent_pair_segments(cache_k, cache_v, device=device,
                                                     token_keep=low)
    if not items:
        return None
    latent_sum = center_sum = None
    count = 0
    for item in items:
        latent, (centers, ids), _ = item["v"]
        ls = latent.float().sum(1)
        latent_sum = ls if latent_sum is None else latent_sum + ls
        if centers is not None:
            counts = torch.zeros(ids.shape[0], centers.shape[1], device=device,
                                 dtype=torch.float32)
            counts.scatter_add_(1, ids, torch.ones_like(ids, dtype=torch.float32))
            cs = torch.einsum("bc,bcd->bd", counts,
                              centers.float().expand(ids.shape[0], -1, -1))
            center_sum = cs if center_sum is None else center_sum + cs
        count += int(latent.shape[1])
    part = nanokv_codec.segments_of(cache_v)[0]
    op = nanokv_codec._operator(str(part["kind"]), int(part["layer"]), device)
    return latent_sum, center_sum, count, op


def _mean_bias(op, B: int, HD: int, center_sum, count: int, device) -> torch.Tensor:
    """bf16(mean) + the mean center per batch item, [B, HD] fp32."""
    base = torch.zeros(B, HD, device=device)
    if op["mean"] is not None:
        base = base + op["mean"].to(torch.bfloat16).float()
    if center_sum is not None:
        base = base + center_sum / count
    return base


def compressed_value_mean(cache_k: Any, cache_v: Any, low: torch.Tensor, heads: int,
                          device: torch.device) -> Optional[torch.Tensor]:
    """LingBot's first moment of the low history values (LingBot
    codec_native_attention.py:465-501) from the latent sums and the center
    counts, never the decoded rows: value = W_dec (sum latent / n) +
    bf16(mean) + (sum_c count_c center_c) / n in fp32, per batch item and
    native head, [B, H, 1, D]; None when no row is low."""
    sums = _low_value_sums(cache_k, cache_v, low, device)
    if sums is None:
        return None
    latent_sum, center_sum, count, op = sums
    mean = op["mean"]
    value = torch.nn.functional.linear(latent_sum / count, op["decoder"].float(),
                                       None if mean is None else mean.to(torch.bfloat16).float())
    if center_sum is not None:
        value = value + center_sum / count
    B, HD = value.shape
    return value.reshape(B, heads, 1, HD // heads)


def value_mean_shift(reader: ReaderLayer, cache_k: Any, cache_v: Any, low: torch.Tensor,
                     device: torch.device) -> Optional[torch.Tensor]:
    """The value-mean correction of LingBot's Fast (codec_native_attention.py
    :779-785) as a per-head shift of the low values, [B, H, D] fp32: for
    the heads of each group whose value lift is low-rank (reader value width
    below the native width), mean - projected, where mean is the first moment
    of the full decode (compressed_value_mean) and projected the mean of the
    group's low value reads after the lift; 0 for the other heads.  projected
    is formed from the same latent and center sums through the group's value
    reader (lift folded in: v_read' = lift^T v_read, v_affine' = v_affine
    lift), as the reads are affine in the latent and the center."""
    if not any(g.vd < g.native_dim for g in reader.groups):
        return None
    sums = _low_value_sums(cache_k, cache_v, low, device)
    if sums is None:
        return None
    latent_sum, center_sum, count, op = sums
    H, D = reader.heads, reader.native_dim
    lat = latent_sum / count                                                  # [B, r]
    B = lat.shape[0]
    base = _mean_bias(op, B, H * D, center_sum, count, device)               # [B, HD]
    value_mean = (torch.nn.functional.linear(lat, op["decoder"].float()) + base).reshape(B, H, D)
    base = base.reshape(B, H, D)
    shift = torch.zeros(B, H, D, device=device, dtype=torch.float32)
    for g in reader.groups:
        if g.vd >= g.native_dim:
            continue
        heads = g.heads.to(device)
        proj = torch.einsum("br,hdr->bhd", lat, g.v_read.float())
        aff = base.index_select(1, heads)
        proj = proj + (aff if g.v_affine is None
                       else torch.einsum("bhe,hed->bhd", aff, g.v_affine.float()))
        shift[:, heads] = value_mean.index_select(1, heads) - proj
    return shift


def fast_history_attention(q: torch.Tensor, cache_k: Any, cache_v: Any,
                           k_cur: Optional[torch.Tensor], v_cur: Optional[torch.Tensor],
                           reader: ReaderLayer, protect: torch.Tensor, *,
                           scale: Optional[float] = None, return_lse: bool = False,
                           rope=None, q_pre: Optional[torch.Tensor] = None, q_rope=None,
                           low: Optional[torch.Tensor] = None,
                           camera: Optional[ops.Camera] = None,
                           q_camera: Optional[ops.Camera] = None,
                           visibility: Optional[ops.Visibility] = None,
                           value_mean_correction: bool = False,
                           out_camera: Optional[ops.Camera] = None):
    """NanoKV-Fast history attention of q [B, H, Q, D]: the protected history
    tokens (bool mask [N] over the cache) and the current chunk are attended
    at full width by every head (mg35.py:192-303), the low history tokens
    (bool mask [N], default: the unprotected ones) through each head's reader
    group (mg35.py:315-347), and the two are merged by LSE (CN:33-42, 308).
    Everything runs in one nkv_fast_attend call: every partition's history
    tiles are decoded once into the call's workspace (the staged schedule)
    or into LDS (the key-chunk kernel, reader ranks above 384); no K/V tensor
    is produced.
    Scale: native_dim ** -0.5 (CN:287).
    RoPE (mg35.py:207-214, 305-336): rope = kv_rope(...) or an ops.RopeTable
    of the cached rows; q is then the rotated query, q_pre [B, H, Q, D] the
    pre-RoPE query that the reader groups project, and q_rope the positions of
    the current chunk's queries (query t at row t).
    Camera (mg35.py:253-257, 310-346): camera = kv_camera(P_inv, ...) of the
    cached rows and q_camera the P^T of the query rows; q, k_cur and v_cur are
    then already transformed, q_pre is not; out_camera, P of the query rows,
    goes on the merged output inside the call (None: the caller applies P).
    visibility: which current keys each query sees.
    value_mean_correction: LingBot's first-moment correction of the low
    values of groups with a low-rank value lift (value_mean_shift)."""
    device = q.device
    B, H, Qn, D = (int(x) for x in q.shape)
    if H != reader.heads or D != reader.native_dim:
        raise ValueError("Reader head/shard layout mismatch")
    key, value = nanokv_codec.history_codecs(cache_k, cache_v, device)
    protect = protect.to(device=device, dtype=torch.bool)
    if protect.numel() != key.tokens:
        raise ValueError("protect must have one entry per history token")
    low = ~protect if low is None else low.to(device=device, dtype=torch.bool)
    if low.numel() != key.tokens or bool((low & protect).any()):
        raise ValueError("low must be a mask over the history disjoint from protect")
    if camera is not None and camera.frame_mat.numel() * camera.tokens_per_frame != key.tokens:
        raise ValueError("the camera's frames must cover exactly the cached rows "
                         "(complete equal-sized frames)")
    protect_rows = torch.nonzero(protect).flatten().to(torch.int32).contiguous()
    low_rows = torch.nonzero(low).flatten().to(torch.int32).contiguous()
    qq = q.to(torch.bfloat16).permute(0, 2, 1, 3)
    kc = None if k_cur is None else k_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    vc = None if v_cur is None else v_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    qp = None
    if rope is not None and (q_pre is None or q_rope is None):
        raise ValueError("RoPE needs q_pre and q_rope for the reader groups")
    if camera is not None and (q_pre is None or q_camera is None):
        raise ValueError("the camera needs q_pre and q_camera for the reader groups")
    if q_pre is not None:
        qp = q_pre.to(torch.bfloat16).permute(0, 2, 1, 3)
    groups = [g.tensors(rope=rope is not None, camera=camera is not None) for g in reader.groups]
    shift = value_mean_shift(reader, cache_k, cache_v, low, device) \
        if value_mean_correction else None
    out, lse = ops.fast_attend(qq, kc, vc, key, value, protect_rows, low_rows, groups,
                               softmax_scale=D ** -0.5 if scale is None else scale,
                               return_lse=return_lse, rope=rope, q_pre=qp, q_rope=q_rope,
                               camera=camera, q_camera=q_camera,
                               visibility=visibility if kc is not None else None,
                               low_shift=shift, out_camera=out_camera)
    out = out.permute(0, 2, 1, 3)
    return (out, lse) if return_lse else out
