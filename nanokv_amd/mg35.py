"""Matrix-Game 3.5 NanoKV-Fast attention hook on the gfx950 kernels.

The drop-in for models/Matrix-Game-3.5/fast/codec_native/mg35.py (cited as
MG35:line): maybe_attention keeps its call signature and its contract (None
for "use the native path", the projected block attention otherwise, and the
cache commit), so causal_self_attention_kv (wan_video_dit.py:438-452) changes
only its import.  Underneath, the whole read is one nkv_fast_attend call:

  protected history rows   decoded in-kernel, RoPE from the per-row cache_freqs
                           table, camera P^-1 in-kernel (MG35:192-215, 253-257)
  mosaic + current keys    k_native / v_raw as they are, under the hole and
                           chunk-id visibility bits (MG35:258-300)
  low history rows         each reader group's projections, RoPE and camera
                           blocks in-kernel (MG35:305-347)
  merge                    log-sum-exp of the partitions (CN/core.py:33-42)

and the output camera P goes on the merged output inside the same call
(o_camera; it commutes with the merge and with block-selection lifts).  The frame routing
(which history rows are active, protected or low, MG35:146-190) is computed
on the host from the frame metadata lists, as the reference's metadata cache
does (CN/metadata_cache.py:48-72).
"""
from __future__ import annotations

import os
from typing import Any, Callable, Optional

import torch

from . import codec_native, nanokv_codec, ops

MODEL = "matrix-game-3.5"
PREFIX = "MG35_CODEC_NATIVE"


# ---------------------------------------------------------------- cache writes
def _identity_write(layer_idx: int, k_pre: torch.Tensor, v_raw: torch.Tensor):
    return k_pre, v_raw


# The cache-write hook the commit runs before encoding (the reference's
# causal_kv_codec.process_cache_write, which in worldplay_method mode returns
# its inputs unchanged after writing optional statistics files).
process_cache_write: Callable = _identity_write


def set_cache_write_hook(fn: Optional[Callable]) -> None:
    """Install the (layer_idx, k_pre, v_raw) -> (k_pre, v_raw) cache-write hook
    (None: the identity)."""
    global process_cache_write
    process_cache_write = fn or _identity_write


def _commit(cache, cur_k_pre, cur_v_raw, *, layer_idx, cur_frames, cur_positions,
            cur_cache_chunk_ids):
    """Append the chunk's pre-RoPE K and raw V as immutable codec segments and
    extend the frame, position and chunk-id metadata (MG35:73-97)."""
    cur_k_pre, cur_v_raw = process_cache_write(int(layer_idx), cur_k_pre.detach(),
                                               cur_v_raw.detach())
    k_value = nanokv_codec.encode_tensor("k", int(layer_idx), cur_k_pre)
    v_value = nanokv_codec.encode_tensor("v", int(layer_idx), cur_v_raw)
    positions = list(cur_frames) if cur_positions is None else [int(v) for v in cur_positions]
    chunk_ids = ([-1] * len(cur_frames) if cur_cache_chunk_ids is None
                 else [int(v) for v in cur_cache_chunk_ids])
    if len(positions) != len(cur_frames) or len(chunk_ids) != len(cur_frames):
        raise ValueError("cache frame metadata length mismatch")
    if nanokv_codec.value_shape(cache.get("k")) is None:
        cache["k"], cache["v"] = k_value, v_value
        cache["positions"], cache["frames"], cache["chunk_ids"] = (positions, list(cur_frames),
                                                                   chunk_ids)
    else:
        old_frames = list(cache.get("frames", []))
        old_chunks = list(cache.get("chunk_ids", [-1] * len(old_frames)))
        cache["k"] = nanokv_codec.concat_values(cache["k"], k_value)
        cache["v"] = nanokv_codec.concat_values(cache["v"], v_value)
        cache["positions"] = list(cache.get("positions", cache.get("frames", []))) + positions
        cache["frames"] = old_frames + list(cur_frames)
        cache["chunk_ids"] = old_chunks + chunk_ids


# ---------------------------------------------------------------- routing
def route(frames, chunk_ids, read_chunk, tokens: int, recent: int, stride: int, sink: int,
          native: bool) -> dict:
    """Frame-level routing of the cached history (MG35:146-185 and its metadata
    cache CN/metadata_cache.py:48-72): a frame is active when it has no chunk
    id (< 0) or the read chunk's; active frames are protected when recent,
    sink or every `stride`-th older frame (CN/core.py:140-152), or all of them
    under native_history; the other active frames are low.  Returns the
    per-token masks (CPU) and counts."""
    if min(recent, stride, sink) < 0:
        raise ValueError("Negative protection policy")
    if tokens and (not frames or tokens % len(frames)):
        raise ValueError("cache tokens must contain complete equal-sized frames")
    n = len(frames)
    per = tokens // n if n else 0
    active = [True] * n
    if read_chunk is not None and len(chunk_ids) == n:
        active = [int(c) < 0 or int(c) == int(read_chunk) for c in chunk_ids]
    old = max(0, n - recent)
    selected = set(range(old, n)) | set(range(min(sink, n)))
    if stride and old:
        selected.update(range(old - 1, -1, -stride))
    protected = [a and (native or i in selected) for i, a in enumerate(active)]
    low = [a and not p for a, p in zip(active, protected)]
    protect_cpu = torch.tensor(protected, dtype=torch.bool).repeat_interleave(per)
    low_cpu = torch.tensor(low, dtype=torch.bool).repeat_interleave(per)
    return dict(protect=protect_cpu, low=low_cpu, active_count=sum(active) * per,
                protected_count=sum(protected) * per, low_count=sum(low) * per)


def _expand_frames(frames, tokens: int):
    """MG35:27-35: one frame id per token of equal-sized frames."""
    if not frames:
        return []
    if tokens % len(frames):
        raise ValueError("tokens must contain complete equal-sized frames")
    return [int(f) for f in frames for _ in range(tokens // len(frames))]


def visibility_keep(q_tokens: int, mosaic_tokens: int, cur_key_tokens: int, cur_frames,
                    hole_keep: Optional[torch.Tensor],
                    cur_cache_chunk_ids) -> Optional[torch.Tensor]:
    """Which mosaic + current keys each current query sees (MG35:258-283):
    mosaic keys by hole_keep, current keys by chunk id (a query of chunk i sees
    chunk i and the anchors (ids < 0); an anchor query sees the anchors).
    bool [q_tokens, mosaic + current] on the CPU, or None when every key is
    visible to every query."""
    keep = torch.ones(mosaic_tokens + cur_key_tokens, dtype=torch.bool)
    if hole_keep is not None:
        keep[:mosaic_tokens] = hole_keep.detach().to("cpu", torch.bool).reshape(-1)
    mask = keep[None].expand(q_tokens, -1).clone()
    if cur_cache_chunk_ids is not None and len(cur_frames):
        ids = torch.as_tensor([int(v) for v in cur_cache_chunk_ids], dtype=torch.long)
        if q_tokens % len(cur_frames) or cur_key_tokens % len(cur_frames):
            raise RuntimeError("Current CUR token count must be divisible by cur_frames for "
                               "chunk masking")
        q_ids = ids.repeat_interleave(q_tokens // len(cur_frames))
        k_ids = ids.repeat_interleave(cur_key_tokens // len(cur_frames))
        key_anchor, query_anchor = k_ids < 0, q_ids < 0
        current_keep = torch.where(query_anchor[:, None], key_anchor[None],
                                   (q_ids[:, None] == k_ids[None]) | key_anchor[None])
        mask[:, mosaic_tokens:] &= current_keep
    return None if bool(mask.all()) else mask


def _frame_camera(mats: torch.Tensor, frames, tokens: int, device) -> ops.Camera:
    """Camera of `tokens` rows in equal-sized frames whose camera indices are
    `frames` (the frames _viewmats selects, MG35:38-51)."""
    if not frames or tokens % len(frames):
        raise ValueError("PRoPE frame count must divide the token sequence")
    return ops.Camera(mats.to(device=device, dtype=torch.float32).contiguous(),
                      torch.as_tensor([int(f) for f in frames], dtype=torch.int32, device=device),
                      tokens // len(frames), "full")


def _rope_table(freqs, disable_t_pairs: int, device) -> ops.RopeTable:
    """The per-row RoPE table of freqs [rows, 1, D/2] complex; with
    prope_disable_t_rope the temporal pairs are the identity (MG35:212-213)."""
    f = torch.as_tensor(freqs)
    if disable_t_pairs:
        f = f.clone()
        f[..., :disable_t_pairs] = 1
    return ops.RopeTable.from_freqs(f, device)


def _native_low_segment(out, lse, groups, qp, all_k_pre, v_raw, native_low, low_keep, freqs_cur,
                        t_pairs, disable_native_rope, camera_info, mosaic_frames, cur_frames,
                        mosaic_tokens, q_rope, q_cam, out_cam, B, H, D):
    """The low_native segment (MG35:241-249, 324-347), merged last into each
    reader group's heads of out [B, Sq, H, D] (lse [B, H, Sq]): the moved
    tokens' pre-RoPE keys and values read through the group's k_affine /
    v_affine (the value lift folded in, as for the codec rows), rotated on
    the reader pairs at their own positions and multiplied by their frames'
    P^-1; the group query (q_reduce, RoPE, P^T) attends them at width 128 with
    its reader columns zero-padded (nkv_reader_rows, then nkv_attend: the
    zero columns add nothing to q.k); P of the query rows on the output; LSE
    merge."""
    device = out.device
    Sk = int(native_low.numel())
    sel = torch.nonzero(native_low).flatten().to(device)
    k_low = all_k_pre.view(B, Sk, H, D).index_select(1, sel)
    v_low = v_raw.view(B, Sk, H, D).index_select(1, sel)
    low_rope = None
    if not disable_native_rope:
        low_rope = _rope_table(torch.as_tensor(freqs_cur).index_select(0, sel.cpu()), t_pairs,
                               device)
    low_cam = None
    if camera_info is not None:
        P_inv = camera_info[1][2]
        # all_current_frames of MG35:245
        tok_frames = (_expand_frames(list(mosaic_frames), mosaic_tokens)
                      + _expand_frames(list(cur_frames), Sk - mosaic_tokens))
        frames_low = [tok_frames[i] for i in sel.tolist()]
        low_cam = ops.Camera(P_inv.to(device=device, dtype=torch.float32).contiguous(),
                             torch.as_tensor(frames_low, dtype=torch.int32, device=device), 1,
                             "full")
    vis = None if low_keep is None else ops.Visibility.from_bool(low_keep, device)
    out = out.clone()
    lse = lse.clone()
    for g in groups:
        heads = g.heads.long()
        q_g = ops.reader_rows(qp.to(torch.bfloat16), g.heads, g.q_reduce, rope=q_rope,
                              pairs=g.rope_pairs if q_rope is not None else None, camera=q_cam,
                              blocks=g.cam_blocks if q_cam is not None else None, out_width=D)
        k_g = ops.reader_rows(k_low, g.heads, g.k_affine, rope=low_rope,
                              pairs=g.rope_pairs if low_rope is not None else None,
                              camera=low_cam, blocks=g.cam_blocks if low_cam is not None else None,
                              out_width=D)
        v_g = ops.reader_rows(v_low, g.heads, g.v_affine, camera=low_cam, out_width=D)
        o_g, l_g = ops.attend(q_g, k_g, v_g, None, None, softmax_scale=D ** -0.5,
                              visibility=vis)
        if out_cam is not None:
            o_g = ops.camera_apply(o_g, out_cam)
        a = out.index_select(2, heads).contiguous()
        la = lse.index_select(1, heads).transpose(1, 2).contiguous()
        m, lm = ops.lse_merge(a, la, o_g.contiguous(), l_g.transpose(1, 2).contiguous())
        out.index_copy_(2, heads, m)
        lse.index_copy_(1, heads, lm.transpose(1, 2).contiguous())
    return out


# ---------------------------------------------------------------- the hook
@torch.no_grad()
def maybe_attention(self_attn, q_pre, q_native, k_native, v_raw, cur_k_pre, freqs_cur,
                    camera_info, *, layer_idx, num_heads, mosaic_tokens, cur_frames,
                    cur_positions, mosaic_frames, cache, cache_freqs, cache_frames,
                    cache_read_chunk_id, cur_cache_chunk_ids, write_cache, hole_keep, a1_pass,
                    all_k_pre=None):
    """Return projected block attention, or None for the untouched native path
    (MG35:100-357)."""
    if os.environ.get("MG35_CODEC_NATIVE_ENABLE", "0").lower() not in {"1", "true", "yes"}:
        return None
    if os.environ.get("MG35_KVCODEC_MODE", "").lower() != "worldplay_method":
        raise RuntimeError("MG codec-native attention requires the frozen worldplay_method cache")
    if a1_pass is not None:
        raise RuntimeError("codec-native deployment and legacy A1 training cannot run together")
    operator_path = os.environ["MG35_KVCODEC_PREPACKED_OPERATOR_PATH"]
    dim = q_pre.shape[-1] // num_heads
    reader, manifest = codec_native.get_layer(PREFIX, MODEL, int(layer_idx), device=q_pre.device,
                                              heads=num_heads, native_dim=dim,
                                              operator_path=operator_path)
    shape = None if cache is None else nanokv_codec.value_shape(cache.get("k"))
    cache_tokens = 0 if shape is None else int(shape[1])
    frames = list(cache_frames or [])
    chunk_ids = [] if cache is None else list(cache.get("chunk_ids", []))
    if reader is None:
        return None
    use_camera = camera_info is not None
    if self_attn.prope_camera_layout != "full" and use_camera:
        raise RuntimeError("calibrated MG low PRoPE currently supports only the formal full layout")

    policy = dict(manifest.get("policy", {}))
    policy.update(manifest.get("layer_policy", {}).get(str(layer_idx), {}))
    recent = int(policy.get("recent_native_frames", 0))
    stride = int(policy.get("anchor_stride", 0))
    sink = int(policy.get("sink_native_frames", 0))
    # low_native: the separately calibrated extension that reads mosaic and /
    # or current tokens through the readers instead of natively
    # (MG35:171-175, 241-249, 324-347)
    low_native = policy.get("low_native", "none")
    Sk = int(k_native.shape[1])
    native_low = torch.zeros(Sk, dtype=torch.bool)
    if cache_tokens and low_native != "none":
        if low_native in ("all", "mosaic"):
            native_low[:mosaic_tokens] = True
        if low_native in ("all", "current"):
            native_low[mosaic_tokens:] = True
    r = route(frames, chunk_ids, cache_read_chunk_id, cache_tokens, recent, stride, sink,
              bool(policy.get("native_history", False)))
    # no old low-dimensional history: the native path is cheaper and
    # numerically authoritative (MG35:187-190)
    if r["low_count"] == 0 and not bool(native_low.any()):
        return None
    if bool(native_low.any()) and all_k_pre is None:
        raise ValueError("low_native needs all_k_pre, the pre-RoPE keys of the mosaic and "
                         "current tokens")

    device = q_pre.device
    B, D, H = int(q_pre.shape[0]), reader.native_dim, num_heads
    Sq = int(q_native.shape[1]) - mosaic_tokens
    q = q_native[:, mosaic_tokens:].reshape(B, Sq, H, D)
    qp = q_pre[:, mosaic_tokens:].reshape(B, Sq, H, D)
    kc = k_native.reshape(B, Sk, H, D)
    vc = v_raw.reshape(B, Sk, H, D)

    disable_native_rope = bool(self_attn.use_prope and use_camera and
                               self_attn.prope_disable_native_rope)
    t_pairs = int(self_attn.rope_t_pairs) if (self_attn.use_prope and use_camera and
                                              self_attn.prope_disable_t_rope) else 0
    kv_rope = q_rope = None
    if not disable_native_rope:
        kv_rope = _rope_table(cache_freqs, t_pairs, device)
        q_rope = _rope_table(freqs_cur[mosaic_tokens:], t_pairs, device)

    kv_cam = q_cam = out_cam = None
    if use_camera:
        P, P_T, P_inv = camera_info[1]
        kv_cam = _frame_camera(P_inv, frames, cache_tokens, device)
        q_cam = _frame_camera(P_T, cur_frames, Sq, device)
        out_cam = _frame_camera(P, cur_frames, Sq, device)
        # the native query and the mosaic / current keys take P^T and P^-1 of
        # their frames (_native_prope, MG35:54-71)
        q = ops.camera_apply(q, q_cam)
        kc, vc = kc.clone(), vc.clone()
        if mosaic_tokens:
            mcam = _frame_camera(P_inv, mosaic_frames, mosaic_tokens, device)
            ops.camera_apply(kc[:, :mosaic_tokens], mcam, out=kc[:, :mosaic_tokens])
            ops.camera_apply(vc[:, :mosaic_tokens], mcam, out=vc[:, :mosaic_tokens])
        if Sk > mosaic_tokens:
            ccam = _frame_camera(P_inv, cur_frames, Sk - mosaic_tokens, device)
            ops.camera_apply(kc[:, mosaic_tokens:], ccam, out=kc[:, mosaic_tokens:])
            ops.camera_apply(vc[:, mosaic_tokens:], ccam, out=vc[:, mosaic_tokens:])

    keep = visibility_keep(Sq, mosaic_tokens, Sk - mosaic_tokens, list(cur_frames), hole_keep,
                           cur_cache_chunk_ids)
    low_keep = None
    if bool(native_low.any()):
        # the native partition keeps the other tokens; the moved tokens keep
        # their visibility in their own segment (MG35:284-286)
        full = torch.ones(Sq, Sk, dtype=torch.bool) if keep is None else keep.cpu()
        low_keep = full[:, native_low]
        low_keep = None if bool(low_keep.all()) else low_keep
        keep = full & ~native_low[None, :]
    vis = None if keep is None else ops.Visibility.from_bool(keep, device)

    key, value = nanokv_codec.history_codecs(cache["k"], cache["v"], device)
    protect_rows = torch.nonzero(r["protect"]).flatten().to(torch.int32).to(device)
    low_rows = torch.nonzero(r["low"]).flatten().to(torch.int32).to(device)
    groups = [g.tensors(rope=kv_rope is not None, camera=use_camera) for g in reader.groups]
    out, lse = ops.fast_attend(q.to(torch.bfloat16), kc.to(torch.bfloat16), vc.to(torch.bfloat16),
                               key, value, protect_rows, low_rows, groups,
                               softmax_scale=reader.native_dim ** -0.5, return_lse=True,
                               rope=kv_rope, q_pre=qp.to(torch.bfloat16), q_rope=q_rope,
                               camera=kv_cam, q_camera=q_cam, visibility=vis, out_camera=out_cam)
    if bool(native_low.any()):
        out = _native_low_segment(out, lse, groups, qp, all_k_pre, v_raw, native_low,
                                  low_keep, freqs_cur, t_pairs, disable_native_rope, camera_info,
                                  mosaic_frames, cur_frames, mosaic_tokens, q_rope, q_cam,
                                  out_cam, B, H, D)
    result = torch.zeros_like(q_native)
    result[:, mosaic_tokens:] = out.reshape(B, Sq, H * D).to(q_native.dtype)
    if write_cache and cache is not None:
        _commit(cache, cur_k_pre, v_raw[:, mosaic_tokens:], layer_idx=layer_idx,
                cur_frames=cur_frames, cur_positions=cur_positions,
                cur_cache_chunk_ids=cur_cache_chunk_ids)
    return self_attn.o(result)
