"""Codec-native attention on the gfx950 kernels.

Mirrors the partition attention and merge helpers of the reference's
models/Matrix-Game-3.5/fast/codec_native/core.py (cited as CN:line) and the
history read of the NanoKV hook (wan_video_dit.py:488-627, decode_pair_values
followed by attention), with the decode fused into the attention kernel:

  attention_lse(q, k, v)           CN:45-72   uncompressed partition, (O, lse)
  merge(out_a, lse_a, out_b, lse_b) CN:33-42  exact LSE merge of partitions
  protected_tokens(frame_ids, ...) CN:140-152 frame-level protection policy
  codec_history_attention(q, cache, k_cur, v_cur)
                                   decode-then-attend of a paired K/V codec
                                   cache plus the current chunk, fused
                                   (nkv_attend); K/V are never materialised

Tensors follow the reference's [B, H, S, D] layout; nothing here runs on the
CPU.
"""
from __future__ import annotations

import math
from typing import Any, Optional

import torch

from . import nanokv_codec, ops


def attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                  mask: Optional[torch.Tensor] = None, *, scale: Optional[float] = None):
    """softmax(q k^T * scale) v with its natural-log LSE for [B, H, S, D]
    inputs (CN:45-72).  An empty key set gives (0, -inf) (CN:48-49).
    Boolean visibility masks are not supported by the fused kernel."""
    if mask is not None:
        raise NotImplementedError("attention masks are not supported by nkv_attend")
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    qq = q.to(torch.bfloat16).permute(0, 2, 1, 3)
    if k.shape[-2] == 0:
        out, lse = ops.attend(qq.contiguous(), None, None, softmax_scale=scale)
    else:
        out, lse = ops.attend(qq.contiguous(), k.to(torch.bfloat16).permute(0, 2, 1, 3),
                              v.to(torch.bfloat16).permute(0, 2, 1, 3), softmax_scale=scale)
    return out.permute(0, 2, 1, 3).to(q.dtype), lse


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


def codec_history_attention(q: torch.Tensor, cache_k: Any, cache_v: Any,
                            k_cur: Optional[torch.Tensor] = None,
                            v_cur: Optional[torch.Tensor] = None, *,
                            scale: Optional[float] = None, return_lse: bool = False):
    """Attention of q [B, H, Q, D] over [decoded history; current chunk] where
    the history is the paired codec cache (nanokv_codec payloads or segment
    lists) and k_cur/v_cur [B, H, Nc, D] are uncompressed.  Equivalent to the
    reference's decode_pair_values + attention (wan_video_dit.py:497-627)
    with the decode fused into nkv_attend."""
    device = q.device
    B, H, Qn, D = (int(x) for x in q.shape)
    key = value = None
    if cache_k is not None and nanokv_codec.value_shape(cache_k) is not None \
            and nanokv_codec.value_shape(cache_k)[1] > 0:
        key, value = nanokv_codec.history_codecs(cache_k, cache_v, device)
    qq = q.to(torch.bfloat16).permute(0, 2, 1, 3)
    kc = None if k_cur is None else k_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    vc = None if v_cur is None else v_cur.to(torch.bfloat16).permute(0, 2, 1, 3)
    out, lse = ops.attend(qq, kc, vc, key, value,
                          softmax_scale=D ** -0.5 if scale is None else scale,
                          return_lse=return_lse)
    out = out.permute(0, 2, 1, 3)
    return (out, lse) if return_lse else out
