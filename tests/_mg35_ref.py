"""Independent restatements of the MG-3.5 hook's routing and visibility, used
as test oracles (test infrastructure: no product code imports this).

route_reference: MG35:155-170 with tensors -- token frame ordinals, the active
  mask from chunk ids, protected_tokens over the frame ordinals
  (CN/core.py:140-152).
keep_reference: MG35:258-283 per (query, key), from the rule as stated there:
  mosaic key j is visible iff hole_keep[j]; the current keys and queries are
  split evenly over the current frames, each frame carrying its chunk id; a
  query of chunk i (i >= 0) sees the current keys of chunk i and the anchors
  (ids < 0); an anchor query sees the anchors only.
"""
import torch

from nanokv_amd import codec_native


def route_reference(frames, chunk_ids, read_chunk, tokens, recent, stride, sink, native):
    n = len(frames)
    ordinal = torch.arange(n).repeat_interleave(tokens // n) if n else torch.empty(0, dtype=torch.long)
    active = torch.ones(tokens, dtype=torch.bool)
    if read_chunk is not None and len(chunk_ids) == n:
        fa = torch.tensor([int(v) < 0 or int(v) == int(read_chunk) for v in chunk_ids],
                          dtype=torch.bool)
        active &= fa.index_select(0, ordinal)
    protect = torch.zeros_like(active)
    if tokens:
        fp = codec_native.protected_tokens(torch.arange(n), recent, stride, sink)
        protect = active & fp.index_select(0, ordinal)
    if native:
        protect = active.clone()
    return protect, active & ~protect


def keep_reference(q_tokens, mosaic_tokens, cur_key_tokens, n_frames, hole_keep, chunk_ids):
    """bool [q_tokens, mosaic + current] as a nested loop, or None if all true."""
    hole = None if hole_keep is None else [bool(x) for x in hole_keep.reshape(-1).tolist()]
    rows = []
    for t in range(q_tokens):
        row = []
        for j in range(mosaic_tokens):
            row.append(True if hole is None else hole[j])
        for c in range(cur_key_tokens):
            if chunk_ids is None or n_frames == 0:
                row.append(True)
                continue
            q_chunk = int(chunk_ids[t // (q_tokens // n_frames)])
            k_chunk = int(chunk_ids[c // (cur_key_tokens // n_frames)])
            if q_chunk < 0:
                row.append(k_chunk < 0)
            else:
                row.append(k_chunk == q_chunk or k_chunk < 0)
        rows.append(row)
    keep = torch.tensor(rows, dtype=torch.bool).reshape(q_tokens, mosaic_tokens + cur_key_tokens)
    return None if bool(keep.all()) else keep
