"""Shared builders for the parity tests: one seeded scenario, two views of it
(device tensors for the HIP path, numpy arrays for the CPU oracle)."""
from __future__ import annotations

import numpy as np
import torch

from nanokv_amd import synth


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16/fp16 tensor -> numpy uint16 bit patterns (host copy)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_u16(a: np.ndarray, dtype=torch.bfloat16, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).to(device)


def scale_name(dtype: torch.dtype) -> str:
    return "fp16" if dtype == torch.float16 else "bf16"


def max_abs_cos(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    diff = float(np.abs(a - b).max()) if a.size else 0.0
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    cos = float(a @ b / (na * nb)) if na > 0 and nb > 0 else (1.0 if na == nb else 0.0)
    return diff, cos


class Scenario:
    """A seeded decode+attend problem encoded by the oracle (so the history
    payload is identical for both sides)."""

    def __init__(self, *, B=1, H=2, D=128, N=200, Q=100, Nc=64, rK=384, rV=256, G=32, C=16,
                 scale_dtype=torch.float16, with_mean=False, id_dtype=torch.uint8,
                 centers=True, seed=0):
        import oracle.oracle as orc
        self.shape = synth.Shape("test", H=H, D=D, N=N, Q=Q, Nc=Nc, rK=rK, rV=rV, G=G, C=max(C, 1),
                                 scale_dtype=scale_dtype, B=B)
        sh = self.shape
        layer = synth.make_layer(sh, seed=seed, with_mean=with_mean)
        self.layer = layer
        self.B, self.H, self.D, self.N, self.Q, self.Nc = B, H, D, N, Q, Nc
        self.G, self.scale_dtype, self.id_dtype = G, scale_dtype, id_dtype
        sname = scale_name(scale_dtype)
        self.hist = []
        for b in range(B):
            item = {}
            for kind, cent, enc, dec, mean in (
                    ("k", layer.centers_k, layer.w_enc_k, layer.w_dec_k, layer.mean_k),
                    ("v", layer.centers_v, layer.w_enc_v, layer.w_dec_v, layer.mean_v)):
                rows = synth.history_rows(sh, cent, N, seed=seed * 100 + b * 10 + (kind == "v"))
                e = orc.encode(rows.numpy(), u16(layer.w_enc_k if kind == "k" else layer.w_enc_v),
                               u16(cent) if centers else None,
                               None if mean is None else mean.numpy(), G, sname, "fp32")
                item[kind] = {
                    "packed": e["packed"], "scales": e["scales"],
                    "w_dec_bf16": u16(dec), "group": G, "scale_dtype": sname,
                    "ids": e["ids"] if centers else None,
                    "centers_bf16": u16(cent) if centers else None,
                    "mean": None if mean is None else mean.numpy(),
                }
            self.hist.append(item)
        g = torch.Generator().manual_seed(seed + 12345)
        self.q = (torch.randn(B, Q, H, D, generator=g) / D ** 0.5).to(torch.bfloat16)
        if Nc:
            kc = [synth.history_rows(sh, layer.centers_k, Nc, seed=seed * 7 + 1000 + b) for b in range(B)]
            vc = [synth.history_rows(sh, layer.centers_v, Nc, seed=seed * 7 + 2000 + b) for b in range(B)]
            self.k_cur = torch.stack(kc).reshape(B, Nc, H, D).to(torch.bfloat16)
            self.v_cur = torch.stack(vc).reshape(B, Nc, H, D).to(torch.bfloat16)
        else:
            self.k_cur = self.v_cur = None
        self.scale = D ** -0.5

    # ---- device side
    def codecs(self, device):
        from nanokv_amd import ops
        if self.N == 0:
            return None, None
        out = []
        for kind in ("k", "v"):
            items = [self.hist[b][kind] for b in range(self.B)]
            packed = torch.from_numpy(np.stack([it["packed"] for it in items])).to(device)
            scales = from_u16(np.stack([it["scales"] for it in items]), self.scale_dtype, device)
            w_dec = from_u16(items[0]["w_dec_bf16"], torch.bfloat16, device)
            ids = centers = mean = None
            if items[0]["ids"] is not None:
                ids = torch.from_numpy(np.stack([it["ids"] for it in items]).astype(np.int64))
                ids = ids.to(self.id_dtype).to(device)
                centers = from_u16(items[0]["centers_bf16"], torch.bfloat16, device)[None]
            if items[0]["mean"] is not None:
                mean = torch.from_numpy(items[0]["mean"]).to(device)
            out.append(ops.Codec(packed=packed, scales=scales, w_dec=w_dec, group=self.G,
                                 ids=ids, centers=centers, mean=mean))
        return out[0], out[1]

    # ---- oracle side
    def reference(self, b, heads=None, **kw):
        import oracle.oracle as orc
        key = self.hist[b]["k"] if self.N else None
        val = self.hist[b]["v"] if self.N else None
        kc = u16(self.k_cur[b]) if self.Nc else None
        vc = u16(self.v_cur[b]) if self.Nc else None
        return orc.decode_attend(u16(self.q[b]), kc, vc, key, val, self.scale, heads=heads,
                                 D=self.D, **kw)


def oracle_groups(payload: dict) -> list:
    """A reader payload (synth.make_readers layout) as the oracle's group
    dicts: bf16 bits per head, None where the matrix is the identity."""
    import torch as _t

    def ident(w):
        return w.shape[-2] == w.shape[-1] and _t.equal(w.float(), _t.eye(w.shape[-1]).expand_as(w))

    out = []
    for g in payload["groups"]:
        out.append({
            "heads": [int(h) for h in g["heads"]],
            "q_reduce": None if ident(g["q_reduce"]) else u16(g["q_reduce"].to(_t.bfloat16)),
            "k_read": u16(g["k_read"].to(_t.bfloat16)),
            "v_read": u16(g["v_read"].to(_t.bfloat16)),
            "k_affine": None if ident(g["k_affine"]) else u16(g["k_affine"].to(_t.bfloat16)),
            "v_affine": None if ident(g["v_affine"]) else u16(g["v_affine"].to(_t.bfloat16)),
            "lift": None if ident(g["lift"]) else u16(g["lift"].to(_t.bfloat16)),
            # camera sub-frame of each 8-dim reader block (camera_selected)
            "cam_blocks": ((g["indices"][:, ::8] // 8) % 4).numpy(),
            "v_cam_blocks": ((g.get("v_indices", g["indices"])[:, ::8] // 8) % 4).numpy(),
        })
    return out


def oracle_codec(cd, b: int = 0, scale_dtype: str = "fp16") -> dict:
    """One batch item of an ops.Codec (flat or a segment table) as the oracle's
    codec dict.  A segment table becomes the concatenation of its segments,
    each segment's ids offset by the rows of the tables before it and the
    tables concatenated: the same center row for every token, so the same
    decode."""
    if cd.segments is None:
        return {"packed": cd.packed[b].cpu().numpy(), "scales": u16(cd.scales[b]),
                "w_dec_bf16": u16(cd.w_dec), "group": cd.group, "scale_dtype": scale_dtype,
                "ids": None if cd.ids is None else cd.ids[b].cpu().numpy().astype(np.int64),
                "centers_bf16": None if cd.centers is None else
                u16(cd.centers[b if cd.centers.shape[0] > 1 else 0]),
                "mean": None if cd.mean is None else cd.mean.cpu().numpy()}
    segs = cd.segments.segments
    ids, tables, base = [], [], 0
    for sg in segs:
        if sg.centers is not None:
            ids.append(sg.ids[b].cpu().numpy().astype(np.int64) + base)
            t = sg.centers[b if sg.centers.shape[0] > 1 else 0]
            tables.append(u16(t))
            base += int(t.shape[0])
    return {"packed": np.concatenate([sg.packed[b].cpu().numpy() for sg in segs]),
            "scales": np.concatenate([u16(sg.scales[b]) for sg in segs]),
            "w_dec_bf16": u16(cd.w_dec), "group": cd.group, "scale_dtype": scale_dtype,
            "ids": np.concatenate(ids) if ids else None,
            "centers_bf16": np.concatenate(tables) if tables else None,
            "mean": None if cd.mean is None else cd.mean.cpu().numpy()}
