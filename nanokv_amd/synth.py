"""Seeded synthetic inputs for the benchmark configurations.

The benchmark shapes have no public checkpoint or dataset behind them, so
history K/V rows are generated with the structure NanoKV's codec exploits:
token i = center[u_i] + G_i diag(1/sqrt(k)) U + eps_i with u_i uniform over
the shared centers, G ~ N(0,1) [N, 64], U an orthonormal [64, HD] basis and
eps ~ N(0, 0.05^2).  Rows are rounded to bf16 (the dtype a backbone's K/V
projection produces) and handed to the encoder as fp32.

Everything is generated with torch.Generator objects seeded explicitly, on
the device requested, so the GPU path and the CPU oracle see the same bits.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass(frozen=True)
class Shape:
    """One attention layer call: H heads of width D, N history tokens (compressed),
    Q query tokens, Nc uncompressed current-chunk tokens, ranks rK/rV, scale group
    G, C shared centers."""
    name: str
    H: int
    D: int
    N: int
    Q: int
    Nc: int
    rK: int
    rV: int
    G: int
    C: int
    scale_dtype: torch.dtype = torch.float16
    B: int = 1

    @property
    def HD(self) -> int:
        return self.H * self.D

    def flops(self) -> dict:
        """Algorithmic flops: attention 4*Q*(N+Nc)*HD and a decode GEMM counted
        once per history token 2*N*(rK+rV)*HD."""
        att_hist = 4.0 * self.B * self.Q * self.N * self.HD
        att_cur = 4.0 * self.B * self.Q * self.Nc * self.HD
        dec = 2.0 * self.B * self.N * (self.rK + self.rV) * self.HD
        return {"attention_history": att_hist, "attention_current": att_cur, "decode": dec,
                "total": att_hist + att_cur + dec}

    def fast_flops(self, n_protect: int, full_heads=None, d: int = None) -> dict:
        """Algorithmic flops of a NanoKV-Fast call: the native partition (the
        n_protect protected rows and the current keys, every head, full
        width), the low partition (identity-reader heads at full width, the
        other heads with K/Q width d and V width D), the full decode of the
        protected rows (all heads) and of the low rows of identity heads, and
        the reader reads of the low rows for the other heads."""
        full_heads = FAST_FULL_HEADS if full_heads is None else full_heads
        d = FAST_READER_D if d is None else d
        nf, nr = len(full_heads), self.H - len(full_heads)
        low = self.N - n_protect
        att_native = 4.0 * self.B * self.Q * (n_protect + self.Nc) * self.HD
        att_low = (4.0 * self.B * self.Q * low * self.D * nf
                   + 2.0 * self.B * self.Q * low * (d + self.D) * nr)
        dec_full = (2.0 * self.B * n_protect * (self.rK + self.rV) * self.HD
                    + 2.0 * self.B * low * (self.rK + self.rV) * self.D * nf)
        reads = 2.0 * self.B * low * (self.rK * d + self.rV * self.D) * nr
        return {"attention_native": att_native, "attention_low": att_low, "decode_full": dec_full,
                "reader_reads": reads, "total": att_native + att_low + dec_full + reads}

    def coeff_stream_bytes(self) -> float:
        """Unique bytes of the compressed history read by one call: packed codes,
        group scales and center ids of K and V."""
        id_bytes = 1 if self.C <= 256 else 2
        # packed codes (r/2 bytes) + 2-byte group scales, for K and V, + one id each
        per_tok = self.rK // 2 + self.rV // 2 + 2 * (self.rK // self.G) + 2 * (self.rV // self.G)
        return float(self.B * self.N * (per_tok + 2 * id_bytes))


# BASELINE.json configurations (index = position in its "configs" list).
CONFIGS = {
    # the CPU reference case: per-32 fp16 scales, fixed orthonormal 512 x 64
    # encoder / decoder (make_layer(..., orthonormal_codec=True))
    0: Shape("cfg0_cpu_h8_d64", H=8, D=64, N=2048, Q=256, Nc=256, rK=64, rV=64, G=32, C=16,
             scale_dtype=torch.float16),
    1: Shape("cfg1_h24_d128_n12480_q1560", H=24, D=128, N=12480, Q=1560, Nc=1560, rK=384,
             rV=384, G=32, C=256),
    2: Shape("cfg2_h24_d128_n49920_q780", H=24, D=128, N=49920, Q=780, Nc=780, rK=384, rV=256,
             G=32, C=1024),
    # NanoKV-Fast on the config-1 shapes (reader layout in make_readers)
    3: Shape("cfg3_fast_h24_d128_n12480_q1560", H=24, D=128, N=12480, Q=1560, Nc=1560, rK=384,
             rV=384, G=32, C=256),
}

# Config 3: 6 of 24 heads keep full-width reads (identity readers), the rest
# read K and Q through random 384->32 / 128->32 projections with V at full
# width; the last 2 frames of 1,560 tokens are protected for every head.
FAST_FULL_HEADS = (0, 4, 8, 12, 16, 20)
FAST_READER_D = 32
FAST_FRAME_TOKENS = 1560
FAST_RECENT_FRAMES = 2


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def orthonormal(rows: int, cols: int, seed: int, device="cpu") -> torch.Tensor:
    """Orthonormal [rows, cols] (rows <= cols) from the QR of a Gaussian, fp32."""
    g = _gen(seed, "cpu")
    a = torch.randn(cols, rows, generator=g, dtype=torch.float64)
    qm, rm = torch.linalg.qr(a)
    qm = qm * torch.sign(torch.diagonal(rm))[None, :]
    return qm.T.contiguous().to(device=device, dtype=torch.float32)


@dataclass
class Layer:
    """Codec operators and shared centers of one layer (K and V)."""
    centers_k: torch.Tensor   # [C, HD] bf16
    centers_v: torch.Tensor
    w_enc_k: torch.Tensor     # [rK, HD] bf16
    w_dec_k: torch.Tensor     # [HD, rK] bf16
    w_enc_v: torch.Tensor
    w_dec_v: torch.Tensor
    mean_k: Optional[torch.Tensor] = None   # [HD] fp32
    mean_v: Optional[torch.Tensor] = None


def make_layer(shape: Shape, seed: int = 0, device="cpu", orthonormal_codec: bool = False,
               with_mean: bool = False) -> Layer:
    """Random codec operators for one layer.

    Decoders are random N(0,1)/sqrt(r) bf16 [HD, r] (independent for K and V)
    and encoders their least-squares inverse bf16(W^T * r / HD); with
    orthonormal_codec the encoder is a fixed orthonormal [r, HD] projection
    and the decoder its transpose (config 0).  Centers are N(0,1) in bf16.
    """
    g = _gen(seed * 1000 + 17, "cpu")
    HD = shape.HD

    def codec(r, sub):
        if orthonormal_codec:
            enc = orthonormal(r, HD, seed * 1000 + sub)
            dec = enc.T.contiguous()
        else:
            dec = torch.randn(HD, r, generator=g) / r ** 0.5
            enc = dec.T * (r / HD)
        return (enc.to(torch.bfloat16).contiguous().to(device),
                dec.to(torch.bfloat16).contiguous().to(device))

    ck = torch.randn(shape.C, HD, generator=g).to(torch.bfloat16).to(device)
    cv = torch.randn(shape.C, HD, generator=g).to(torch.bfloat16).to(device)
    ek, dk = codec(shape.rK, 1)
    ev, dv = codec(shape.rV, 2)
    mk = mv = None
    if with_mean:
        mk = (0.1 * torch.randn(HD, generator=g)).to(device)
        mv = (0.1 * torch.randn(HD, generator=g)).to(device)
    return Layer(ck, cv, ek, dk, ev, dv, mk, mv)


def history_rows(shape: Shape, centers: torch.Tensor, n: int, seed: int,
                 device="cpu") -> torch.Tensor:
    """n structured K or V rows [n, HD] (bf16 values as fp32)."""
    g = _gen(seed, device)
    HD = shape.HD
    basis = orthonormal(64, HD, seed + 7, device)
    u = torch.randint(0, centers.shape[0], (n,), generator=g, device=device)
    gcoef = torch.randn(n, 64, generator=g, device=device)
    decay = torch.arange(1, 65, device=device, dtype=torch.float32).rsqrt()
    eps = 0.05 * torch.randn(n, HD, generator=g, device=device)
    rows = centers.to(device).float()[u] + (gcoef * decay) @ basis + eps
    return rows.to(torch.bfloat16).float()


def queries(shape: Shape, seed: int, device="cpu") -> torch.Tensor:
    """q [B, Q, H, D] bf16 ~ N(0,1)/sqrt(D)."""
    g = _gen(seed, device)
    q = torch.randn(shape.B, shape.Q, shape.H, shape.D, generator=g, device=device)
    return (q / shape.D ** 0.5).to(torch.bfloat16)


def make_readers(shape: Shape, layer: Layer, seed: int = 0, full_heads=FAST_FULL_HEADS,
                 d: int = FAST_READER_D) -> dict:
    """A NanoKV-Fast reader payload (the layout CN/core.py:207-224 loads) for
    config 3: one identity group over full_heads (q_reduce = k_affine =
    v_affine = lift = I, k_read / v_read = the head's decoder rows, so its
    low read equals the full decode) and one group over the other heads with
    random N(0,1)/sqrt(fan-in) bf16 q_reduce [D, d], k_read [d, rK] and
    k_affine [D, d], v_read = the head's V decoder rows and identity
    v_affine / lift.  Tensors are fp32 on the CPU (bf16-representable), as
    reader checkpoints store them."""
    g = _gen(seed * 1000 + 29, "cpu")
    H, D = shape.H, shape.D
    full = [h for h in range(H) if h in set(full_heads)]
    low = [h for h in range(H) if h not in set(full_heads)]
    wk = layer.w_dec_k.float().cpu().reshape(H, D, shape.rK)
    wv = layer.w_dec_v.float().cpu().reshape(H, D, shape.rV)
    eye = torch.eye(D)

    def bf(t):
        return t.to(torch.bfloat16).float()

    def group(heads, dd, identity):
        n = len(heads)
        hs = torch.tensor(heads, dtype=torch.long)
        if identity:
            qr = eye.expand(n, D, D).clone()
            kr = wk[hs].clone()
            ka = eye.expand(n, D, D).clone()
        else:
            qr = bf(torch.randn(n, D, dd, generator=g) / D ** 0.5)
            kr = bf(torch.randn(n, dd, shape.rK, generator=g) / shape.rK ** 0.5)
            ka = bf(torch.randn(n, D, dd, generator=g) / D ** 0.5)
        return {"heads": hs, "indices": torch.arange(dd).expand(n, dd).clone(),
                "v_indices": torch.arange(D).expand(n, D).clone(),
                "q_reduce": qr, "k_read": kr, "v_read": wv[hs].clone(),
                "k_affine": ka, "v_affine": eye.expand(n, D, D).clone(),
                "lift": eye.expand(n, D, D).clone()}

    groups = [group(full, D, True)]
    if low:
        groups.append(group(low, d, False))
    return {"groups": groups, "heads": H, "native_dim": D, "rank": shape.rK}


def fast_protect_mask(shape: Shape, frame_tokens: int = FAST_FRAME_TOKENS,
                      recent: int = FAST_RECENT_FRAMES, device="cpu") -> torch.Tensor:
    """bool [N]: history tokens of the last `recent` frames (protected)."""
    frames = (shape.N + frame_tokens - 1) // frame_tokens
    frame_of = torch.arange(shape.N, device=device) // frame_tokens
    return frame_of >= frames - recent


def camera_matrices(sets: int, seed: int, sub_frames: int = 4):
    """PRoPE projection matrices as _prepare_projection_matrices builds them
    (camera_rope.py:195-222): for each of `sets` matrix sets and each
    sub-frame a camera with a random rotation, a translation of N(0, 0.3)
    per axis and normalised focal lengths in [0.8, 1.2]; P = lift(K) . V,
    P^T, and P^-1 = invert_SE3(V) . lift(K^-1) (camera_rope.py:318-337).
    Returns (P, P_T, P_inv), fp32 [1, sets, sub_frames, 4, 4] on the CPU."""
    g = _gen(seed * 1000 + 41, "cpu")
    n = sets * sub_frames
    q, r = torch.linalg.qr(torch.randn(n, 3, 3, generator=g, dtype=torch.float64))
    rot = q * torch.sign(torch.diagonal(r, dim1=-2, dim2=-1))[:, None, :]
    rot = torch.where(torch.det(rot)[:, None, None] < 0, -rot, rot)      # det +1
    t = 0.3 * torch.randn(n, 3, generator=g, dtype=torch.float64)
    f = 0.8 + 0.4 * torch.rand(n, 2, generator=g, dtype=torch.float64)
    view = torch.zeros(n, 4, 4, dtype=torch.float64)
    view[:, :3, :3], view[:, :3, 3], view[:, 3, 3] = rot, t, 1.0
    k = torch.zeros(n, 4, 4, dtype=torch.float64)
    k[:, 0, 0], k[:, 1, 1], k[:, 2, 2], k[:, 3, 3] = f[:, 0], f[:, 1], 1.0, 1.0
    k_inv = torch.zeros_like(k)
    k_inv[:, 0, 0], k_inv[:, 1, 1], k_inv[:, 2, 2], k_inv[:, 3, 3] = 1 / f[:, 0], 1 / f[:, 1], 1.0, 1.0
    view_inv = torch.zeros_like(view)
    view_inv[:, :3, :3] = rot.transpose(-1, -2)
    view_inv[:, :3, 3] = -(rot.transpose(-1, -2) @ t[:, :, None])[:, :, 0]
    view_inv[:, 3, 3] = 1.0
    P = (k @ view).float()
    P_inv = (view_inv @ k_inv).float()
    shape = (1, sets, sub_frames, 4, 4)
    return (P.reshape(shape).contiguous(), P.transpose(-1, -2).reshape(shape).contiguous(),
            P_inv.reshape(shape).contiguous())
