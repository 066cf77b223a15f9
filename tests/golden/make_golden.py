"""Writes the small golden fixtures in this directory from the CPU oracle.

The reference ships no tensors or test vectors for this path, so these
fixtures freeze the oracle's outputs on seeded inputs: the CPU suite checks
the oracle still reproduces them, and the GPU suite checks the HIP kernels
against them.  Run from the repository root:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle.oracle as orc  # noqa: E402

OUT = Path(__file__).resolve().parent


def bf16(x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


def main():
    rng = np.random.default_rng(20260804)
    fx = {}
    # quantiser cases: (rows, r, group, scale dtype, quant mode)
    for name, (rows, r, g, sd, qm) in {
        "q_g32_fp16_fp32": (16, 384, 32, "fp16", "fp32"),
        "q_row_bf16_bf16": (16, 384, 384, "bf16", "bf16"),
        "q_g64_bf16_fp32": (16, 256, 64, "bf16", "fp32"),
    }.items():
        x = (rng.standard_normal((rows, r)) * np.exp(rng.standard_normal((rows, 1)))).astype(np.float32)
        x[0] = 0.0
        packed, scales, _ = orc.quant_pack(x, g, sd, qm)
        fx[f"{name}__coeff"] = x
        fx[f"{name}__packed"] = packed
        fx[f"{name}__scales"] = scales
    # assignment + decode + attention on a tiny layer: H=2, D=128, r=64, G=32, C=8
    H, D, r, G, C, N, Qn, Nc = 2, 128, 64, 32, 8, 64, 24, 16
    HD = H * D
    centers = bf16(rng.standard_normal((C, HD)))
    w_dec = bf16(rng.standard_normal((HD, r)) / np.sqrt(r))
    w_enc = bf16(orc.bf16_to_f32(w_dec).T * (r / HD))
    mean = (0.1 * rng.standard_normal(HD)).astype(np.float32)
    u = rng.integers(0, C, N)
    rows = orc.bf16_to_f32(bf16(orc.bf16_to_f32(centers)[u] + 0.3 * rng.standard_normal((N, HD))))
    enc = orc.encode(rows, w_enc, centers, mean, G, "fp16", "fp32")
    q = bf16(rng.standard_normal((Qn, H, D)) / np.sqrt(D))
    kc = bf16(rng.standard_normal((Nc, H, D)))
    vc = bf16(rng.standard_normal((Nc, H, D)))
    codec = dict(packed=enc["packed"], scales=enc["scales"], w_dec_bf16=w_dec, group=G,
                 scale_dtype="fp16", ids=enc["ids"], centers_bf16=centers, mean=mean)
    decoded = orc.decode(**codec)
    out, lse = orc.decode_attend(q, kc, vc, codec, codec, D ** -0.5, D=D)
    fx.update({
        "layer__rows": rows, "layer__centers": centers, "layer__w_enc": w_enc,
        "layer__w_dec": w_dec, "layer__mean": mean, "layer__ids": enc["ids"].astype(np.int32),
        "layer__coeff": enc["coeff"], "layer__packed": enc["packed"], "layer__scales": enc["scales"],
        "layer__decoded": decoded, "layer__q": q, "layer__k_cur": kc, "layer__v_cur": vc,
        "layer__out": out.astype(np.float32), "layer__lse": lse.astype(np.float32),
    })
    np.savez_compressed(OUT / "codec_small.npz", **fx)
    print(f"wrote {OUT / 'codec_small.npz'} ({len(fx)} arrays)")


if __name__ == "__main__":
    main()
