"""Golden fixtures (tests/golden/codec_small.npz, written by
tests/golden/make_golden.py): the CPU oracle must reproduce them exactly and
the HIP kernels must match them (bit-exact codes/scales/ids, tolerance for
the fused attention)."""
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as orc

FX = np.load(Path(__file__).resolve().parent / "golden" / "codec_small.npz")
QUANT = {"q_g32_fp16_fp32": (32, "fp16", "fp32"), "q_row_bf16_bf16": (384, "bf16", "bf16"),
         "q_g64_bf16_fp32": (64, "bf16", "fp32")}


@pytest.mark.parametrize("name", sorted(QUANT))
def test_oracle_reproduces_quant_fixtures(name):
    g, sd, qm = QUANT[name]
    packed, scales, _ = orc.quant_pack(FX[f"{name}__coeff"], g, sd, qm)
    assert np.array_equal(packed, FX[f"{name}__packed"])
    assert np.array_equal(scales, FX[f"{name}__scales"])


def test_oracle_reproduces_layer_fixture():
    e = orc.encode(FX["layer__rows"], FX["layer__w_enc"], FX["layer__centers"], FX["layer__mean"],
                   32, "fp16", "fp32")
    assert np.array_equal(e["ids"], FX["layer__ids"])
    assert np.array_equal(e["packed"], FX["layer__packed"])
    assert np.array_equal(e["scales"], FX["layer__scales"])
    dec = orc.decode(FX["layer__packed"], FX["layer__scales"], FX["layer__w_dec"], 32, "fp16",
                     FX["layer__ids"], FX["layer__centers"], FX["layer__mean"])
    assert np.array_equal(dec, FX["layer__decoded"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(QUANT))
def test_hip_quant_matches_fixtures(dev, name):
    import torch
    from nanokv_amd import ops
    g, sd, qm = QUANT[name]
    dt = torch.float16 if sd == "fp16" else torch.bfloat16
    packed, scales = ops.quant_pack(torch.from_numpy(FX[f"{name}__coeff"]).to(dev), g, dt, qm)
    assert np.array_equal(packed.cpu().numpy(), FX[f"{name}__packed"])
    assert np.array_equal(scales.cpu().view(torch.int16).numpy().view(np.uint16),
                          FX[f"{name}__scales"])


@pytest.mark.gpu
def test_hip_layer_matches_fixture(dev):
    import torch
    from nanokv_amd import ops
    from tests._helpers import from_u16, max_abs_cos
    rows = torch.from_numpy(FX["layer__rows"]).to(dev)
    centers = from_u16(FX["layer__centers"], torch.bfloat16, dev)
    w_enc = from_u16(FX["layer__w_enc"], torch.bfloat16, dev)
    w_dec = from_u16(FX["layer__w_dec"], torch.bfloat16, dev)
    mean = torch.from_numpy(FX["layer__mean"]).to(dev)
    ids = ops.assign(rows, centers, torch.int32)
    assert np.array_equal(ids.cpu().numpy(), FX["layer__ids"])
    codec = ops.Codec(packed=torch.from_numpy(FX["layer__packed"])[None].to(dev),
                      scales=from_u16(FX["layer__scales"], torch.float16, dev)[None],
                      w_dec=w_dec, group=32, ids=ids.to(torch.uint8)[None],
                      centers=centers[None], mean=mean)
    dec = ops.decode(codec, 256)[0].float().cpu().numpy()
    np.testing.assert_allclose(dec, orc.bf16_to_f32(FX["layer__decoded"]), rtol=2 ** -7, atol=2 ** -7)
    q = from_u16(FX["layer__q"], torch.bfloat16, dev)[None]
    kc = from_u16(FX["layer__k_cur"], torch.bfloat16, dev)[None]
    vc = from_u16(FX["layer__v_cur"], torch.bfloat16, dev)[None]
    out, lse = ops.attend(q, kc, vc, codec, codec)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), FX["layer__out"])
    assert diff <= 2e-2 and cos >= 0.9995
    assert np.abs(lse[0].cpu().numpy() - FX["layer__lse"]).max() < 2e-3
