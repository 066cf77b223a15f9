"""INT8 codec operators on the GPU (nkv_int8_pack / nkv_int8_dequant) against
the oracle, bit-exact, and the prepacked operator file
(mg35_worldplay_operator_int8_v1) loaded by preload_operator_weights: the
registered bf16 weights are the GPU dequant, and encoding / decoding with
them equals registering those bf16 weights directly."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import nanokv_codec as nc, ops, synth
from tests._helpers import u16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols,group", [(384, 3072, 0), (384, 3072, 128), (3072, 384, 0),
                                             (100, 77, 7), (5, 1, 1)])
def test_int8_pack_dequant_bitexact(dev, rows, cols, group):
    g = torch.Generator().manual_seed(rows + cols)
    w = torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g))
    if rows > 3:
        w[3] = 0.0  # a zero row: the 1e-12 floor
    packed = ops.int8_pack(w.to(dev), group)
    torch.cuda.synchronize()
    rq, rs = orc.int8_pack(w.numpy(), group)
    assert packed["group_size"] == (group or cols)
    assert np.array_equal(packed["qweight"].cpu().numpy(), rq)
    assert np.array_equal(u16(packed["scale"]), rs)
    out = ops.int8_dequant(packed)
    torch.cuda.synchronize()
    assert np.array_equal(u16(out), orc.int8_dequant(rq, rs, group or cols))


def test_preload_prepacked_operator_file(dev, tmp_path, monkeypatch):
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    sh = synth.Shape("int8", H=2, D=128, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=6, with_mean=True)
    # the artifact directories the entries record must be this deployment's
    for name in ("basis", "dec_k", "qat_v"):
        (tmp_path / name).mkdir()
    monkeypatch.setenv("MG35_KVCODEC_BASIS_DIR", str(tmp_path / "basis"))
    monkeypatch.setenv("MG35_KVCODEC_DECODER_DIR_K", str(tmp_path / "dec_k"))
    monkeypatch.setenv("MG35_KVCODEC_DECODER_DIR_V", str(tmp_path / "qat_v"))
    monkeypatch.delenv("MG35_WORLDPLAY_RUNG", raising=False)
    monkeypatch.delenv("MG35_KVCODEC_CENTER_STORAGE", raising=False)
    monkeypatch.delenv("NANOKV_PORTABLE_CODEC_SHA256", raising=False)
    entries = {}
    for kind, enc, dec, mean in (("k", lay.w_enc_k, lay.w_dec_k, lay.mean_k),
                                 ("v", lay.w_enc_v, lay.w_dec_v, lay.mean_v)):
        pe = nc.pack_operator(enc.float(), dev, group_size=0)
        pd = nc.pack_operator(dec.float(), dev, group_size=64)
        entries[f"{kind}:07"] = {
            "mean": mean.cpu(),
            "encoder": {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in pe.items()},
            "decoder": {k: (v.cpu() if torch.is_tensor(v) else v) for k, v in pd.items()},
            "basis_dir": str(tmp_path / "basis"),
            "decoder_dir": str(tmp_path / "dec_k") if kind == "k" else "",
            "qat_dir": str(tmp_path / "qat_v") if kind == "v" else "",
        }
    path = tmp_path / "codec.pt"
    torch.save({"format": nc.PREPACKED_FORMAT, "entries": entries, "rung": "full",
                "center_storage": "bf16", "center_block_size": 64}, path)
    nc.preload_operator_weights(dev, str(path))
    for kind in ("k", "v"):
        e = entries[f"{kind}:07"]
        op = nc._operator(kind, 7, dev)
        for part in ("encoder", "decoder"):
            p = e[part]
            ref = orc.int8_dequant(p["qweight"].numpy(), u16(p["scale"]), p["group_size"])
            assert np.array_equal(u16(op[part]), ref), (kind, part)
    # encode + decode through the int8 operators = through their bf16 dequant
    nc.register_centers("k", 7, lay.centers_k.to(dev))
    nc.register_centers("v", 7, lay.centers_v.to(dev))
    x = synth.history_rows(sh, lay.centers_k, 50, seed=3).to(dev)[None].to(torch.bfloat16)
    payload = nc.encode_tensor("k", 7, x)
    dec_int8 = nc.decode_value(payload, dtype=torch.bfloat16, device=dev)
    op = nc._operator("k", 7, dev)
    nc.register_operator("k", 8, encoder=op["encoder"], decoder=op["decoder"], mean=op["mean"])
    nc.register_centers("k", 8, lay.centers_k.to(dev))
    payload8 = nc.encode_tensor("k", 8, x)
    for key in ("packed_codes", "scale", "ids"):
        assert torch.equal(payload[key], payload8[key]), key
    assert torch.equal(dec_int8, nc.decode_value(payload8, dtype=torch.bfloat16, device=dev))
