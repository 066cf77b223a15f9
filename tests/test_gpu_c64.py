"""The C64 center fit on the GPU (nkv_c64_fit) against the oracle: labels
equal and centers bit-exact (both sum each cluster's rows in fp64 in row
order); encode_tensor without a shared table fits, keeps the fit's labels
as ids and stores bf16 centers."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import nanokv_codec as nc, ops, synth
from tests._helpers import u16

pytestmark = pytest.mark.gpu


def _chunk(B, S, HD, C0, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(C0, HD, generator=g) * 2
    pick = torch.randint(0, C0, (B, S), generator=g)
    return (base[pick] + 0.5 * torch.randn(B, S, HD, generator=g)).float()


@pytest.mark.parametrize("B,S,HD,C,iters", [(1, 1560, 3072, 64, 2), (2, 300, 512, 16, 2),
                                            (1, 257, 96, 256, 1), (1, 50, 40, 7, 3),
                                            (2, 64, 128, 8, 0)])
def test_c64_fit_matches_oracle(dev, B, S, HD, C, iters):
    x = _chunk(B, S, HD, max(C // 4, 2), seed=S + C)
    draw = torch.Generator(device="cpu").manual_seed(20260804 + 3)
    init = torch.randperm(S, generator=draw)[:C].to(torch.int32)
    centers, labels = ops.c64_fit(x.to(dev), init.to(dev), iters)
    torch.cuda.synchronize()
    rc, rl = orc.c64_fit(x.numpy(), init.numpy(), iters)
    assert np.array_equal(labels.cpu().numpy().astype(np.int64), rl)
    assert np.array_equal(centers.cpu().numpy(), rc)


def test_encode_tensor_c64_path(dev, monkeypatch):
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    monkeypatch.setenv("MG35_KVCODEC_C64_CLUSTERS", "24")
    sh = synth.Shape("c64", H=2, D=128, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=9, with_mean=True)
    nc.register_operator("k", 11, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev),
                         mean=lay.mean_k.to(dev))
    nc.register_centers("k", 11, None)
    x = synth.history_rows(sh, lay.centers_k, 200, seed=4)[None].to(torch.bfloat16)
    payload = nc.encode_tensor("k", 11, x.to(dev))
    draw = torch.Generator(device="cpu").manual_seed(20260804 + 11)
    init = torch.randperm(200, generator=draw)[:24]
    rc, rl = orc.c64_fit(x.float().numpy(), init.numpy(), 2)
    assert np.array_equal(payload["ids"][0].cpu().numpy().astype(np.int64), rl[0])
    assert np.array_equal(u16(payload["centers"][0]), orc.f32_to_bf16(rc[0]))
    # the payload decodes (adding back each row's stored center) as the oracle does
    dec = nc.decode_value(payload, dtype=torch.bfloat16, device=dev)[0].float().cpu().numpy()
    view = nc.codec_view(payload, dev)
    ref = orc.bf16_to_f32(orc.decode(
        view.packed[0].cpu().numpy(), u16(view.scales[0]), u16(view.w_dec), view.group, "fp16",
        view.ids[0].cpu().numpy().astype(np.int64), u16(view.centers[0]), view.mean.cpu().numpy()))
    np.testing.assert_allclose(dec, ref, rtol=2 ** -7, atol=2 ** -7)
