"""The segment-list paths of the codec API against the oracle:
select_value (MG:612-694) keeps fully selected segments and decodes, slices
and re-encodes a cut one (the re-encode's C64 fit, ids and centers checked
bit for bit against the oracle on the decoded rows it was given);
direct_latent_pair_segments (MG:707-798) exposes each kept segment's latent
rows, ids, center tables and mean without reconstructing K/V."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import nanokv_codec as nc, synth
from tests._helpers import u16

pytestmark = pytest.mark.gpu

LAYER = 17


@pytest.fixture
def cache(dev, monkeypatch):
    monkeypatch.setenv("MG35_KVCODEC_C64_CLUSTERS", "24")
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    sh = synth.Shape("sel", H=2, D=128, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=LAYER, with_mean=True)
    for kind, enc, dec, mean in (("k", lay.w_enc_k, lay.w_dec_k, lay.mean_k),
                                 ("v", lay.w_enc_v, lay.w_dec_v, lay.mean_v)):
        nc.register_operator(kind, LAYER, encoder=enc.to(dev), decoder=dec.to(dev),
                             mean=mean.to(dev))
        nc.register_centers(kind, LAYER, None)
    ck = cv = None
    for i, n in enumerate((100, 150, 120)):
        k = synth.history_rows(sh, lay.centers_k, n, seed=60 + i)[None].to(torch.bfloat16).to(dev)
        v = synth.history_rows(sh, lay.centers_v, n, seed=70 + i)[None].to(torch.bfloat16).to(dev)
        ck = nc.concat_values(ck, nc.encode_tensor("k", LAYER, k))
        cv = nc.concat_values(cv, nc.encode_tensor("v", LAYER, v))
    return ck, cv


def test_select_value_cut_segment(dev, cache):
    ck, _ = cache
    segs = nc.segments_of(ck)
    wanted = list(range(0, 100)) + list(range(120, 250)) + list(range(250, 370))
    sel = nc.select_value(ck, torch.tensor(wanted), kind="k", layer=LAYER, dtype=torch.bfloat16,
                          device=dev)
    out = nc.segments_of(sel)
    assert len(out) == 3
    assert out[0] is segs[0] and out[2] is segs[2]       # whole segments are reused
    cut = out[1]
    assert tuple(cut["shape"]) == (1, 130, 256)
    # the re-encode sees the decoded rows 20..149 of segment 1 (MG:641-690)
    rows = nc.decode_value(segs[1], dtype=torch.bfloat16, device=dev)[:, 20:150].float()
    x = rows.cpu().numpy()
    draw = torch.Generator(device="cpu").manual_seed(20260804 + LAYER)
    init = torch.randperm(130, generator=draw)[:24]
    rc, rl = orc.c64_fit(x, init.numpy(), 2)
    assert np.array_equal(cut["ids"][0].cpu().numpy().astype(np.int64), rl[0])
    assert np.array_equal(u16(cut["centers"][0]), orc.f32_to_bf16(rc[0]))
    # its codes and scales are the quantiser's on the projected residual
    view = nc.codec_view(cut, dev)
    res = orc.residual_bf16(x[0], orc.f32_to_bf16(rc[0]), rl[0], view.mean.cpu().numpy())
    coeff = orc.project(res, u16(nc._operator("k", LAYER, dev)["encoder"]))
    ref_packed, ref_scales, _ = orc.quant_pack(coeff.astype(np.float32), 32, "fp16", "fp32")
    # the GPU sums the projection in fp32; codes may differ only where a
    # coefficient sits on a rounding boundary
    mism = np.count_nonzero(view.packed[0].cpu().numpy() != ref_packed)
    assert mism <= 0.002 * ref_packed.size, mism
    # order and range errors, as the reference raises them (MG:625-694)
    with pytest.raises(RuntimeError, match="sorted in-range"):
        nc.select_value(ck, torch.tensor([5, 3]), kind="k", layer=LAYER, dtype=torch.bfloat16,
                        device=dev)
    with pytest.raises(RuntimeError, match="sorted in-range"):
        nc.select_value(ck, torch.tensor(list(range(100)) + [400]), kind="k", layer=LAYER,
                        dtype=torch.bfloat16, device=dev)
    assert nc.select_value(ck, torch.tensor([], dtype=torch.long), kind="k", layer=LAYER,
                           dtype=torch.bfloat16, device=dev) is None


def test_direct_latent_pair_segments(dev, cache):
    ck, cv = cache
    keep = torch.zeros(370, dtype=torch.bool)
    keep[10:60] = True          # segment 0, partly
    keep[300:370] = True        # segment 2, partly; segment 1 has nothing kept
    res = nc.direct_latent_pair_segments(ck, cv, device=dev, token_keep=keep)
    assert len(res) == 2
    segs_k, segs_v = nc.segments_of(ck), nc.segments_of(cv)
    for item, si, lo, hi in ((res[0], 0, 10, 60), (res[1], 2, 300, 370)):
        start = (0, 100, 250)[si]
        assert item["length"] == hi - lo
        assert torch.equal(item["logical_indices"].cpu(), torch.arange(lo, hi))
        for kind, part in (("k", segs_k[si]), ("v", segs_v[si])):
            latent, (centers, ids), mean = item[kind]
            view = nc.codec_view(part, dev)
            local = np.arange(lo - start, hi - start)
            ref = orc.unpack_latent(view.packed[0].cpu().numpy(), u16(view.scales[0]), 128, 32,
                                    "fp16", row_index=local)
            assert np.array_equal(u16(latent[0]), ref)
            assert np.array_equal(ids[0].cpu().numpy(), view.ids[0].cpu().numpy()[local])
            assert torch.equal(centers, view.centers.float())
            assert torch.equal(mean, view.mean)
    with pytest.raises(ValueError, match="length mismatch"):
        nc.direct_latent_pair_segments(ck, cv, device=dev, token_keep=keep[:-1])


def test_pca_rung_payloads(dev, monkeypatch):
    """MG35_WORLDPLAY_RUNG=pca: encode_tensor projects the rows themselves (no
    centers, semantic False, MG:338-342); the fused read of such segments
    meets the bar against the oracle's decode-then-attend."""
    from nanokv_amd import codec_native
    from tests._helpers import max_abs_cos, oracle_codec
    monkeypatch.setenv("MG35_WORLDPLAY_RUNG", "pca")
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    sh = synth.Shape("pca", H=2, D=128, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=3)
    for kind, enc, dec in (("k", lay.w_enc_k, lay.w_dec_k), ("v", lay.w_enc_v, lay.w_dec_v)):
        nc.register_operator(kind, 41, encoder=enc.to(dev), decoder=dec.to(dev))
    ck = cv = None
    for i in range(3):
        k = synth.history_rows(sh, lay.centers_k, 90, seed=80 + i)[None].to(torch.bfloat16).to(dev)
        v = synth.history_rows(sh, lay.centers_v, 90, seed=90 + i)[None].to(torch.bfloat16).to(dev)
        pk, pv = nc.encode_tensor("k", 41, k), nc.encode_tensor("v", 41, v)
        assert pk["semantic"] is False and pk["centers"] is None and pk["ids"] is None
        ck, cv = nc.concat_values(ck, pk), nc.concat_values(cv, pv)
    g = torch.Generator().manual_seed(2)
    q = (torch.randn(1, 2, 300, 128, generator=g) / 128 ** 0.5).to(torch.bfloat16).to(dev)
    out = codec_native.codec_history_attention(q, ck, cv)
    key, value = nc.history_codecs(ck, cv, dev)
    assert key.segments is not None and not key.segments.has_centers
    ref, _ = orc.decode_attend(u16(q[0].permute(1, 0, 2)), None, None,
                               oracle_codec(key, 0, "bf16"), oracle_codec(value, 0, "bf16"),
                               128 ** -0.5)
    diff, cos = max_abs_cos(out[0].permute(1, 0, 2).float().cpu().numpy(), ref)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
