"""The reference-compatible API end to end on the GPU: encode_tensor chunks,
concat_values segment lists, decode_value / decode_pair_selected and the
fused codec_history_attention, against the oracle's decode-then-attend."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, nanokv_codec as nc, synth
from tests._helpers import max_abs_cos, u16

pytestmark = pytest.mark.gpu

H, D = 2, 128


def _setup(dev, layer, shared, monkeypatch, r=128, C=16):
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    monkeypatch.setenv("MG35_KVCODEC_C64_CLUSTERS", "8")
    sh = synth.Shape("api", H=H, D=D, N=0, Q=0, Nc=0, rK=r, rV=r, G=32, C=C)
    lay = synth.make_layer(sh, seed=layer, with_mean=True)
    nc.register_operator("k", layer, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev),
                         mean=lay.mean_k.to(dev))
    nc.register_operator("v", layer, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev),
                         mean=lay.mean_v.to(dev))
    nc.register_centers("k", layer, lay.centers_k.to(dev) if shared else None)
    nc.register_centers("v", layer, lay.centers_v.to(dev) if shared else None)
    return sh, lay


def _oracle_rows(payload, dev):
    """Oracle decode of one encoded segment (batch item 0) -> float32 [S, HD]."""
    view = nc.codec_view(payload, dev)
    return orc.bf16_to_f32(orc.decode(
        view.packed[0].cpu().numpy(), u16(view.scales[0]), u16(view.w_dec), view.group, "fp16",
        view.ids[0].cpu().numpy().astype(np.int64), u16(view.centers[0]),
        view.mean.cpu().numpy()))


@pytest.mark.parametrize("shared", [True, False])
def test_encode_concat_attend(dev, monkeypatch, shared):
    layer = 3 if shared else 4
    sh, lay = _setup(dev, layer, shared, monkeypatch)
    chunks_k, chunks_v = [], []
    cache_k = cache_v = None
    for c in range(3):
        k = synth.history_rows(sh, lay.centers_k, 40, seed=10 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 40, seed=20 + c).to(dev)[None].to(torch.bfloat16)
        pk, pv = nc.encode_tensor("k", layer, k), nc.encode_tensor("v", layer, v)
        assert pk["codec"] == nc.CODEC and pk["scale"].shape == (1, 40, 4)
        chunks_k.append(pk)
        chunks_v.append(pv)
        cache_k, cache_v = nc.concat_values(cache_k, pk), nc.concat_values(cache_v, pv)
    assert nc.value_shape(cache_k) == (1, 120, H * D)
    # decode_value: per-segment decode, concatenated, vs the oracle
    dk = nc.decode_value(cache_k, dtype=torch.bfloat16, device=dev)[0].float().cpu().numpy()
    ref_k = np.concatenate([_oracle_rows(p, dev) for p in chunks_k], 0)
    np.testing.assert_allclose(dk, ref_k, rtol=2 ** -7, atol=2 ** -7)
    ref_v = np.concatenate([_oracle_rows(p, dev) for p in chunks_v], 0)
    # decode_pair_selected returns exactly the decode_value rows
    keep = torch.zeros(120, dtype=torch.bool)
    keep[[0, 5, 41, 119]] = True
    sk, sv = nc.decode_pair_selected(cache_k, cache_v, keep, dtype=torch.bfloat16, device=dev)
    full_k = nc.decode_value(cache_k, dtype=torch.bfloat16, device=dev)
    assert torch.equal(sk, full_k[:, keep.to(dev)])
    # fused history attention vs decode-then-attend
    g = torch.Generator().manual_seed(7)
    q = (torch.randn(1, H, 50, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 16, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 16, D, generator=g).to(torch.bfloat16).to(dev)
    out, lse = codec_native.codec_history_attention(q, cache_k, cache_v, kc, vc, return_lse=True)
    kk = np.concatenate([ref_k.reshape(120, H, D), orc.bf16_to_f32(u16(kc[0].permute(1, 0, 2)))], 0)
    vv = np.concatenate([ref_v.reshape(120, H, D), orc.bf16_to_f32(u16(vc[0].permute(1, 0, 2)))], 0)
    ro, rl = orc.attention(orc.bf16_to_f32(u16(q[0])), kk.transpose(1, 0, 2), vv.transpose(1, 0, 2),
                           D ** -0.5)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ro)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - rl).max() < 2e-3


def test_attention_lse_and_merge(dev):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, H, 30, D, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, H, 70, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(1, H, 70, D, generator=g).to(torch.bfloat16).to(dev)
    o1, l1 = codec_native.attention_lse(q, k[:, :, :25], v[:, :, :25])
    o2, l2 = codec_native.attention_lse(q, k[:, :, 25:], v[:, :, 25:])
    om, lm = codec_native.merge(o1, l1, o2, l2)
    oj, lj = codec_native.attention_lse(q, k, v)
    diff, cos = max_abs_cos(om.float().cpu().numpy(), oj.float().cpu().numpy())
    assert diff < 1e-2 and cos > 0.9999
    ref, ref_l = orc.attention(q[0].float().cpu().numpy(), k[0].float().cpu().numpy(),
                               v[0].float().cpu().numpy(), D ** -0.5)
    diff, cos = max_abs_cos(oj[0].float().cpu().numpy(), ref)
    assert diff <= 2e-2 and cos >= 0.9995
    oe, le = codec_native.attention_lse(q, k[:, :, :0], v[:, :, :0])
    assert torch.all(oe == 0) and torch.all(torch.isneginf(le))


def test_history_attention_with_read_time_rope(dev, monkeypatch):
    """codec_history_attention(rope=kv_rope(...)) against the reference's order
    of operations: decode_pair_values, rope_apply(cache_k_pre, cache_freqs),
    attention (wan_video_dit.py:497-627)."""
    layer = 5
    sh, lay = _setup(dev, layer, True, monkeypatch)
    cache_k = cache_v = None
    chunks_k, chunks_v = [], []
    for c in range(3):
        k = synth.history_rows(sh, lay.centers_k, 40, seed=30 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 40, seed=40 + c).to(dev)[None].to(torch.bfloat16)
        pk, pv = nc.encode_tensor("k", layer, k), nc.encode_tensor("v", layer, v)
        chunks_k.append(pk)
        chunks_v.append(pv)
        cache_k, cache_v = nc.concat_values(cache_k, pk), nc.concat_values(cache_v, pv)
    from nanokv_amd import ops
    freqs = ops.rope_bands(D, 64)  # the model's (temporal, row, column) bands
    positions, gh, gw = [9, 4, 12], 5, 8  # three cached frames of 5 x 8 tokens
    rope = codec_native.kv_rope(freqs, positions, gh, gw, dev)
    g = torch.Generator().manual_seed(11)
    q = (torch.randn(1, H, 37, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 9, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 9, D, generator=g).to(torch.bfloat16).to(dev)
    out, lse = codec_native.codec_history_attention(q, cache_k, cache_v, kc, vc,
                                                    return_lse=True, rope=rope)
    ref_k = np.concatenate([_oracle_rows(p, dev) for p in chunks_k], 0)
    ref_v = np.concatenate([_oracle_rows(p, dev) for p in chunks_v], 0)
    table = orc.kv_freqs(tuple(b.numpy() for b in freqs), positions, gh, gw)
    k_rot = orc.bf16_to_f32(orc.rope_apply(orc.f32_to_bf16(ref_k.reshape(120, H, D)), table))
    kk = np.concatenate([k_rot, orc.bf16_to_f32(u16(kc[0].permute(1, 0, 2)))], 0)
    vv = np.concatenate([ref_v.reshape(120, H, D), orc.bf16_to_f32(u16(vc[0].permute(1, 0, 2)))], 0)
    ro, rl = orc.attention(orc.bf16_to_f32(u16(q[0])), kk.transpose(1, 0, 2),
                           vv.transpose(1, 0, 2), D ** -0.5)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ro)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - rl).max() < 2e-3


def test_history_attention_with_rope_and_camera(dev, monkeypatch):
    """codec_history_attention(rope=..., camera=kv_camera(...)) against the
    reference's order for the decoded history: rope_apply, then P^-1 of each
    frame on keys and values (CN/mg35.py:54-71), then attention."""
    layer = 6
    sh, lay = _setup(dev, layer, True, monkeypatch)
    cache_k = cache_v = None
    chunks_k, chunks_v = [], []
    for c in range(3):
        k = synth.history_rows(sh, lay.centers_k, 40, seed=50 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 40, seed=60 + c).to(dev)[None].to(torch.bfloat16)
        pk, pv = nc.encode_tensor("k", layer, k), nc.encode_tensor("v", layer, v)
        chunks_k.append(pk)
        chunks_v.append(pv)
        cache_k, cache_v = nc.concat_values(cache_k, pk), nc.concat_values(cache_v, pv)
    from nanokv_amd import ops
    freqs = ops.rope_bands(D, 64)
    positions, gh, gw = [2, 7, 3], 5, 8
    rope = codec_native.kv_rope(freqs, positions, gh, gw, dev)
    g = torch.Generator().manual_seed(12)
    P_inv = torch.eye(4).expand(1, 2, 4, 4, 4) + 0.3 * torch.randn(1, 2, 4, 4, 4, generator=g)
    frames = [1, 0, 1]
    camera = codec_native.kv_camera(P_inv, frames, gh * gw, dev)
    q = (torch.randn(1, H, 37, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 9, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 9, D, generator=g).to(torch.bfloat16).to(dev)
    out, lse = codec_native.codec_history_attention(q, cache_k, cache_v, kc, vc,
                                                    return_lse=True, rope=rope, camera=camera)
    ref_k = np.concatenate([_oracle_rows(p, dev) for p in chunks_k], 0)
    ref_v = np.concatenate([_oracle_rows(p, dev) for p in chunks_v], 0)
    table = orc.kv_freqs(tuple(b.numpy() for b in freqs), positions, gh, gw)
    row_mats = P_inv[0].numpy()[np.repeat(frames, gh * gw)]
    k_rot = orc.rope_apply(orc.f32_to_bf16(ref_k.reshape(120, H, D)), table)
    k_cam = orc.bf16_to_f32(orc.camera_apply(k_rot, row_mats))
    v_cam = orc.bf16_to_f32(orc.camera_apply(orc.f32_to_bf16(ref_v.reshape(120, H, D)), row_mats))
    kk = np.concatenate([k_cam, orc.bf16_to_f32(u16(kc[0].permute(1, 0, 2)))], 0)
    vv = np.concatenate([v_cam, orc.bf16_to_f32(u16(vc[0].permute(1, 0, 2)))], 0)
    ro, rl = orc.attention(orc.bf16_to_f32(u16(q[0])), kk.transpose(1, 0, 2),
                           vv.transpose(1, 0, 2), D ** -0.5)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ro)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - rl).max() < 2e-3
