"""GPU parity at BASELINE's other configurations, encoded on the GPU and
checked against the oracle on the same bits:
  cfg0  the encoder at HD = 512, r = 64, 16 centers, per-32 fp16 scales
        (orthonormal 512 x 64 codec), its decode, and the whole layer's
        attention at D = 64;
  cfg2  N = 49,920, Q = Nc = 780, 1,024 centers with 16-bit ids, rK = 384 /
        rV = 256: bit-exact assignment at C = 1,024 and the full fused call on
        a head subset;
  cfg4  a two-layer slice of the rollout step: per layer the fused call over
        16 frames x 1,560 rows of history, then the chunk's K / V encoded
        into a slot of the history (the commit), then the call again."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import ops, synth
from tests._helpers import max_abs_cos, u16

pytestmark = pytest.mark.gpu

MAX_ABS, MIN_COS = 2e-2, 0.9995


def _oracle_codec(e, dec, cent, G, mean=None):
    return {"packed": e["packed"].cpu().numpy(), "scales": u16(e["scales"]), "w_dec_bf16": u16(dec),
            "group": G, "scale_dtype": "fp16", "ids": e["ids"].cpu().numpy().astype(np.int64),
            "centers_bf16": u16(cent), "mean": mean}


def test_cfg0_encoder_and_decode(dev):
    sh = synth.CONFIGS[0]
    assert (sh.HD, sh.rK, sh.C, sh.G, sh.scale_dtype) == (512, 64, 16, 32, torch.float16)
    lay = synth.make_layer(sh, seed=0, device=dev, orthonormal_codec=True)
    for kind, cent, enc, dec in (("k", lay.centers_k, lay.w_enc_k, lay.w_dec_k),
                                 ("v", lay.centers_v, lay.w_enc_v, lay.w_dec_v)):
        rows = synth.history_rows(sh, cent, sh.N, seed=1 + (kind == "v"), device=dev)
        e = ops.encode(rows, enc, centers=cent, group=sh.G, scale_dtype=sh.scale_dtype)
        ref = orc.encode(rows.cpu().numpy(), u16(enc), u16(cent), None, sh.G, "fp16", "fp32")
        assert np.array_equal(e["ids"].cpu().numpy().astype(np.int64), ref["ids"]), kind
        # codes and scales bit-exact given the GPU's own fp32 coefficients
        rp, rs, _ = orc.quant_pack(e["coeff"].cpu().numpy(), sh.G, "fp16", "fp32")
        assert np.array_equal(e["packed"].cpu().numpy(), rp), kind
        assert np.array_equal(u16(e["scales"]), rs), kind
        # the coefficients themselves to fp32 accumulation-order rounding
        np.testing.assert_allclose(e["coeff"].cpu().numpy(), ref["coeff"], rtol=0, atol=2e-5)
        codec = ops.Codec(packed=e["packed"][None], scales=e["scales"][None], w_dec=dec,
                          group=sh.G, ids=e["ids"][None], centers=cent[None])
        got = ops.decode(codec, sh.HD)[0]
        want = orc.decode(**_oracle_codec(e, dec, cent, sh.G))
        diff = np.abs(orc.bf16_to_f32(u16(got)) - orc.bf16_to_f32(want)).max()
        assert diff <= 3 * 2 ** -7 * max(1.0, float(np.abs(orc.bf16_to_f32(want)).max())), kind


def test_cfg0_layer_on_the_gpu(dev):
    """Config 0's whole layer on the GPU at D = 64: the history (2,048 rows of
    K and V) encoded by nkv_encode, then one nkv_attend of 256 queries over it
    and 256 current keys, against the oracle's decode-then-SDPA on the same
    payload (the GPU's codes and scales)."""
    sh = synth.CONFIGS[0]
    assert (sh.H, sh.D, sh.N, sh.Q, sh.Nc) == (8, 64, 2048, 256, 256)
    lay = synth.make_layer(sh, seed=0, device=dev, orthonormal_codec=True)
    codecs, payload = [], []
    for kind, cent, enc, dec in (("k", lay.centers_k, lay.w_enc_k, lay.w_dec_k),
                                 ("v", lay.centers_v, lay.w_enc_v, lay.w_dec_v)):
        rows = synth.history_rows(sh, cent, sh.N, seed=1 + (kind == "v"), device=dev)
        e = ops.encode(rows, enc, centers=cent, group=sh.G, scale_dtype=sh.scale_dtype)
        codecs.append(ops.Codec(packed=e["packed"][None], scales=e["scales"][None], w_dec=dec,
                                group=sh.G, ids=e["ids"][None], centers=cent[None]))
        payload.append(_oracle_codec(e, dec, cent, sh.G))
    g = torch.Generator(device=dev).manual_seed(5)
    q = (torch.randn(1, sh.Q, sh.H, sh.D, generator=g, device=dev) / sh.D ** 0.5).to(torch.bfloat16)
    kc = synth.history_rows(sh, lay.centers_k, sh.Nc, seed=7, device=dev)
    vc = synth.history_rows(sh, lay.centers_v, sh.Nc, seed=8, device=dev)
    kc = kc.view(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    vc = vc.view(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    out, lse = ops.attend(q, kc, vc, codecs[0], codecs[1])
    ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), payload[0], payload[1],
                                     sh.D ** -0.5, D=sh.D)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3


def test_cfg2_assign_1024_centers_bit_exact(dev):
    sh = synth.CONFIGS[2]
    lay = synth.make_layer(sh, seed=2, device=dev)
    rows = synth.history_rows(sh, lay.centers_k, 4096, seed=9, device=dev)
    ids = ops.assign(rows, lay.centers_k)
    assert ids.dtype == torch.int16
    ref = orc.assign(rows.cpu().numpy(), u16(lay.centers_k))
    assert np.array_equal(ids.cpu().numpy().astype(np.int64) & 0xFFFF, ref)


def test_cfg2_full_call_subset_heads(dev):
    sh = synth.CONFIGS[2]
    assert (sh.N, sh.Q, sh.Nc, sh.C, sh.rK, sh.rV) == (49920, 780, 780, 1024, 384, 256)
    lay = synth.make_layer(sh, seed=0, device=dev)
    codecs, refs = [], []
    for kind, cent, enc, dec in (("k", lay.centers_k, lay.w_enc_k, lay.w_dec_k),
                                 ("v", lay.centers_v, lay.w_enc_v, lay.w_dec_v)):
        rows = synth.history_rows(sh, cent, sh.N, seed=1 + (kind == "v"), device=dev)
        e = ops.encode(rows, enc, centers=cent, group=sh.G, scale_dtype=sh.scale_dtype)
        del rows
        assert e["ids"].dtype == torch.int16
        codecs.append(ops.Codec(packed=e["packed"][None], scales=e["scales"][None], w_dec=dec,
                                group=sh.G, ids=e["ids"][None], centers=cent[None]))
        refs.append(_oracle_codec(e, dec, cent, sh.G))
    q = synth.queries(sh, seed=3, device=dev)
    kc = synth.history_rows(sh, lay.centers_k, sh.Nc, seed=4, device=dev)
    vc = synth.history_rows(sh, lay.centers_v, sh.Nc, seed=5, device=dev)
    kc = kc.reshape(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    vc = vc.reshape(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    out, lse = ops.attend(q, kc, vc, codecs[0], codecs[1])
    heads = [0, 11, 23]
    ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), refs[0], refs[1],
                                     sh.D ** -0.5, heads=heads, D=sh.D)
    diff, cos = max_abs_cos(out[0][:, heads].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0][heads].cpu().numpy() - ref_lse).max() < 2e-3


def test_cfg4_rollout_slice(dev):
    """Two layers of the config-4 step at its shapes (H = 24, D = 128, 16
    frames x 1,560 history rows, a 1,560-token chunk; the config-1 codec)."""
    sh = synth.CONFIGS[1]
    F, T, H, D, G = 16, 1560, sh.H, sh.D, sh.G
    N, HD = F * T, sh.HD
    heads = [3, 20]
    g = torch.Generator(device=dev).manual_seed(44)
    for li in range(2):
        lay = synth.make_layer(sh, seed=100 + li, device=dev)
        ring = []
        for kind, cent, enc, dec in (("k", lay.centers_k, lay.w_enc_k, lay.w_dec_k),
                                     ("v", lay.centers_v, lay.w_enc_v, lay.w_dec_v)):
            rows = synth.history_rows(sh, cent, N, seed=1000 + 2 * li + (kind == "v"), device=dev)
            e = ops.encode(rows, enc, centers=cent, group=G, scale_dtype=sh.scale_dtype)
            ring.append((e, enc, cent, dec))
        codecs = [ops.Codec(packed=e["packed"][None], scales=e["scales"][None], w_dec=dec,
                            group=G, ids=e["ids"][None], centers=cent[None])
                  for (e, enc, cent, dec) in ring]
        q = (torch.randn(1, T, H, D, generator=g, device=dev) / D ** 0.5).to(torch.bfloat16)
        k = synth.history_rows(sh, lay.centers_k, T, seed=500 + li, device=dev)
        v = synth.history_rows(sh, lay.centers_v, T, seed=600 + li, device=dev)
        kb = k.view(1, T, H, D).to(torch.bfloat16)
        vb = v.view(1, T, H, D).to(torch.bfloat16)

        def check():
            out, lse = ops.attend(q, kb, vb, codecs[0], codecs[1])
            refs = [_oracle_codec(e, dec, cent, G) for (e, enc, cent, dec) in ring]
            ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kb[0]), u16(vb[0]), refs[0], refs[1],
                                             D ** -0.5, heads=heads, D=D)
            diff, cos = max_abs_cos(out[0][:, heads].float().cpu().numpy(), ref)
            assert diff <= MAX_ABS and cos >= MIN_COS, (li, diff, cos)
            assert np.abs(lse[0][heads].cpu().numpy() - ref_lse).max() < 2e-3
        check()
        # the commit, as bench.py --config 4 runs it: the chunk's bf16 K and V,
        # strided views of one [T, 3 HD] projection output, encoded in one
        # batched call into frame slot 5 of the history
        slot = slice(5 * T, 6 * T)
        qkv = torch.empty(T, 3 * HD, device=dev, dtype=torch.bfloat16)
        qkv[:, HD:2 * HD] = kb.view(T, HD)
        qkv[:, 2 * HD:] = vb.view(T, HD)
        views = (qkv[:, HD:2 * HD], qkv[:, 2 * HD:])
        coeffs = [torch.empty(T, sh.rK, device=dev, dtype=torch.float32) for _ in range(2)]
        ops.encode_batch([{"x": x, "w_enc": enc, "centers": cent,
                           "out": {"packed": e["packed"][slot], "scales": e["scales"][slot],
                                   "ids": e["ids"][slot], "coeff": c}}
                          for (e, enc, cent, dec), x, c in zip(ring, views, coeffs)],
                         group=G, scale_dtype=sh.scale_dtype)
        for (e, enc, cent, dec), x, c in zip(ring, views, coeffs):
            ref = orc.encode(x.float().cpu().numpy(), u16(enc), u16(cent), None, G, "fp16", "fp32")
            assert np.array_equal(e["ids"][slot].cpu().numpy().astype(np.int64), ref["ids"])
            rp, rs, _ = orc.quant_pack(c.cpu().numpy(), G, "fp16", "fp32")
            assert np.array_equal(e["packed"][slot].cpu().numpy(), rp)
            assert np.array_equal(u16(e["scales"][slot]), rs)
        check()
