"""GPU parity of NanoKV-Fast (nkv_fast_attend) against the oracle's
restatement of hybrid_attention (oracle.fast_attend): max-abs <= 2e-2 and
cosine >= 0.9995 in bf16, for reader widths 32 / 64 / 128, contiguous and
scattered protected rows, with and without centers / mean, and the full
config-3 shape on a subset of heads."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, ops, synth
from tests._helpers import Scenario, max_abs_cos, oracle_codec, oracle_groups, u16

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9995


def _run(sc, dev, payload, prot, heads=None):
    key, value = sc.codecs(dev)
    reader = codec_native.ReaderLayer(payload, dev)
    N = sc.N
    low = np.setdiff1d(np.arange(N), prot)
    pr = torch.from_numpy(prot.astype(np.int32)).to(dev)
    lr = torch.from_numpy(low.astype(np.int32)).to(dev)
    kc = None if sc.k_cur is None else sc.k_cur.to(dev)
    vc = None if sc.v_cur is None else sc.v_cur.to(dev)
    out, lse = ops.fast_attend(sc.q.to(dev), kc, vc, key, value, pr, lr,
                               [g.tensors() for g in reader.groups])
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    groups = oracle_groups(payload)
    for b in range(sc.B):
        kcb = None if sc.k_cur is None else u16(sc.k_cur[b])
        vcb = None if sc.v_cur is None else u16(sc.v_cur[b])
        ref, ref_lse = orc.fast_attend(u16(sc.q[b]), kcb, vcb, sc.hist[b]["k"], sc.hist[b]["v"],
                                       prot, low, groups, sc.scale, heads=heads, D=sc.D)
        hs = list(range(sc.H)) if heads is None else heads
        diff, cos = max_abs_cos(out[b][:, hs], ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (b, diff, cos)
        assert np.abs(lse[b][hs] - ref_lse).max() < 2e-3
    return out, lse


def _payload(sc, full_heads, d, seed=0):
    return synth.make_readers(sc.shape, sc.layer, seed=seed, full_heads=full_heads, d=d)


@pytest.mark.parametrize("d", [32, 64, 128])
def test_fast_reader_widths(dev, d):
    sc = Scenario(H=4, N=700, Q=150, Nc=64, rK=384, rV=256, G=32, C=16)
    _run(sc, dev, _payload(sc, (1,), d), np.arange(500, 700))


@pytest.mark.parametrize("d", [32, 64])
def test_fast_reader_widths_staged(dev, d):
    """Without read-time RoPE or camera the reader groups run the staged schedule at
    their width (K image [128][d], flash at K/Q width d): a ragged history,
    means and centers, fp16 group scales."""
    sc = Scenario(H=4, N=900, Q=1040, Nc=70, rK=384, rV=256, G=32, C=16, with_mean=True,
                  seed=d)
    _run(sc, dev, _payload(sc, (2,), d, seed=d), np.arange(700, 900))


@pytest.mark.parametrize("prot", ["recent", "scattered", "none", "all"])
def test_fast_partitions(dev, prot):
    sc = Scenario(H=2, N=600, Q=100, Nc=40, rK=256, rV=256, G=32, C=8, with_mean=True)
    N = sc.N
    rows = {"recent": np.arange(400, N),
            "scattered": np.concatenate([np.arange(0, 30), np.arange(250, 260), np.arange(590, N)]),
            "none": np.array([], np.int64), "all": np.arange(N)}[prot]
    _run(sc, dev, _payload(sc, (0,), 32), rows)


@pytest.mark.parametrize("G,scale_dtype,centers", [(384, torch.bfloat16, True),
                                                   (32, torch.float16, False)])
def test_fast_codec_variants(dev, G, scale_dtype, centers):
    sc = Scenario(H=2, N=420, Q=70, Nc=33, rK=384, rV=384, G=G, C=12, scale_dtype=scale_dtype,
                  centers=centers)
    _run(sc, dev, _payload(sc, (1,), 32), np.arange(300, 420))


def test_fast_batch_and_no_current(dev):
    sc = Scenario(B=2, H=3, N=300, Q=90, Nc=0, rK=128, rV=128, G=32, C=10)
    _run(sc, dev, _payload(sc, (0, 2), 64), np.arange(200, 300))


def test_fast_identity_readers_equal_full_attention(dev):
    # identity readers: the hybrid result is full attention (CN/core.py:258-262)
    sc = Scenario(H=2, N=512, Q=130, Nc=50, rK=256, rV=256, G=32, C=16)
    key, value = sc.codecs(dev)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    reader = codec_native.ReaderLayer(_payload(sc, (0, 1), 128), dev)
    pr = torch.arange(300, 512, dtype=torch.int32, device=dev)
    lr = torch.arange(0, 300, dtype=torch.int32, device=dev)
    of, lf = ops.fast_attend(q, kc, vc, key, value, pr, lr, [g.tensors() for g in reader.groups])
    oa, la = ops.attend(q, kc, vc, key, value)
    diff, cos = max_abs_cos(of.float().cpu().numpy(), oa.float().cpu().numpy())
    assert diff < 1.5e-2 and cos > 0.9999, (diff, cos)
    assert torch.allclose(lf, la, atol=2e-4)


def test_fast_history_attention_api(dev, monkeypatch):
    # the reference-shaped entry: payload caches, a frame protection mask and a ReaderLayer
    from nanokv_amd import nanokv_codec as nc
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    H, D, layer = 2, 128, 7
    sh = synth.Shape("api", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=layer)
    nc.register_operator("k", layer, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev))
    nc.register_operator("v", layer, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev))
    nc.register_centers("k", layer, lay.centers_k.to(dev))
    nc.register_centers("v", layer, lay.centers_v.to(dev))
    cache_k = cache_v = None
    for c in range(4):  # four frames of 50 tokens
        k = synth.history_rows(sh, lay.centers_k, 50, seed=30 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 50, seed=40 + c).to(dev)[None].to(torch.bfloat16)
        cache_k = nc.concat_values(cache_k, nc.encode_tensor("k", layer, k))
        cache_v = nc.concat_values(cache_v, nc.encode_tensor("v", layer, v))
    frames = torch.arange(200, device=dev) // 50
    protect = codec_native.protected_tokens(frames, recent=1, stride=2)
    # frame 3 (recent) plus frames 2 and 0 (every 2nd run back from the newest old one)
    assert protect.view(4, 50).all(1).tolist() == [True, False, True, True]
    payload = synth.make_readers(sh, lay, full_heads=(1,), d=32)
    reader = codec_native.ReaderLayer(payload, dev)
    g = torch.Generator().manual_seed(11)
    q = (torch.randn(1, H, 40, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 20, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 20, D, generator=g).to(torch.bfloat16).to(dev)
    out, lse = codec_native.fast_history_attention(q, cache_k, cache_v, kc, vc, reader, protect,
                                                   return_lse=True)
    assert out.shape == (1, H, 40, D) and lse.shape == (1, H, 40)
    # oracle over the same payload bits
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    assert key.segments is not None and len(key.segments.segments) == 4

    def od(cd):
        return oracle_codec(cd, 0, "bf16" if cd.scale_dtype == torch.bfloat16 else "fp16")
    prot = torch.nonzero(protect).flatten().cpu().numpy()
    low = torch.nonzero(~protect).flatten().cpu().numpy()
    ref, ref_lse = orc.fast_attend(u16(q[0].permute(1, 0, 2)), u16(kc[0].permute(1, 0, 2)),
                                   u16(vc[0].permute(1, 0, 2)), od(key), od(value), prot, low,
                                   oracle_groups(payload), D ** -0.5, D=D)
    diff, cos = max_abs_cos(out[0].permute(1, 0, 2).float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)


def test_fast_cfg3_shape_subset_heads(dev):
    """Config-3 call (H=24, D=128, N=12480, Q=Nc=1560, 6 identity heads, 18
    heads at d=32, last 2 frames protected), encoded on the GPU; the oracle
    checks one identity head and two reader heads."""
    sh = synth.CONFIGS[3]
    layer = synth.make_layer(sh, seed=0, device=dev)
    codecs = []
    for kind, cent, enc, dec in (("k", layer.centers_k, layer.w_enc_k, layer.w_dec_k),
                                 ("v", layer.centers_v, layer.w_enc_v, layer.w_dec_v)):
        rows = synth.history_rows(sh, cent, sh.N, seed=1 + (kind == "v"), device=dev)
        e = ops.encode(rows, enc, centers=cent, group=sh.G, scale_dtype=sh.scale_dtype)
        codecs.append(ops.Codec(packed=e["packed"][None], scales=e["scales"][None], w_dec=dec,
                                group=sh.G, ids=e["ids"][None], centers=cent[None]))
    q = synth.queries(sh, seed=3, device=dev)
    kc = synth.history_rows(sh, layer.centers_k, sh.Nc, seed=4, device=dev)
    vc = synth.history_rows(sh, layer.centers_v, sh.Nc, seed=5, device=dev)
    kc = kc.reshape(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    vc = vc.reshape(1, sh.Nc, sh.H, sh.D).to(torch.bfloat16)
    payload = synth.make_readers(sh, layer)
    reader = codec_native.ReaderLayer(payload, dev)
    protect = synth.fast_protect_mask(sh, device=dev)
    pr = torch.nonzero(protect).flatten().to(torch.int32)
    lr = torch.nonzero(~protect).flatten().to(torch.int32)
    out, lse = ops.fast_attend(q, kc, vc, codecs[0], codecs[1], pr, lr,
                               [g.tensors() for g in reader.groups])
    heads = [0, 5, 23]
    key = {"packed": codecs[0].packed[0].cpu().numpy(), "scales": u16(codecs[0].scales[0]),
           "w_dec_bf16": u16(layer.w_dec_k), "group": sh.G, "scale_dtype": "fp16",
           "ids": codecs[0].ids[0].cpu().numpy().astype(np.int64),
           "centers_bf16": u16(layer.centers_k)}
    val = {"packed": codecs[1].packed[0].cpu().numpy(), "scales": u16(codecs[1].scales[0]),
           "w_dec_bf16": u16(layer.w_dec_v), "group": sh.G, "scale_dtype": "fp16",
           "ids": codecs[1].ids[0].cpu().numpy().astype(np.int64),
           "centers_bf16": u16(layer.centers_v)}
    ref, ref_lse = orc.fast_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), key, val,
                                   pr.cpu().numpy(), lr.cpu().numpy(), oracle_groups(payload),
                                   sh.D ** -0.5, heads=heads, D=sh.D)
    diff, cos = max_abs_cos(out[0][:, heads].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0][heads].cpu().numpy() - ref_lse).max() < 2e-3


@pytest.mark.parametrize("d", [32, 64])
def test_fast_rope_matches_oracle(dev, d):
    """RoPE through every partition (CN/mg35.py:207-214, 305-336): protected
    keys rotated at their rows, reader queries from q_pre rotated on the
    group's retained pairs, reader keys likewise; readers keep a random set
    of complete original pairs."""
    sc = Scenario(H=4, N=700, Q=150, Nc=64, rK=384, rV=256, G=32, C=16, with_mean=True, seed=d)
    payload = _payload(sc, (1,), d)
    rng = np.random.default_rng(d)
    for g in payload["groups"]:
        n, dd = g["indices"].shape
        if dd == sc.D:
            continue
        pairs = np.stack([np.sort(rng.choice(sc.D // 2, dd // 2, replace=False)) for _ in range(n)])
        g["indices"] = torch.from_numpy(np.stack([2 * pairs, 2 * pairs + 1], 2).reshape(n, dd))
    reader = codec_native.ReaderLayer(payload, dev)
    key, value = sc.codecs(dev)
    bands = ops.rope_bands(sc.D, 64)
    rope = ops.Rope.from_bands(bands, [3, 8], 10, 35, dev)          # 2 frames of 350 rows
    q_rope = ops.Rope.from_bands(bands, [12], 10, 15, dev)          # the 150 queries
    q_pre = sc.q.to(dev)
    q = ops.rope_apply(q_pre, q_rope)
    prot = np.arange(500, 700)
    low = np.setdiff1d(np.arange(sc.N), prot)
    pr = torch.from_numpy(prot.astype(np.int32)).to(dev)
    lr = torch.from_numpy(low.astype(np.int32)).to(dev)
    out, lse = ops.fast_attend(q, sc.k_cur.to(dev), sc.v_cur.to(dev), key, value, pr, lr,
                               [g.tensors(rope=True) for g in reader.groups], rope=rope,
                               q_pre=q_pre, q_rope=q_rope)
    torch.cuda.synchronize()
    t = torch.view_as_complex(rope.cs_t.cpu()).numpy()
    h = torch.view_as_complex(rope.cs_h.cpu()).numpy()
    w = torch.view_as_complex(rope.cs_w.cpu()).numpy()
    key_freqs = orc.kv_freqs((t, h, w), rope.frame_pos.cpu().numpy(), 10, 35)
    q_freqs = orc.kv_freqs(tuple(torch.view_as_complex(b.cpu()).numpy()
                                 for b in (q_rope.cs_t, q_rope.cs_h, q_rope.cs_w)),
                           q_rope.frame_pos.cpu().numpy(), 10, 15)
    groups = oracle_groups(payload)
    for g, pg in zip(groups, payload["groups"]):
        ind = pg["indices"].numpy()
        g["rope_pairs"] = ind[:, ::2] // 2
    ref, ref_lse = orc.fast_attend(u16(q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), sc.hist[0]["k"],
                                   sc.hist[0]["v"], prot, low, groups, sc.scale, D=sc.D,
                                   key_freqs=key_freqs, q_pre_bf16=u16(sc.q[0]), q_freqs=q_freqs)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3


def test_fast_rope_requires_pairs_and_query_positions(dev):
    sc = Scenario(H=2, N=200, Q=40, Nc=0, rK=128, rV=128, G=32, C=8)
    payload = _payload(sc, (0,), 32)
    payload["groups"][1]["indices"] = torch.arange(32).flip(0).expand(1, 32).clone()  # not pairs
    reader = codec_native.ReaderLayer(payload, dev)
    with pytest.raises(ValueError, match="complete original pairs"):
        reader.groups[1].tensors(rope=True)
    key, value = sc.codecs(dev)
    rope = ops.Rope.from_bands(ops.rope_bands(128, 16), [0, 1], 10, 10, dev)
    pr = torch.arange(100, 200, dtype=torch.int32, device=dev)
    lr = torch.arange(0, 100, dtype=torch.int32, device=dev)
    from nanokv_amd import _lib
    with pytest.raises(_lib.NanoKVError, match="q_pre and q_rope"):
        ops.fast_attend(sc.q.to(dev), None, None, key, value, pr, lr,
                        [reader.groups[0].tensors(rope=True)], rope=rope)


@pytest.mark.parametrize("vd", [64, 128])
def test_fast_value_lift(dev, vd):
    """A reader group with a learned value lift [vd, D] (CN/core.py:202-204):
    the oracle lifts each low partition's bf16 output before the merge, as the
    reference does; the kernels read V through the folded matrices."""
    sc = Scenario(H=4, N=600, Q=120, Nc=40, rK=256, rV=256, G=32, C=12, with_mean=True, seed=vd)
    payload = _payload(sc, (0,), 32)
    g = torch.Generator().manual_seed(vd)
    low = payload["groups"][1]
    n, D = len(low["heads"]), sc.D

    def bf(t):
        return t.to(torch.bfloat16).float()

    low["v_read"] = bf(torch.randn(n, vd, sc.shape.rV, generator=g) / sc.shape.rV ** 0.5)
    low["v_affine"] = bf(torch.randn(n, D, vd, generator=g) / D ** 0.5)
    low["lift"] = bf(torch.randn(n, vd, D, generator=g) / vd ** 0.5)
    low["v_indices"] = torch.arange(vd).expand(n, vd).clone()
    _run(sc, dev, payload, np.arange(400, 600))


def test_fast_value_mean_correction(dev, monkeypatch):
    """LingBot's value-mean correction (codec_native_attention.py:465-501,
    779-785) in the fused path: for a group with a low-rank value lift
    (vd = 64 < 128), every low value is shifted by mean - projected, where
    mean is the first moment of the low rows' full decode and projected the
    mean of their lifted reader value reads.  Both are formed here in fp64
    from the oracle's latents and reads, independently of the library's
    closed form, and the result is checked against the oracle's Fast with
    that shift."""
    from nanokv_amd import nanokv_codec as nc
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    H, D, layer, vd = 3, 128, 9, 64
    sh = synth.Shape("vmc", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=layer, with_mean=True)
    nc.register_operator("k", layer, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev),
                         mean=lay.mean_k.to(dev))
    nc.register_operator("v", layer, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev),
                         mean=lay.mean_v.to(dev))
    nc.register_centers("k", layer, None)  # per-segment C64 tables
    nc.register_centers("v", layer, None)
    monkeypatch.setenv("MG35_KVCODEC_C64_CLUSTERS", "8")
    cache_k = cache_v = None
    for c in range(3):
        k = synth.history_rows(sh, lay.centers_k, 64, seed=50 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 64, seed=60 + c).to(dev)[None].to(torch.bfloat16)
        cache_k = nc.concat_values(cache_k, nc.encode_tensor("k", layer, k))
        cache_v = nc.concat_values(cache_v, nc.encode_tensor("v", layer, v))
    protect = torch.zeros(192, dtype=torch.bool, device=dev)
    protect[128:] = True
    payload = synth.make_readers(sh, lay, full_heads=(0,), d=32)
    low_g = payload["groups"][1]
    n = len(low_g["heads"])
    gen = torch.Generator().manual_seed(5)

    def bf(t):
        return t.to(torch.bfloat16).float()
    low_g["v_read"] = bf(torch.randn(n, vd, sh.rV, generator=gen) / sh.rV ** 0.5)
    low_g["v_affine"] = bf(torch.randn(n, D, vd, generator=gen) / D ** 0.5)
    low_g["lift"] = bf(torch.randn(n, vd, D, generator=gen) / vd ** 0.5)
    low_g["v_indices"] = torch.arange(vd).expand(n, vd).clone()
    reader = codec_native.ReaderLayer(payload, dev)
    q = (torch.randn(1, H, 30, D, generator=gen) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 16, D, generator=gen).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 16, D, generator=gen).to(torch.bfloat16).to(dev)
    out = codec_native.fast_history_attention(q, cache_k, cache_v, kc, vc, reader, protect,
                                              value_mean_correction=True)
    plain = codec_native.fast_history_attention(q, cache_k, cache_v, kc, vc, reader, protect)
    # the shift, in fp64 from the oracle's pieces
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    sname = "bf16" if value.scale_dtype == torch.bfloat16 else "fp16"
    ov, ok = oracle_codec(value, 0, sname), oracle_codec(key, 0, sname)
    low = np.arange(128)
    lat = orc.bf16_to_f32(orc.unpack_latent(ov["packed"], ov["scales"], sh.rV, ov["group"],
                                            sname, row_index=low)).astype(np.float64)
    w = orc.bf16_to_f32(ov["w_dec_bf16"]).astype(np.float64)            # [HD, r]
    cen = orc.bf16_to_f32(ov["centers_bf16"]).astype(np.float64)[np.asarray(ov["ids"])[low]]
    mean_bf = orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(ov["mean"], np.float32)))
    full_mean = (lat @ w.T).mean(0) + mean_bf + cen.mean(0)              # [HD]
    groups = oracle_groups(payload)
    shift = np.zeros((H, D))
    g1 = groups[1]
    for i, h in enumerate(g1["heads"]):
        vt, vb = orc.reader_tables(ov.get("centers_bf16"), ov.get("mean"), h, g1["v_affine"][i], D)
        vl = orc.bf16_to_f32(orc.reader_read(ov, low, g1["v_read"][i], vt, vb)).astype(np.float64)
        projected = vl.mean(0) @ orc.bf16_to_f32(g1["lift"][i]).astype(np.float64)
        shift[h] = full_mean[h * D:(h + 1) * D] - projected
    got_shift = codec_native.value_mean_shift(reader, cache_k, cache_v, ~protect, dev)
    assert np.abs(got_shift[0].cpu().numpy() - shift).max() < 2e-2 * max(1.0, np.abs(shift).max())
    assert np.abs(shift).max() > 1e-2  # the correction is not trivial here
    ref, _ = orc.fast_attend(u16(q[0].permute(1, 0, 2)), u16(kc[0].permute(1, 0, 2)),
                             u16(vc[0].permute(1, 0, 2)), ok, ov, np.arange(128, 192), low,
                             groups, D ** -0.5, D=D, low_shift=shift)
    diff, cos = max_abs_cos(out[0].permute(1, 0, 2).float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    # heads of the identity group (full width) are not corrected
    assert torch.equal(out[:, 0].view(torch.int16), plain[:, 0].view(torch.int16))


def test_fast_back_to_back_calls_and_graph_replay(dev):
    """Back-to-back multi-partition calls with different queries on a user
    stream, and a captured graph of the call replayed with new queries (eager
    calls between the replays), give the outputs of calls made one at a time
    with a synchronisation after each."""
    sc = Scenario(H=4, N=700, Q=300, Nc=64, rK=384, rV=256, G=32, C=16, with_mean=True, seed=5)
    key, value = sc.codecs(dev)
    reader = codec_native.ReaderLayer(_payload(sc, (1,), 32, seed=5), dev)
    groups = [g.tensors() for g in reader.groups]
    prot = torch.arange(500, 700, dtype=torch.int32, device=dev)
    low = torch.arange(0, 500, dtype=torch.int32, device=dev)
    kc, vc = sc.k_cur.to(dev), sc.v_cur.to(dev)
    g = torch.Generator().manual_seed(9)
    qs = [(torch.randn(sc.q.shape, generator=g) / 8).to(torch.bfloat16).to(dev) for _ in range(4)]

    def call(q):
        return ops.fast_attend(q, kc, vc, key, value, prot, low, groups)[0]

    ref = []
    for q in qs:
        ref.append(call(q).clone())
        torch.cuda.synchronize()
    user = torch.cuda.Stream()
    with torch.cuda.stream(user):
        outs = [call(q) for q in qs]
    torch.cuda.synchronize()
    for o, r in zip(outs, ref):
        assert torch.equal(o, r)
    # a graph of one call, replayed with each query copied into its input
    q_in = qs[0].clone()
    call(q_in)                      # warm-up: plans and side stream exist
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = call(q_in)
    for i in (1, 2, 3, 0):
        q_in.copy_(qs[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref[i]), i
        # eager work between replays
        assert torch.equal(call(qs[i]), ref[i])
        torch.cuda.synchronize()
