"""GPU parity of the fused decode+attention kernel against the oracle's
decode-then-SDPA path: max-abs <= 2e-2 and cosine >= 0.9995 in bf16."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import ops
from tests._helpers import Scenario, max_abs_cos, u16

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COS = 0.9995


def _check(sc, dev, splits=0, heads=None, schedule="auto"):
    key, value = sc.codecs(dev)
    kc = None if sc.k_cur is None else sc.k_cur.to(dev)
    vc = None if sc.v_cur is None else sc.v_cur.to(dev)
    out, lse = ops.attend(sc.q.to(dev), kc, vc, key, value, splits=splits, schedule=schedule)
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    for b in range(sc.B):
        ref, ref_lse = sc.reference(b, heads=heads)
        hs = list(range(sc.H)) if heads is None else heads
        diff, cos = max_abs_cos(out[b][:, hs], ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (b, diff, cos)
        fin = np.isfinite(ref_lse)
        assert np.array_equal(fin, np.isfinite(lse[b][hs]))
        if fin.any():
            assert np.abs(lse[b][hs][fin] - ref_lse[fin]).max() < 2e-3
    return out, lse


SCHEDULES = ["query_tiles", "key_chunks"]


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("D,B,with_mean", [(64, 1, False), (64, 2, True), (32, 1, True)])
def test_attend_narrow_heads(dev, D, B, with_mean, schedule):
    """Heads narrower than 128 (BASELINE config 0 has D = 64) run through the
    D = 128 kernels on zero-padded operands: the same bar against the
    oracle's decode-then-SDPA at width D, on both schedules, with a mean,
    two batch items and a strided query / output."""
    sc = Scenario(B=B, H=3, D=D, N=300, Q=70, Nc=40, rK=64, rV=128, G=32, C=8,
                  with_mean=with_mean, seed=D + B)
    _check(sc, dev, schedule=schedule)
    # q and out as column slices of wider buffers (16-byte aligned rows)
    key, value = sc.codecs(dev)
    wide_q = torch.zeros(B, sc.Q, sc.H, 2 * D, dtype=torch.bfloat16, device=dev)
    wide_q[..., D:] = sc.q.to(dev)
    wide_o = torch.full((B, sc.Q, sc.H, 2 * D), 7.0, dtype=torch.bfloat16, device=dev)
    out, _ = ops.attend(wide_q[..., D:], sc.k_cur.to(dev), sc.v_cur.to(dev), key, value,
                        out=wide_o[..., :D], schedule=schedule)
    ref, _ = ops.attend(sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value,
                        schedule=schedule)
    assert torch.equal(wide_o[..., :D], ref)
    assert bool((wide_o[..., D:] == 7.0).all())


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("N,Nc,Q", [(200, 64, 100), (257, 37, 300), (64, 0, 1), (0, 100, 33),
                                    (1000, 130, 513)])
def test_attend_shapes(dev, N, Nc, Q, schedule):
    _check(Scenario(H=2, N=N, Q=Q, Nc=Nc, rK=384, rV=256, G=32, C=16), dev, schedule=schedule)


# key-chunk edges: exact/partial chunks (256 keys), partial 32-key steps,
# query tiles of 64 with a 1..32-query remainder (single query block)
@pytest.mark.parametrize("N,Nc,Q", [(256, 0, 64), (512, 256, 128), (255, 1, 65), (1, 31, 96),
                                    (300, 513, 200), (767, 0, 31), (0, 257, 97)])
def test_attend_key_chunk_edges(dev, N, Nc, Q):
    _check(Scenario(H=2, N=N, Q=Q, Nc=Nc, rK=256, rV=384, G=32, C=16), dev, schedule="key_chunks")


# many query blocks with long current-key runs (the staged schedule at
# these sizes): partial current chunks and tiles, a partial last query block
@pytest.mark.parametrize("N,Nc,Q", [(300, 600, 1100), (0, 300, 1530), (256, 1, 1024)])
def test_attend_current_chunk_query_shares(dev, N, Nc, Q):
    _check(Scenario(H=2, N=N, Q=Q, Nc=Nc, rK=128, rV=128, G=32, C=8), dev, schedule="key_chunks")


@pytest.mark.parametrize("splits", [1, 2, 5, 0])
def test_attend_splits(dev, splits):
    _check(Scenario(H=2, N=700, Q=260, Nc=100, rK=128, rV=64, G=32, C=8), dev, splits=splits)


@pytest.mark.parametrize("G,scale_dtype,with_mean,id_dtype,centers", [
    (384, torch.bfloat16, False, torch.uint8, True),
    (32, torch.float16, True, torch.int16, True),
    (64, torch.bfloat16, True, torch.int32, True),
    (32, torch.float16, False, torch.uint8, False),
])
@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attend_codec_variants(dev, G, scale_dtype, with_mean, id_dtype, centers, schedule):
    _check(Scenario(H=2, N=300, Q=70, Nc=40, rK=384, rV=384, G=G, C=40, scale_dtype=scale_dtype,
                    with_mean=with_mean, id_dtype=id_dtype, centers=centers), dev,
           schedule=schedule)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attend_batch(dev, schedule):
    _check(Scenario(B=2, H=3, N=150, Q=90, Nc=20, rK=256, rV=256, G=32, C=12), dev,
           schedule=schedule)


def test_attend_schedules_agree(dev):
    # the two decompositions compute the same attention; key chunks is AUTO's
    # choice whenever the codecs fit it
    sc = Scenario(H=2, N=900, Q=400, Nc=120, rK=384, rV=384, G=32, C=16)
    key, value = sc.codecs(dev)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    oa, la = ops.attend(q, kc, vc, key, value, schedule="query_tiles")
    ob, lb = ops.attend(q, kc, vc, key, value, schedule="key_chunks")
    oc, lc = ops.attend(q, kc, vc, key, value)
    diff, cos = max_abs_cos(oa.float().cpu().numpy(), ob.float().cpu().numpy())
    assert diff < 1e-2 and cos > 0.9999, (diff, cos)
    assert torch.allclose(la, lb, atol=1e-4)
    assert torch.equal(oc, ob) and torch.equal(lc, lb)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attend_empty_keys(dev, schedule):
    q = torch.randn(1, 5, 2, 128, device=dev).to(torch.bfloat16)
    out, lse = ops.attend(q, None, None, schedule=schedule)
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def test_lse_merge(dev):
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4, 50, 128, generator=g).to(torch.bfloat16)
    b = torch.randn(4, 50, 128, generator=g).to(torch.bfloat16)
    la = torch.randn(4, 50, generator=g) * 3
    lb = torch.randn(4, 50, generator=g) * 3
    la[0, :5] = -float("inf")
    lb[0, 3:8] = -float("inf")
    out, lse = ops.lse_merge(a.to(dev), la.to(dev), b.to(dev), lb.to(dev))
    ref, ref_lse = orc.merge(a.float().numpy(), la.numpy(), b.float().numpy(), lb.numpy())
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=1e-6, atol=1e-6)


def test_attend_merge_equals_joint(dev):
    # attending history and current separately and merging by LSE equals one joint call
    sc = Scenario(H=2, N=300, Q=64, Nc=80, rK=128, rV=128, G=32, C=8)
    key, value = sc.codecs(dev)
    q = sc.q.to(dev)
    kc, vc = sc.k_cur.to(dev), sc.v_cur.to(dev)
    o1, l1 = ops.attend(q, None, None, key, value)
    o2, l2 = ops.attend(q, kc, vc)
    oj, lj = ops.attend(q, kc, vc, key, value)
    om, lm = ops.lse_merge(o1.permute(0, 2, 1, 3).contiguous(), l1,
                           o2.permute(0, 2, 1, 3).contiguous(), l2)
    diff, cos = max_abs_cos(om.float().cpu().numpy(),
                            oj.permute(0, 2, 1, 3).float().cpu().numpy())
    assert diff < 1e-2 and cos > 0.9999
    assert torch.allclose(lm, lj, atol=1e-4)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_attend_cfg1_shape_subset_heads(dev, schedule):
    """Full config-1 call (H=24, D=128, N=12480, Q=Nc=1560, r=384, G=32 fp16,
    C=256), encoded on the GPU; the oracle checks heads 0, 11 and 23."""
    from nanokv_amd import synth
    sh = synth.CONFIGS[1]
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
    out, lse = ops.attend(q, kc, vc, codecs[0], codecs[1], schedule=schedule)
    heads = [0, 11, 23]
    key = {"packed": codecs[0].packed[0].cpu().numpy(), "scales": u16(codecs[0].scales[0]),
           "w_dec_bf16": u16(layer.w_dec_k), "group": sh.G, "scale_dtype": "fp16",
           "ids": codecs[0].ids[0].cpu().numpy().astype(np.int64),
           "centers_bf16": u16(layer.centers_k)}
    val = {"packed": codecs[1].packed[0].cpu().numpy(), "scales": u16(codecs[1].scales[0]),
           "w_dec_bf16": u16(layer.w_dec_v), "group": sh.G, "scale_dtype": "fp16",
           "ids": codecs[1].ids[0].cpu().numpy().astype(np.int64),
           "centers_bf16": u16(layer.centers_v)}
    ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), key, val, sh.D ** -0.5,
                                     heads=heads)
    diff, cos = max_abs_cos(out[0][:, heads].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0][heads].cpu().numpy() - ref_lse).max() < 2e-3
