"""GPU parity of NanoKV-Fast's one-launch staged path: with no read-time
RoPE or camera and at most three reader groups,
nkv_fast_attend decodes every partition's tiles in one launch, attends all of
them in one flash launch and merges each head's native and low partitions in
one combine (the value-mean shift folded in), with identity readers reading
the layer's own queries, center tables and means through head maps.  Checked
against the oracle's hybrid_attention restatement: max-abs <= 2e-2, cosine
>= 0.9995, |dlse| < 2e-3."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, ops, synth
from tests._helpers import Scenario, max_abs_cos, oracle_codec, oracle_groups, u16
from tests.test_gpu_fast import MAX_ABS, MIN_COS, _payload, _run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,rV", [(32, 384), (64, 128)])
def test_fast_staged_mixed_groups(dev, d, rV):
    """An identity group and a group at width d in one launch (equal and
    different K/V ranks: one decode launch or two)."""
    sc = Scenario(H=4, N=1000, Q=1060, Nc=90, rK=384, rV=rV, G=32, C=16, with_mean=True,
                  seed=3 + d)
    _run(sc, dev, _payload(sc, (0, 3), d, seed=d), np.arange(780, 1000))


@pytest.mark.parametrize("prot", ["none", "scattered", "all"])
def test_fast_staged_partitions(dev, prot):
    """No protected rows (the native partition holds the current keys
    alone), scattered protected rows, and every row protected (no low
    partition: the native attention alone)."""
    sc = Scenario(H=2, N=700, Q=1030, Nc=40, rK=256, rV=256, G=32, C=8, with_mean=True, seed=4)
    N = sc.N
    rows = {"none": np.array([], np.int64),
            "scattered": np.concatenate([np.arange(0, 40), np.arange(300, 310), np.arange(650, N)]),
            "all": np.arange(N)}[prot]
    _run(sc, dev, _payload(sc, (1,), 32), rows)


@pytest.mark.parametrize("G,scale_dtype,id_dtype,centers,mean", [
    (384, torch.bfloat16, torch.int16, True, False),
    (32, torch.float16, torch.uint8, False, True),
])
def test_fast_staged_codec_variants(dev, G, scale_dtype, id_dtype, centers, mean):
    sc = Scenario(H=2, N=520, Q=1050, Nc=33, rK=384, rV=384, G=G, C=12, scale_dtype=scale_dtype,
                  id_dtype=id_dtype, centers=centers, with_mean=mean, seed=G)
    _run(sc, dev, _payload(sc, (1,), 32), np.arange(400, 520))


def test_fast_staged_batch_no_current(dev):
    """Two batch items, no current keys, two identity heads around a d=64 one."""
    sc = Scenario(B=2, H=3, N=450, Q=1024, Nc=0, rK=128, rV=128, G=32, C=10, seed=5)
    _run(sc, dev, _payload(sc, (0, 2), 64), np.arange(300, 450))


def test_fast_staged_identity_equals_full_attention(dev):
    """Identity readers over every head: the merged partitions are full
    attention (CN/core.py:258-262), so the one-launch combine of two
    partitions matches nkv_attend over all rows."""
    sc = Scenario(H=2, N=900, Q=1100, Nc=50, rK=256, rV=256, G=32, C=16, with_mean=True, seed=6)
    key, value = sc.codecs(dev)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    reader = codec_native.ReaderLayer(_payload(sc, (0, 1), 128), dev)
    pr = torch.arange(600, 900, dtype=torch.int32, device=dev)
    lr = torch.arange(0, 600, dtype=torch.int32, device=dev)
    of, lf = ops.fast_attend(q, kc, vc, key, value, pr, lr, [g.tensors() for g in reader.groups])
    oa, la = ops.attend(q, kc, vc, key, value)
    diff, cos = max_abs_cos(of.float().cpu().numpy(), oa.float().cpu().numpy())
    assert diff < 1.5e-2 and cos > 0.9999, (diff, cos)
    assert torch.allclose(lf, la, atol=2e-4)


def test_fast_staged_low_shift_and_no_lse(dev):
    """A low-partition shift per (batch item, head) folded into the combine
    (the value-mean correction's form), against the oracle's merge of the
    shifted low output; and the call without an LSE output gives the same
    output bits."""
    sc = Scenario(B=2, H=3, N=800, Q=1040, Nc=60, rK=256, rV=256, G=32, C=8, with_mean=True, seed=7)
    payload = _payload(sc, (1,), 32, seed=7)
    key, value = sc.codecs(dev)
    reader = codec_native.ReaderLayer(payload, dev)
    prot = np.arange(600, 800)
    low = np.arange(600)
    pr = torch.from_numpy(prot.astype(np.int32)).to(dev)
    lr = torch.from_numpy(low.astype(np.int32)).to(dev)
    shift = torch.randn(sc.B, sc.H, sc.D, generator=torch.Generator().manual_seed(8)) * 0.05
    args = (sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value, pr, lr,
            [g.tensors() for g in reader.groups])
    out, lse = ops.fast_attend(*args, low_shift=shift.to(dev))
    out2, none = ops.fast_attend(*args, low_shift=shift.to(dev), return_lse=False)
    torch.cuda.synchronize()
    assert none is None and torch.equal(out.view(torch.int16), out2.view(torch.int16))
    groups = oracle_groups(payload)
    for b in range(sc.B):
        ref, ref_lse = orc.fast_attend(u16(sc.q[b]), u16(sc.k_cur[b]), u16(sc.v_cur[b]),
                                       sc.hist[b]["k"], sc.hist[b]["v"], prot, low, groups,
                                       sc.scale, D=sc.D, low_shift=shift[b].double().numpy())
        diff, cos = max_abs_cos(out[b].float().cpu().numpy(), ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (b, diff, cos)
        assert np.abs(lse[b].cpu().numpy() - ref_lse).max() < 2e-3


def test_fast_staged_segments(dev, monkeypatch):
    """Segmented payload caches through the reference-shaped entry: the
    identity group reads each segment's own center table through the head
    map, the d=32 group the concatenated projected tables."""
    from nanokv_amd import nanokv_codec as nc
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    monkeypatch.setenv("NANOKV_QUANT_MODE", "fp32")
    H, D, layer = 2, 128, 12
    sh = synth.Shape("api", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=8)
    lay = synth.make_layer(sh, seed=layer)
    nc.register_operator("k", layer, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev))
    nc.register_operator("v", layer, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev))
    nc.register_centers("k", layer, lay.centers_k.to(dev))
    nc.register_centers("v", layer, lay.centers_v.to(dev))
    cache_k = cache_v = None
    for c in range(4):  # four frames of 150 tokens
        k = synth.history_rows(sh, lay.centers_k, 150, seed=70 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 150, seed=80 + c).to(dev)[None].to(torch.bfloat16)
        cache_k = nc.concat_values(cache_k, nc.encode_tensor("k", layer, k))
        cache_v = nc.concat_values(cache_v, nc.encode_tensor("v", layer, v))
    protect = torch.zeros(600, dtype=torch.bool, device=dev)
    protect[450:] = True
    payload = synth.make_readers(sh, lay, full_heads=(1,), d=32)
    reader = codec_native.ReaderLayer(payload, dev)
    g = torch.Generator().manual_seed(13)
    q = (torch.randn(1, H, 1040, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 30, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 30, D, generator=g).to(torch.bfloat16).to(dev)
    out, lse = codec_native.fast_history_attention(q, cache_k, cache_v, kc, vc, reader, protect,
                                                   return_lse=True)
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
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3


def _multi_payload(sc, spec, seed=0):
    """A reader payload with one group per (heads, d) of spec (d None: an
    identity group), each cut from synth.make_readers over those heads."""
    groups = []
    for i, (heads, d) in enumerate(spec):
        others = tuple(h for h in range(sc.H) if h not in heads)
        if d is None:
            pl = synth.make_readers(sc.shape, sc.layer, seed=seed + i, full_heads=tuple(heads), d=32)
            groups.append(pl["groups"][0])
        else:
            pl = synth.make_readers(sc.shape, sc.layer, seed=seed + i, full_heads=others, d=d)
            groups.append(pl["groups"][1])
    return {"groups": groups, "heads": sc.H, "native_dim": sc.D, "rank": sc.shape.rK}


@pytest.mark.parametrize("spec", [
    # three groups: the native partition and three readers fill one launch
    [([0], None), ([1, 2], 32), ([3], 64)],
    # four groups: more partitions than one launch holds, run group by group
    [([0], None), ([1, 2], 32), ([3], 64), ([4], 32)],
])
def test_fast_staged_group_counts(dev, spec):
    H = max(max(hs) for hs, _ in spec) + 1
    sc = Scenario(H=H, N=800, Q=300, Nc=40, rK=256, rV=256, G=32, C=16, with_mean=True,
                  seed=20 + len(spec))
    _run(sc, dev, _multi_payload(sc, spec, seed=len(spec)), np.arange(600, 800))
