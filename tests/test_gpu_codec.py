"""GPU parity of the codec kernels against the CPU oracle (bit-exact where the
contract is integer/byte work: INT4 codes, scales, center ids, unpacked
latents)."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import ops, synth
from tests._helpers import from_u16, scale_name, u16

pytestmark = pytest.mark.gpu


def _coeff(rows, r, seed, kind="normal"):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, r, generator=g)
    if kind == "mixed":
        x = x * torch.exp(2 * torch.randn(rows, 1, generator=g))
        x[::7] = 0.0                      # all-zero rows: scale = eps / 7
        x[1::11] *= 1e-30                 # fp16 scale underflow
        x[2::13] *= 1e6                   # fp16 scale overflow (inf)
    return x.float().contiguous()


@pytest.mark.parametrize("r,group", [(384, 32), (384, 384), (256, 64), (64, 32), (40, 8)])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("quant_mode", ["fp32", "bf16"])
def test_quant_pack_bit_exact(dev, r, group, scale_dtype, quant_mode):
    for seed, kind in ((1, "normal"), (2, "mixed")):
        x = _coeff(333, r, seed, kind)
        packed, scales = ops.quant_pack(x.to(dev), group, scale_dtype, quant_mode)
        rp, rs, _ = orc.quant_pack(x.numpy(), group, scale_name(scale_dtype), quant_mode)
        assert np.array_equal(packed.cpu().numpy(), rp), (seed, kind)
        assert np.array_equal(u16(scales), rs), (seed, kind)


def test_quant_pack_half_ties(dev):
    # x / s lands exactly on k + 0.5: s = 7/7 = 1 when the row amax is 7.
    vals = np.array([7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 6.5, -6.5, 3.5, 4.5, 5.5, -7.0, 0.0,
                     0.49999997, 1.0000001] + [0.0] * 16, np.float32)[None]
    x = torch.from_numpy(vals)
    packed, scales = ops.quant_pack(x.to(dev), 32, torch.bfloat16, "fp32")
    rp, rs, codes = orc.quant_pack(vals, 32, "bf16", "fp32")
    assert np.array_equal(packed.cpu().numpy(), rp)
    assert np.array_equal(u16(scales), rs)
    assert list(codes[0, :14]) == [7, 0, 2, 2, 0, -2, -2, 6, -6, 4, 4, 6, -7, 0]


def test_quant_pack_empty(dev):
    x = torch.zeros(0, 64, device=dev)
    packed, scales = ops.quant_pack(x, 32)
    assert packed.shape == (0, 32) and scales.shape == (0, 2)


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("r,group", [(384, 32), (384, 384), (256, 32)])
def test_unpack_bit_exact(dev, scale_dtype, r, group):
    g = torch.Generator().manual_seed(5)
    rows = 517
    packed = torch.randint(0, 256, (rows, r // 2), generator=g, dtype=torch.uint8)
    scales = (torch.rand(rows, r // group, generator=g) * 3).to(scale_dtype)
    out = ops.unpack(packed.to(dev), scales.to(dev), r, group)
    ref = orc.unpack_latent(packed.numpy(), u16(scales), r, group, scale_name(scale_dtype))
    assert np.array_equal(u16(out), ref)
    idx = torch.tensor([0, 5, 516, 5, 100], dtype=torch.int32)
    out = ops.unpack(packed.to(dev), scales.to(dev), r, group, row_index=idx.to(dev))
    ref = orc.unpack_latent(packed.numpy(), u16(scales), r, group, scale_name(scale_dtype),
                            row_index=idx.numpy())
    assert np.array_equal(u16(out), ref)


@pytest.mark.parametrize("C,id_dtype", [(16, torch.uint8), (256, torch.uint8),
                                         (300, torch.int16), (70, torch.int32)])
def test_assign_bit_exact(dev, C, id_dtype):
    shape = synth.Shape("t", H=4, D=128, N=0, Q=0, Nc=0, rK=64, rV=64, G=32, C=C)
    layer = synth.make_layer(shape, seed=3)
    x = synth.history_rows(shape, layer.centers_k, 777, seed=9)
    ids = ops.assign(x.to(dev), layer.centers_k.to(dev), id_dtype)
    ref = orc.assign(x.numpy(), u16(layer.centers_k))
    got = ids.cpu().to(torch.int64).numpy()
    if id_dtype == torch.int16:
        got = got & 0xFFFF
    assert np.array_equal(got, ref)


def test_assign_exact_ties(dev):
    # duplicated centers and rows exactly midway between two centers: the
    # first index must win (torch.argmin semantics, MG:320).
    HD = 64
    c = np.zeros((6, HD), np.float32)
    c[0, 0], c[1, 0], c[2, 0] = 1.0, 1.0, -1.0   # 0 and 1 duplicate
    c[3, 1], c[4, 1], c[5, 2] = 2.0, -2.0, 4.0
    centers = torch.from_numpy(c).to(torch.bfloat16)
    x = np.zeros((5, HD), np.float32)
    x[1, 0] = 0.5          # nearer 0/1 (tie -> 0)
    x[2, 1] = 0.0          # equidistant from 0,1,2 (all at distance 1) -> 0
    x[3, 1], x[3, 0] = 0.0, -0.5   # nearest 2
    x[4, 2] = 2.0          # equidistant from 5 (dist 4) and ... check oracle decides
    ids = ops.assign(torch.from_numpy(x).to(dev), centers.to(dev), torch.int32)
    ref = orc.assign(x, u16(centers))
    assert np.array_equal(ids.cpu().numpy(), ref)
    assert ref[1] == 0 and ref[2] == 0 and ref[3] == 2


@pytest.mark.parametrize("group,scale_dtype,quant_mode,with_mean",
                         [(32, torch.float16, "fp32", False), (384, torch.bfloat16, "fp32", True),
                          (32, torch.bfloat16, "bf16", True)])
def test_encode_parity(dev, group, scale_dtype, quant_mode, with_mean):
    shape = synth.Shape("t", H=4, D=128, N=0, Q=0, Nc=0, rK=384, rV=384, G=group, C=64)
    layer = synth.make_layer(shape, seed=4, with_mean=with_mean)
    x = synth.history_rows(shape, layer.centers_k, 300, seed=11)
    mean = layer.mean_k
    got = ops.encode(x.to(dev), layer.w_enc_k.to(dev), centers=layer.centers_k.to(dev),
                     mean=None if mean is None else mean.to(dev), group=group,
                     scale_dtype=scale_dtype, quant_mode=quant_mode)
    ref = orc.encode(x.numpy(), u16(layer.w_enc_k), u16(layer.centers_k),
                     None if mean is None else mean.numpy(), group, scale_name(scale_dtype),
                     quant_mode)
    # center ids: bit-exact
    assert np.array_equal(got["ids"].cpu().numpy().astype(np.int64), ref["ids"])
    # projection: fp32 GEMM vs fp64-accumulated oracle
    coeff = got["coeff"].cpu().numpy()
    np.testing.assert_allclose(coeff, ref["coeff"], rtol=2e-5, atol=2e-5)
    # codes and scales are bit-exact given the identical fp32 projected input
    rp, rs, _ = orc.quant_pack(coeff, group, scale_name(scale_dtype), quant_mode)
    assert np.array_equal(got["packed"].cpu().numpy(), rp)
    assert np.array_equal(u16(got["scales"]), rs)


@pytest.mark.parametrize("H,D", [(3, 32), (2, 64)])
def test_encode_parity_narrow_rows(dev, H, D):
    # row widths of 96 and 128 (not multiples of 256): the projection takes the
    # general GEMM kernel instead of the split-K one
    shape = synth.Shape("t", H=H, D=D, N=0, Q=0, Nc=0, rK=64, rV=64, G=32, C=20)
    layer = synth.make_layer(shape, seed=8)
    x = synth.history_rows(shape, layer.centers_k, 150, seed=12)
    got = ops.encode(x.to(dev), layer.w_enc_k.to(dev), centers=layer.centers_k.to(dev), group=32,
                     scale_dtype=torch.float16)
    ref = orc.encode(x.numpy(), u16(layer.w_enc_k), u16(layer.centers_k), None, 32, "fp16", "fp32")
    assert np.array_equal(got["ids"].cpu().numpy().astype(np.int64), ref["ids"])
    coeff = got["coeff"].cpu().numpy()
    np.testing.assert_allclose(coeff, ref["coeff"], rtol=2e-5, atol=2e-5)
    rp, rs, _ = orc.quant_pack(coeff, 32, "fp16", "fp32")
    assert np.array_equal(got["packed"].cpu().numpy(), rp)
    assert np.array_equal(u16(got["scales"]), rs)


@pytest.mark.parametrize("id_dtype", [torch.uint8, torch.int32])
def test_assign_near_ties_exact(dev, id_dtype):
    # HD = 256, C <= 256: the bf16 MFMA search.  Rows on the exact midpoint of
    # two centers tie (the first index must win); rows moved a hair off a
    # midpoint differ by far less than the search's error bound, so both
    # kinds go through the exact fp64 re-evaluation of their candidates.
    # small-integer centers: every product and sum below is exact in fp64, so
    # the ties are exact whatever the summation order
    g = torch.Generator().manual_seed(31)
    C, HD = 24, 256
    centers = torch.randint(-8, 9, (C, HD), generator=g).to(torch.bfloat16)
    cf = centers.float()
    a = torch.randint(0, C, (64,), generator=g)
    b = (a + 1 + torch.randint(0, C - 1, (64,), generator=g)) % C
    mid = 0.5 * (cf[a] + cf[b])                      # exact in fp32
    nudge = (cf[b] - cf[a]) * 2.0 ** -20              # toward b: b wins by a hair
    x = torch.cat([mid, mid + nudge, mid - nudge, cf[a] + torch.randint(-1, 2, (64, HD), generator=g)])
    ids = ops.assign(x.to(dev), centers.to(dev), id_dtype)
    got = ids.cpu().to(torch.int64).numpy()
    ref = orc.assign(x.numpy(), u16(centers))
    assert np.array_equal(got, ref)
    assert np.array_equal(ref[:64], np.minimum(a, b).numpy())


@pytest.mark.parametrize("C,HD,id_dtype", [(24, 256, torch.uint8), (256, 512, torch.uint8),
                                            (200, 768, torch.int32)])
def test_assign_bf16_rows_near_ties_exact(dev, C, HD, id_dtype):
    """The search over bf16 rows (nkv_encode with x_bf16, one MFMA pass):
    rows on the exact midpoint of two small-integer centers tie (the first
    index wins); rows moved one bf16 step of one coordinate off a midpoint
    differ by far less than the search's error bound, so both go through the
    exact fp64 re-evaluation; the ids equal oracle.assign on x.float()."""
    g = torch.Generator().manual_seed(32 + C)
    centers = torch.randint(-8, 9, (C, HD), generator=g).to(torch.bfloat16)
    cf = centers.float()
    n = 96
    a = torch.randint(0, C, (n,), generator=g)
    b = (a + 1 + torch.randint(0, C - 1, (n,), generator=g)) % C
    mid = 0.5 * (cf[a] + cf[b])                      # half-integers: exact in bf16
    j = (cf[b] - cf[a]).abs().argmax(1)              # a coordinate where a and b differ
    step = torch.zeros(n, HD)
    step[torch.arange(n), j] = torch.sign(cf[b] - cf[a])[torch.arange(n), j] * 2.0 ** -6
    x = torch.cat([mid, mid + step, mid - step,
                   cf[a] + torch.randint(-1, 2, (n, HD), generator=g)]).to(torch.bfloat16)
    assert torch.equal(x.float().to(torch.bfloat16), x)
    w_enc = (torch.randn(64, HD, generator=g) / HD ** 0.5).to(torch.bfloat16)
    got = ops.encode(x.to(dev), w_enc.to(dev), centers=centers.to(dev), group=32,
                     id_dtype=id_dtype)
    ids = got["ids"].cpu().to(torch.int64).numpy()
    ref = orc.assign(x.float().numpy(), u16(centers))
    assert np.array_equal(ids, ref)
    assert np.array_equal(ref[:n], np.minimum(a, b).numpy())
    assert np.array_equal(ref[n:2 * n], b.numpy()) and np.array_equal(ref[2 * n:3 * n], a.numpy())
    # the same rows as fp32 take the two-pass search: same ids
    got32 = ops.encode(x.float().to(dev), w_enc.to(dev), centers=centers.to(dev), group=32,
                       id_dtype=id_dtype)
    assert torch.equal(got32["ids"], got["ids"])


def test_assign_rows_not_multiple_of_16(dev):
    # HD = 72: the fp64 VALU search (the MFMA search needs HD % 16 == 0)
    g = torch.Generator().manual_seed(21)
    centers = torch.randn(40, 72, generator=g).to(torch.bfloat16)
    x = (centers.float()[torch.randint(0, 40, (90,), generator=g)]
         + 0.3 * torch.randn(90, 72, generator=g))
    ids = ops.assign(x.to(dev), centers.to(dev), torch.int32)
    assert np.array_equal(ids.cpu().numpy(), orc.assign(x.numpy(), u16(centers)))


def test_encode_into_cache_slot(dev):
    # ops.encode(out=...) writes a chunk straight into a slot of a larger cache
    shape = synth.Shape("t", H=4, D=128, N=0, Q=0, Nc=0, rK=384, rV=384, G=32, C=64)
    layer = synth.make_layer(shape, seed=5)
    x = synth.history_rows(shape, layer.centers_k, 200, seed=6).to(dev)
    kw = dict(centers=layer.centers_k.to(dev), group=32, scale_dtype=torch.float16)
    ref = ops.encode(x, layer.w_enc_k.to(dev), **kw)
    cache = {"packed": torch.zeros(600, 192, dtype=torch.uint8, device=dev),
             "scales": torch.zeros(600, 12, dtype=torch.float16, device=dev),
             "ids": torch.zeros(600, dtype=torch.uint8, device=dev)}
    sl = slice(200, 400)
    got = ops.encode(x, layer.w_enc_k.to(dev), **kw,
                     out={"packed": cache["packed"][sl], "scales": cache["scales"][sl],
                          "ids": cache["ids"][sl],
                          "coeff": torch.empty(200, 384, device=dev)})
    assert got["packed"].data_ptr() == cache["packed"][sl].data_ptr()
    for k in ("packed", "scales", "ids"):
        assert torch.equal(cache[k][sl], ref[k])
        assert not cache[k][:200].bool().any() and not cache[k][400:].bool().any()
    with pytest.raises(ValueError):
        ops.encode(x, layer.w_enc_k.to(dev), **kw, out={"packed": cache["packed"][:100]})


@pytest.mark.parametrize("with_mean", [False, True])
def test_encode_batch_equals_single_encodes(dev, with_mean):
    """nkv_encode_batch: three problems of one shape with their own rows
    (ragged counts), operators, centers and means give, each, the bits of
    nkv_encode on that problem; a bf16 input, also as a strided view, gives
    the bits of the fp32 encode of its values (value.float() is exact)."""
    shape = synth.Shape("t", H=4, D=128, N=0, Q=0, Nc=0, rK=384, rV=384, G=32, C=64)
    probs, singles = [], []
    for i, n in enumerate((300, 77, 129)):
        layer = synth.make_layer(shape, seed=20 + i, with_mean=with_mean)
        x = synth.history_rows(shape, layer.centers_k, n, seed=30 + i).to(dev)
        kw = dict(w_enc=layer.w_enc_k.to(dev), centers=layer.centers_k.to(dev),
                  mean=None if layer.mean_k is None else layer.mean_k.to(dev))
        probs.append(dict(x=x, **kw))
        singles.append(ops.encode(x, **kw, group=32, scale_dtype=torch.float16))
    got = ops.encode_batch(probs, group=32, scale_dtype=torch.float16)
    for g, r in zip(got, singles):
        for k in ("packed", "scales", "ids", "coeff"):
            assert torch.equal(g[k], r[k]), k
    # bf16 rows: contiguous, and strided views of one [rows, 3 HD] buffer
    xb = [p["x"].to(torch.bfloat16) for p in probs]
    wide = [torch.zeros(b.shape[0], 3 * b.shape[1], dtype=torch.bfloat16, device=dev) for b in xb]
    for w, b in zip(wide, xb):
        w[:, 512:1024] = b
    for inputs in (xb, [w[:, 512:1024] for w in wide]):
        got = ops.encode_batch([dict(p, x=b) for p, b in zip(probs, inputs)], group=32,
                               scale_dtype=torch.float16)
        for g, p, b in zip(got, probs, xb):
            r = ops.encode(b.float(), **{k: v for k, v in p.items() if k != "x"}, group=32,
                           scale_dtype=torch.float16)
            for k in ("packed", "scales", "ids", "coeff"):
                assert torch.equal(g[k], r[k]), k


def test_encode_batch_rejects_mixed_problems(dev):
    shape = synth.Shape("t", H=4, D=128, N=0, Q=0, Nc=0, rK=384, rV=384, G=32, C=64)
    layer = synth.make_layer(shape, seed=3)
    x = synth.history_rows(shape, layer.centers_k, 40, seed=4).to(dev)
    p = dict(x=x, w_enc=layer.w_enc_k.to(dev), centers=layer.centers_k.to(dev))
    with pytest.raises(Exception, match="share"):
        ops.encode_batch([p, dict(p, centers=None)], group=32)
    with pytest.raises(Exception, match="share"):
        ops.encode_batch([p, dict(p, x=x.to(torch.bfloat16))], group=32)


@pytest.mark.parametrize("with_mean,id_dtype", [(False, torch.uint8), (True, torch.int16)])
def test_decode_parity(dev, with_mean, id_dtype):
    from tests._helpers import Scenario
    sc = Scenario(B=2, H=2, N=150, Q=1, Nc=0, rK=384, rV=256, G=32, C=20, with_mean=with_mean,
                  id_dtype=id_dtype)
    key, value = sc.codecs(dev)
    for codec, kind in ((key, "k"), (value, "v")):
        out = ops.decode(codec, sc.H * sc.D)
        for b in range(sc.B):
            ref = orc.bf16_to_f32(orc.decode(**sc.hist[b][kind]))
            got = out[b].float().cpu().numpy()
            # fp32 accumulation order differs from the oracle; each of the two bf16
            # roundings (GEMM+bias, +center) may land one ulp apart.  The first ulp is
            # relative to the pre-center value (O(1) here), hence the absolute term.
            np.testing.assert_allclose(got, ref, rtol=2 ** -7, atol=2 ** -7)
        idx = torch.tensor([3, 0, 149, 77], dtype=torch.int32, device=dev)
        sel = ops.decode(codec, sc.H * sc.D, row_index=idx)
        np.testing.assert_array_equal(u16(sel), u16(out[:, idx.long().cpu()]))
