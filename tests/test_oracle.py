"""Pins the CPU oracle (oracle/) with checks that do not restate its code:
hand-computed known answers, independent library routines (torch, numpy),
brute force and exact rational arithmetic, and invariants."""
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle.oracle as orc

RNG = np.random.default_rng(1234)


# ------------------------------------------------------------ conversions
def test_conversions_bf16_exhaustive_against_torch():
    # every bf16 pattern widened, then random floats and ties narrowed, vs torch
    bits = np.arange(65536, dtype=np.uint16)
    wide = orc.bf16_to_f32(bits)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(wide.view(np.uint32), ref.view(np.uint32))
    x = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** RNG.integers(-40, 39, 200000),
        wide[np.isfinite(wide)],
        (wide[np.isfinite(wide)].view(np.uint32) + np.uint32(0x8000)).view(np.float32),  # exact ties
        np.array([np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-45, 3.4e38], np.float32),
    ]).astype(np.float32)
    x = x[np.isfinite(x) | np.isinf(x)]
    got = orc.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_conversions_f16_against_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    h = bits.view(np.float16)
    wide = orc.f16_to_f32(bits)
    ok = ~np.isnan(h)
    assert np.array_equal(wide[ok].view(np.uint32), h[ok].astype(np.float32).view(np.uint32))
    x = np.concatenate([
        RNG.standard_normal(200000).astype(np.float32) * np.float32(2.0) ** RNG.integers(-30, 20, 200000),
        h[np.isfinite(h)].astype(np.float32),
        # midpoints between consecutive fp16 values (ties to even)
        ((h[np.isfinite(h)][:-1].astype(np.float64) + h[np.isfinite(h)][1:].astype(np.float64)) / 2
         ).astype(np.float32),
        np.array([65504.0, 65519.99, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26,
                  3 * 2.0 ** -26, 0.0, -0.0], np.float32),
    ]).astype(np.float32)
    got = orc.f32_to_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------ quantiser
def _codes_brute(x: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Nearest code among -7..7 to x/s by exhaustive search; ties go to the
    even code (round-half-even then clamp)."""
    q = (x.astype(np.float32) / s.astype(np.float32)).astype(np.float64)
    ks = np.arange(-7, 8)
    d = np.abs(q[..., None] - ks)
    best = d.min(-1, keepdims=True)
    cand = np.where(np.isclose(d, best, rtol=0, atol=0), ks, 99)
    even = np.where(cand % 2 == 0, cand, 99).min(-1)
    first = cand.min(-1)
    ntie = (cand != 99).sum(-1)
    return np.where(ntie > 1, even, first).astype(np.int8)


@pytest.mark.parametrize("r,group", [(64, 32), (64, 64), (384, 32), (40, 8)])
def test_quant_brute_force(r, group):
    x = (RNG.standard_normal((257, r)) * np.exp(RNG.standard_normal((257, 1)))).astype(np.float32)
    packed, scales, codes = orc.quant_pack(x, group, "bf16", "fp32")
    g = x.reshape(257, r // group, group)
    s = np.maximum(np.abs(g).max(-1, keepdims=True), np.float32(np.finfo(np.float32).eps)) / np.float32(7)
    assert np.array_equal(codes.reshape(g.shape), _codes_brute(g, s.astype(np.float32)))
    # stored scales are torch's bf16 of s
    ref = torch.from_numpy(s[..., 0].astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(scales.reshape(257, -1), ref.view(np.uint16))
    # |x - code * s| <= s/2 wherever the code is not clamped
    err = np.abs(g - codes.reshape(g.shape) * s)
    assert np.all(err <= s / 2 * (1 + 1e-6) + 1e-30)


def test_quant_known_answers():
    # row amax 7 -> s = 1: x/s lands on half ties, which round to even
    x = np.zeros((1, 32), np.float32)
    x[0, :13] = [7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 6.5, -6.5, 3.5, 4.5, 5.5, -7.0]
    packed, scales, codes = orc.quant_pack(x, 32, "bf16", "fp32")
    assert list(codes[0, :13]) == [7, 0, 2, 2, 0, -2, -2, 6, -6, 4, 4, 6, -7]
    assert scales[0, 0] == 0x3F80  # bf16(1.0)
    # packing: byte j = (c[2j] + 7) | (c[2j+1] + 7) << 4
    assert packed[0, 0] == (7 + 7) | ((0 + 7) << 4)
    assert packed[0, 1] == (2 + 7) | ((2 + 7) << 4)
    assert packed[0, 6] == (-7 + 7) | ((0 + 7) << 4)


def test_quant_zero_row_and_fp16_range():
    eps = np.float32(np.finfo(np.float32).eps)
    x = np.zeros((4, 32), np.float32)
    x[1, 0] = 1e6      # s = 1e6/7 overflows fp16 -> inf
    x[2, 0] = 1e-30    # below the FLT_EPSILON clamp: s = eps/7, code 0
    x[3, 0] = 1e-6     # s = 1.43e-7: an fp16 subnormal (2 * 2^-24 after rounding)
    _, scales, codes = orc.quant_pack(x, 32, "fp16", "fp32")
    assert scales[0, 0] == np.float16(eps / np.float32(7)).view(np.uint16) == 0
    assert np.all(codes[0] == 0)
    assert scales[1, 0] == 0x7C00 and codes[1, 0] == 7
    assert scales[2, 0] == 0x0000 and codes[2, 0] == 0
    assert scales[3, 0] == 0x0002 and codes[3, 0] == 7


def test_quant_bf16_mode_matches_torch_bf16_ops():
    """MG:349-351 executed with torch bf16 tensors (torch's own rounding)."""
    x = (RNG.standard_normal((64, 384)) * 3).astype(np.float32)
    _, scales, codes = orc.quant_pack(x, 384, "bf16", "bf16")
    coeff = torch.from_numpy(x).to(torch.bfloat16)
    scale = coeff.abs().amax(-1, keepdim=True).clamp_min(torch.finfo(torch.float32).eps) / 7.0
    ref_codes = (coeff / scale).round().clamp(-7, 7).to(torch.int8).numpy()
    assert np.array_equal(codes, ref_codes)
    assert np.array_equal(scales, scale.view(torch.int16).numpy().view(np.uint16))


def test_pack_unpack_roundtrip_all_pairs():
    a, b = np.meshgrid(np.arange(-7, 8), np.arange(-7, 8))
    codes = np.stack([a.ravel(), b.ravel()], 1).astype(np.int8)
    packed = orc.pack_codes(codes)
    assert packed.size == codes.size // 2
    assert np.array_equal(orc.unpack_codes(packed, codes.size), codes.reshape(-1))
    # MG:285-286 rejects nibbles outside [0, 16): codes 9 and -8
    with pytest.raises(RuntimeError):
        orc.pack_codes(np.array([9, 0], np.int8))
    with pytest.raises(RuntimeError):
        orc.pack_codes(np.array([0, -8], np.int8))


def test_quant_pack_agrees_with_pack_codes():
    x = RNG.standard_normal((33, 64)).astype(np.float32)
    packed, _, codes = orc.quant_pack(x, 32, "fp16", "fp32")
    assert np.array_equal(packed.reshape(-1), orc.pack_codes(codes))


@pytest.mark.parametrize("scale_dtype", ["bf16", "fp16"])
def test_unpack_latent_against_torch(scale_dtype):
    packed = RNG.integers(0, 256, (50, 96), dtype=np.uint8)
    dt = torch.float16 if scale_dtype == "fp16" else torch.bfloat16
    s = torch.rand(50, 6) * 4
    sbits = s.to(dt).view(torch.int16).numpy().view(np.uint16)
    got = orc.unpack_latent(packed, sbits, 192, 32, scale_dtype)
    codes = torch.from_numpy(orc.unpack_codes(packed, 50 * 192).astype(np.int64)).reshape(50, 192)
    ref = (codes.float() * s.to(dt).float().repeat_interleave(32, 1)).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    idx = np.array([3, 0, 49], np.int32)
    got_sel = orc.unpack_latent(packed, sbits, 192, 32, scale_dtype, row_index=idx)
    assert np.array_equal(got_sel, got[idx])


# ------------------------------------------------------------ assignment
def test_assign_exact_rational_brute_force():
    for seed in range(5):
        rng = np.random.default_rng(seed)
        x = (rng.standard_normal((9, 24)) * 2).astype(np.float32)
        c = torch.from_numpy(rng.standard_normal((7, 24)).astype(np.float32)).to(torch.bfloat16)
        cbits = c.view(torch.int16).numpy().view(np.uint16)
        cf = orc.bf16_to_f32(cbits)
        got = orc.assign(x, cbits)
        for n in range(9):
            d = [sum((Fraction(float(x[n, k])) - Fraction(float(cf[j, k]))) ** 2 for k in range(24))
                 for j in range(7)]
            assert got[n] == int(np.argmin([float(v - min(d)) for v in d]))
            assert d[got[n]] == min(d) and d.index(min(d)) == got[n]


def test_assign_ties_pick_lowest_index():
    c = np.zeros((4, 8), np.float32)
    c[0, 0] = c[1, 0] = 1.0   # duplicates
    c[2, 0] = -1.0
    c[3, 1] = 3.0
    cbits = orc.f32_to_bf16(c)
    x = np.zeros((3, 8), np.float32)
    x[1, 0] = 0.25          # nearest 0 and 1 (tie -> 0)
    # x[0] = 0 is equidistant from 0, 1, 2 -> 0 ; x[2] near center 3
    x[2, 1] = 2.0
    assert list(orc.assign(x, cbits)) == [0, 0, 3]


def test_residual_against_torch():
    x = RNG.standard_normal((20, 64)).astype(np.float32)
    c = torch.from_numpy(RNG.standard_normal((5, 64)).astype(np.float32)).to(torch.bfloat16)
    ids = RNG.integers(0, 5, 20).astype(np.int32)
    mean = RNG.standard_normal(64).astype(np.float32)
    got = orc.residual_bf16(x, c.view(torch.int16).numpy().view(np.uint16), ids, mean)
    ref = ((torch.from_numpy(x) - c.float()[torch.from_numpy(ids).long()]) - torch.from_numpy(mean)
           ).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


# ------------------------------------------------------------ decode
def test_decode_epilogue_against_torch_bf16_ops():
    """rows = bf16(acc + bf16(mean)); rows.add_(fp32 center) in a bf16 tensor
    (MG:438-454), evaluated with torch's own bf16 arithmetic."""
    acc = (RNG.standard_normal((40, 64)) * 3).astype(np.float32)
    mean = RNG.standard_normal(64).astype(np.float32)
    c = torch.from_numpy(RNG.standard_normal((6, 64)).astype(np.float32)).to(torch.bfloat16)
    ids = RNG.integers(0, 6, 40).astype(np.int32)
    out = np.empty((40, 64), np.uint16)
    orc.lib().nkvo_decode_epilogue(acc.ctypes.data, mean.ctypes.data,
                                   c.view(torch.int16).numpy().ctypes.data, ids.ctypes.data,
                                   40, 64, out.ctypes.data)
    rows = (torch.from_numpy(acc) + torch.from_numpy(mean).to(torch.bfloat16).float()).to(torch.bfloat16)
    rows.add_(c.float()[torch.from_numpy(ids).long()])
    assert np.array_equal(out, rows.view(torch.int16).numpy().view(np.uint16))


def test_decode_matches_torch_linear_reference():
    """decode() vs the reference formula run with torch fp64 GEMM + bf16 ops."""
    r, hd, n = 64, 128, 30
    w = torch.randn(hd, r, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    enc = torch.randn(r, hd, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    c = torch.randn(4, hd, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    x = (torch.randn(n, hd, generator=torch.Generator().manual_seed(6)) * 2).numpy()
    u = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    e = orc.encode(x, u(enc), u(c), None, 32, "bf16", "fp32")
    got = orc.bf16_to_f32(orc.decode(e["packed"], e["scales"], u(w), 32, "bf16", e["ids"], u(c)))
    codes = torch.from_numpy(e["codes"].astype(np.float64))
    s = torch.from_numpy(orc.bf16_to_f32(e["scales"]).astype(np.float64)).repeat_interleave(32, 1)
    latent = (codes * s).to(torch.bfloat16).double()
    acc = (latent @ w.double().T).float()
    ref = acc.to(torch.bfloat16)
    ref = (ref.float() + c.float()[torch.from_numpy(e["ids"]).long()]).to(torch.bfloat16)
    assert np.array_equal(got, ref.float().numpy())


# ------------------------------------------------------------ attention / merge
def test_attention_against_torch_sdpa():
    q = RNG.standard_normal((3, 17, 16))
    k = RNG.standard_normal((3, 29, 16))
    v = RNG.standard_normal((3, 29, 16))
    out, lse = orc.attention(q, k, v, 0.3)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), scale=0.3)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-12, atol=1e-12)
    ref_lse = torch.logsumexp(torch.from_numpy(q) @ torch.from_numpy(k).transpose(1, 2) * 0.3, -1)
    np.testing.assert_allclose(lse, ref_lse.numpy(), rtol=1e-12, atol=1e-12)
    out0, lse0 = orc.attention(q, k[:, :0], v[:, :0], 0.3)
    assert np.all(out0 == 0) and np.all(np.isneginf(lse0))


def test_merge_of_partitions_equals_joint_attention():
    q = RNG.standard_normal((2, 11, 8))
    k = RNG.standard_normal((2, 40, 8))
    v = RNG.standard_normal((2, 40, 8))
    oa, la = orc.attention(q, k[:, :13], v[:, :13], 0.5)
    ob, lb = orc.attention(q, k[:, 13:], v[:, 13:], 0.5)
    om, lm = orc.merge(oa, la, ob, lb)
    oj, lj = orc.attention(q, k, v, 0.5)
    np.testing.assert_allclose(om, oj, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lm, lj, rtol=1e-12, atol=1e-12)
    # empty partitions: (0, -inf) is the identity; two empties stay (0, -inf)
    e_o, e_l = np.zeros_like(oa), np.full(la.shape, -np.inf)
    o1, l1 = orc.merge(oa, la, e_o, e_l)
    np.testing.assert_allclose(o1, oa, rtol=1e-15)
    o2, l2 = orc.merge(e_o, e_l, e_o, e_l)
    assert np.all(o2 == 0) and np.all(np.isneginf(l2))


# ------------------------------------------------------------ partition policy
def _protected_sets(count, recent, stride, sink):
    """Set-based statement of metadata_cache.route (CN/metadata_cache.py:64-68)."""
    old = max(0, count - recent)
    sel = set(range(old, count)) | set(range(min(sink, count)))
    if stride and old:
        sel |= set(range(old - 1, -1, -stride))
    return [i in sel for i in range(count)]


def test_protected_frames_known_answers():
    assert list(orc.protected_frames(8, 2, 0, 0)) == [False] * 6 + [True] * 2
    assert list(orc.protected_frames(8, 2, 3, 1)) == [True, False, True, False, False, True, True, True]
    assert list(orc.protected_frames(3, 5, 2, 0)) == [True] * 3
    assert list(orc.protected_frames(0, 2, 1, 1)) == []


def test_protected_frames_exhaustive_small():
    for count in range(0, 12):
        for recent in range(0, 5):
            for stride in range(0, 5):
                for sink in range(0, 3):
                    assert list(orc.protected_frames(count, recent, stride, sink)) == \
                        _protected_sets(count, recent, stride, sink)


def test_masked_attention_against_torch_sdpa():
    """oracle.attention with a boolean mask: rows that see a key equal torch's
    SDPA with the same attn_mask in fp64 (a library routine); rows that see
    none give (0, -inf) (the reference's blockwise path); an all-True mask is
    no mask."""
    g = torch.Generator().manual_seed(3)
    H, Q, N, D = 2, 9, 13, 16
    q = torch.randn(H, Q, D, generator=g, dtype=torch.float64)
    k = torch.randn(H, N, D, generator=g, dtype=torch.float64)
    v = torch.randn(H, N, D, generator=g, dtype=torch.float64)
    mask = torch.rand(Q, N, generator=g) > 0.5
    mask[3] = False
    mask[5] = True
    out, lse = orc.attention(q.numpy(), k.numpy(), v.numpy(), 0.25, mask=mask.numpy())
    seen = mask.any(1)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q[:, seen], k, v, attn_mask=mask[seen][None], scale=0.25)
    np.testing.assert_allclose(out[:, seen.numpy()], ref.numpy(), rtol=1e-12, atol=1e-12)
    s = (q @ k.transpose(1, 2)) * 0.25
    ref_lse = torch.logsumexp(s.masked_fill(~mask[None], -np.inf), -1)
    np.testing.assert_allclose(lse[:, seen.numpy()], ref_lse[:, seen].numpy(), rtol=1e-12)
    assert np.all(out[:, 3] == 0) and np.all(np.isneginf(lse[:, 3]))
    full, full_lse = orc.attention(q.numpy(), k.numpy(), v.numpy(), 0.25, mask=np.ones((Q, N), bool))
    plain, plain_lse = orc.attention(q.numpy(), k.numpy(), v.numpy(), 0.25)
    np.testing.assert_array_equal(full, plain)
    np.testing.assert_array_equal(full_lse, plain_lse)


def test_decode_attend_row_list_equals_selected_codec():
    """decode_attend(hist_rows) equals decode_attend over a codec holding only
    those rows (its packed codes, scales and ids sliced by the same rows)."""
    from tests._helpers import Scenario, u16
    sc = Scenario(H=2, D=32, N=70, Q=10, Nc=6, rK=64, rV=64, G=32, C=5)
    rows = np.array([3, 4, 9, 20, 21, 22, 50, 69])
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]

    def sliced(c):
        c = dict(c)
        c["packed"], c["scales"], c["ids"] = c["packed"][rows], c["scales"][rows], c["ids"][rows]
        return c
    a, la = orc.decode_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val,
                              sc.scale, D=sc.D, hist_rows=rows)
    b, lb = orc.decode_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), sliced(key),
                              sliced(val), sc.scale, D=sc.D)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(la, lb)
