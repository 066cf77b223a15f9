"""Pins of the oracle's RoPE restatement (oracle.rope_bands, kv_freqs,
rope_rotate, rope_apply) by checks that do not restate its formula:

* each band entry against exp(1j * n * theta^(-2i/dim)) evaluated one element
  at a time with Python's math module, and against torch.polar of the same
  angles (the library routine the reference's tables come from);
* the band widths for several head dims (t gets D - 2*(D//3) dims);
* the token layout of kv_freqs against a hand-built token;
* the rotation's invariants in fp64: pair norms are kept, rotations compose
  by adding angles, and q(m) . k(n) depends only on n - m (a swapped pair
  order, a wrong sign or a wrong band would break one of these);
* the bf16 result against torch's view_as_complex product, the reference's
  own formulation of rope_apply.
"""
import cmath
import math

import numpy as np
import pytest
import torch

import oracle.oracle as orc


@pytest.mark.parametrize("D,widths", [(128, (22, 21, 21)), (64, (11, 10, 10)),
                                      (96, (16, 16, 16)), (12, (2, 2, 2))])
def test_band_widths(D, widths):
    t, h, w = orc.rope_bands(D, 8)
    assert (t.shape[1], h.shape[1], w.shape[1]) == widths
    assert t.shape[0] == h.shape[0] == w.shape[0] == 8


def test_bands_closed_form():
    theta = 10000.0
    t, h, w = orc.rope_bands(128, 64, theta)
    for band, dim in ((t, 44), (h, 42), (w, 42)):
        for n in (0, 1, 7, 63):
            for i in (0, 1, band.shape[1] // 2, band.shape[1] - 1):
                expect = cmath.exp(1j * n * theta ** (-(2 * i) / dim))
                assert abs(band[n, i] - expect) <= 4e-16 * max(1, n)
        assert np.all(band[0] == 1.0)


def test_bands_match_torch_polar():
    t, h, w = orc.rope_bands(128, 200)
    for band, dim in ((t, 44), (h, 42), (w, 42)):
        inv = 1.0 / (10000.0 ** (torch.arange(0, dim, 2)[: dim // 2].double() / dim))
        ang = torch.outer(torch.arange(200), inv)
        ref = torch.polar(torch.ones_like(ang), ang).numpy()
        # same angles; cos/sin of two libraries agree to an ulp or two
        assert np.max(np.abs(band - ref)) < 1e-15


def test_kv_freqs_layout():
    bands = orc.rope_bands(128, 16)
    pos, gh, gw = [3, 0, 9], 4, 5
    f = orc.kv_freqs(bands, pos, gh, gw)
    assert f.shape == (3 * gh * gw, 64)
    for frame, p in enumerate(pos):
        for r in range(gh):
            for c in range(gw):
                n = frame * gh * gw + r * gw + c
                hand = np.concatenate([bands[0][p], bands[1][r], bands[2][c]])
                assert np.array_equal(f[n], hand)


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_rotation_keeps_pair_norms():
    bands = orc.rope_bands(128, 32)
    f = orc.kv_freqs(bands, [0, 5, 31], 3, 4)
    x = _rand((f.shape[0], 2, 128), 1)
    y = orc.rope_rotate(x, f)
    nx = np.hypot(x[..., 0::2], x[..., 1::2])
    ny = np.hypot(y[..., 0::2], y[..., 1::2])
    np.testing.assert_allclose(ny, nx, rtol=1e-14, atol=0)
    # position (frame 0 at t = 0, row 0, column 0) is the identity
    assert np.array_equal(y[0], x[0])


def test_rotations_compose():
    bands = orc.rope_bands(128, 64)
    x = _rand((12, 1, 128), 2)
    fa = orc.kv_freqs(bands, [3], 3, 4)
    fb = orc.kv_freqs(bands, [11], 3, 4)
    # the t band adds positions (3 + 11); the h / w bands add the token's own angle twice
    two = orc.kv_freqs(bands, [14], 3, 4)
    twice_hw = np.concatenate([two[:, :22], fa[:, 22:] * fb[:, 22:]], axis=1)
    y = orc.rope_rotate(orc.rope_rotate(x, fa), fb)
    np.testing.assert_allclose(y, orc.rope_rotate(x, twice_hw), rtol=0, atol=1e-13)


def test_score_depends_on_offset_only():
    bands = orc.rope_bands(128, 128)
    q = _rand((1, 1, 128), 3)
    k = _rand((1, 1, 128), 4)
    scores = {}
    for m, n in ((5, 9), (50, 54), (100, 104), (0, 4), (7, 2), (77, 72)):
        fq = orc.kv_freqs(bands, [m], 1, 1)
        fk = orc.kv_freqs(bands, [n], 1, 1)
        scores[(m, n)] = float(np.sum(orc.rope_rotate(q, fq) * orc.rope_rotate(k, fk)))
    same = [scores[(5, 9)], scores[(50, 54)], scores[(100, 104)], scores[(0, 4)]]
    np.testing.assert_allclose(same, same[0], rtol=1e-12)
    np.testing.assert_allclose(scores[(77, 72)], scores[(7, 2)], rtol=1e-12)
    assert abs(scores[(5, 9)] - scores[(7, 2)]) > 1e-6  # the offset's sign matters


def test_rope_apply_matches_torch_complex_product():
    bands = orc.rope_bands(128, 40)
    f = orc.kv_freqs(bands, [39, 1, 17, 0], 5, 6)
    S, H = f.shape[0], 3
    x = torch.randn(S, H, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    got = orc.rope_apply(bits, f)
    # the reference's formulation (wan_video_dit.py:185-192)
    xc = torch.view_as_complex(x.double().reshape(S, H, -1, 2))
    ref = torch.view_as_real(xc * torch.from_numpy(f)[:, None, :]).flatten(2).to(torch.bfloat16)
    ref_bits = ref.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref_bits)


def test_decode_attend_with_rope_rotates_history_keys():
    """key_freqs changes the scores exactly as rotating the decoded keys does:
    attending with identity frequencies (all positions 0) equals no RoPE."""
    from tests._helpers import Scenario, u16
    sc = Scenario(H=2, N=40, Q=6, Nc=0, rK=64, rV=64, G=32, C=4)
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    q = u16(sc.q[0])
    ones = np.ones((sc.N, 64), np.complex128)
    a, la = orc.decode_attend(q, None, None, key, val, 128 ** -0.5)
    b, lb = orc.decode_attend(q, None, None, key, val, 128 ** -0.5, key_freqs=ones)
    assert np.array_equal(a, b) and np.array_equal(la, lb)
    f = orc.kv_freqs(orc.rope_bands(128, 8), [1, 6], 4, 5)
    c, lc = orc.decode_attend(q, None, None, key, val, 128 ** -0.5, key_freqs=f)
    assert np.abs(c - a).max() > 1e-3
    assert math.isfinite(float(lc.max()))


# ---------------------------------------------------------------- NanoKV-Fast
def _fast_rope_problem(D=32, N=90, Q=12, Nc=10):
    from tests._helpers import Scenario, u16
    sc = Scenario(H=2, D=D, N=N, Q=Q, Nc=Nc, rK=64, rV=64, G=32, C=6, with_mean=True)
    bands = orc.rope_bands(D, 16)
    key_freqs = orc.kv_freqs(bands, [2, 9, 4], 5, 6)[:N]           # 3 frames of 30 rows
    q_freqs = orc.kv_freqs(bands, [11], 3, 4)[:Q]                   # the current frame
    q_pre = u16(sc.q[0])
    q = orc.rope_apply(q_pre, q_freqs)                              # the hook's rotated query
    return sc, bands, key_freqs, q_freqs, q_pre, q


@pytest.mark.parametrize("split", ["recent", "anchors", "none", "all"])
def test_fast_rope_identity_readers_equal_full_decode(split):
    """Identity readers (CN/core.py:258-262) reduce NanoKV-Fast with RoPE to the
    full decode -> rope_apply -> attention of every history row, whatever the
    split: the low partition's q_low is rope(q_pre) = q and its keys are the
    rotated full decode."""
    from nanokv_amd import synth
    from tests._helpers import max_abs_cos, oracle_groups, u16
    sc, _, key_freqs, q_freqs, q_pre, q = _fast_rope_problem()
    N = sc.N
    prot = {"recent": np.arange(60, N), "anchors": np.array([0, 1, 2, 30, 31, 50, 88, 89]),
            "none": np.array([], np.int64), "all": np.arange(N)}[split]
    low = np.setdiff1d(np.arange(N), prot)
    payload = synth.make_readers(sc.shape, sc.layer, full_heads=tuple(range(sc.H)))
    groups = oracle_groups(payload)
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    out, lse = orc.fast_attend(q, u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val, prot, low,
                               groups, sc.scale, D=sc.D, key_freqs=key_freqs, q_pre_bf16=q_pre,
                               q_freqs=q_freqs)
    ref, ref_lse = orc.decode_attend(q, u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val, sc.scale,
                                     D=sc.D, key_freqs=key_freqs)
    diff, cos = max_abs_cos(out, ref)
    assert diff < 2e-2 and cos > 0.9999, (split, diff, cos)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-4)


def test_fast_rope_selection_reader_pins_pair_map():
    """A reader that keeps original pairs P (q_reduce = k_affine = the 0/1
    selection of dims 2p, 2p+1; k_read = the head's decoder rows of those
    dims) makes the low partition attention over exactly those dims of the
    rotated full keys and queries: a wrong pair index or band breaks it."""
    from tests._helpers import max_abs_cos, u16
    sc, _, key_freqs, q_freqs, q_pre, q = _fast_rope_problem(N=80, Nc=0)
    D, H = sc.D, sc.H
    pairs = np.array([[0, 3, 7, 15], [14, 6, 9, 2]])                # 4 pairs -> d = 8 per head
    d = 2 * pairs.shape[1]
    dims = np.stack([np.stack([2 * p, 2 * p + 1], 1).reshape(-1) for p in pairs])  # [H, d]
    sel = np.zeros((H, D, d), np.float32)
    for h in range(H):
        sel[h, dims[h], np.arange(d)] = 1.0
    wk = orc.bf16_to_f32(sc.hist[0]["k"]["w_dec_bf16"]).reshape(H, D, -1)
    group = {"heads": [0, 1], "q_reduce": orc.f32_to_bf16(sel),
             "k_read": orc.f32_to_bf16(np.stack([wk[h][dims[h]] for h in range(H)])),
             "v_read": sc.hist[0]["v"]["w_dec_bf16"].reshape(H, D, -1),
             "k_affine": orc.f32_to_bf16(sel), "v_affine": None, "rope_pairs": pairs}
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    low = np.arange(sc.N)
    out, lse = orc.fast_attend(q, None, None, key, val, np.array([], np.int64), low, [group],
                               sc.scale, D=D, key_freqs=key_freqs, q_pre_bf16=q_pre,
                               q_freqs=q_freqs)
    # the same attention from the full, rotated decode restricted to the dims
    kfull = orc.rope_apply(orc.decode(**key).reshape(sc.N, H, D), key_freqs)
    vfull = orc.bf16_to_f32(orc.decode(**val).reshape(sc.N, H, D))
    qf = orc.bf16_to_f32(q)
    kf = orc.bf16_to_f32(kfull)
    for h in range(H):
        ro, rl = orc.attention(qf[None, :, h, dims[h]], kf[None, :, h, dims[h]], vfull[None, :, h],
                               sc.scale)
        diff, cos = max_abs_cos(out[:, h], ro[0])
        assert diff < 1e-2 and cos > 0.9999, (h, diff, cos)
        np.testing.assert_allclose(lse[h], rl[0], atol=1e-4)
