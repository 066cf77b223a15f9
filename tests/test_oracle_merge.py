"""Pins of the oracle's partition merges of the HY and LingBot Fast paths
(oracle.lift_lse_combine, oracle.finish) by what the mathematics fixes:
merging two attention partitions by their LSEs equals one softmax over the
union of their keys, so a lifted low partition merged into the native one
equals attending both key sets at once with the low values lifted; the
PRoPE quartet mix is the Main lift by a block-structured matrix; the
value-mean correction shifts every low value by mean - projected."""
import numpy as np

import oracle.oracle as orc


def _attend(q, k, v, scale):
    s = (q @ k.T) * scale
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    return (p @ v) / p.sum(-1, keepdims=True), (m[:, 0] + np.log(p.sum(-1)))


def _union(q, kn, vn, ql, kl, vl_lifted, scale):
    s = np.concatenate([(q @ kn.T) * scale, (ql @ kl.T) * scale], 1)
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p @ np.concatenate([vn, vl_lifted], 0)) / p.sum(-1, keepdims=True)


def _expand_mix(mix):
    """The [Dlow, 128] matrix of the PRoPE quartet mix: L[4k+c, 4j+c] = mix[k, j]."""
    kq, jn = mix.shape
    L = np.zeros((4 * kq, 4 * jn))
    for c in range(4):
        L[c::4, c::4] = mix
    return L


def test_lift_lse_combine_is_one_softmax_over_both_key_sets():
    rng = np.random.default_rng(0)
    B, H, Q, Dl, Nn, Nl = 2, 3, 7, 64, 11, 9
    scale = 128 ** -0.5
    native = np.empty((2 * B, H, Q, 128))
    low = np.empty((2 * B, H, Q, Dl))
    nl = np.empty((2 * B, H, Q))
    hl = np.empty((2 * B, H, Q))
    main_lift = rng.normal(size=(H, Dl, 128)) / 8
    mix = rng.normal(size=(H, Dl // 4, 32)) / 4
    want = np.empty_like(native)
    for b in range(2 * B):
        for h in range(H):
            q, ql = rng.normal(size=(Q, 128)), rng.normal(size=(Q, Dl))
            kn, vn = rng.normal(size=(Nn, 128)), rng.normal(size=(Nn, 128))
            kl, vl = rng.normal(size=(Nl, Dl)), rng.normal(size=(Nl, Dl))
            native[b, h], nl[b, h] = _attend(q, kn, vn, scale)
            low[b, h], hl[b, h] = _attend(ql, kl, vl, scale)
            L = main_lift[h] if b < B else _expand_mix(mix[h])
            want[b, h] = _union(q, kn, vn, ql, kl, vl @ L, scale)
    got = orc.lift_lse_combine(native, nl, low, main_lift, mix, hl)
    assert np.abs(got - want).max() < 1e-12


def test_lift_lse_combine_empty_partitions():
    rng = np.random.default_rng(1)
    native = rng.normal(size=(2, 1, 3, 128))
    low = rng.normal(size=(2, 1, 3, 32))
    lift = rng.normal(size=(1, 32, 128))
    mix = rng.normal(size=(1, 8, 32))
    lse = rng.normal(size=(2, 1, 3))
    ninf = np.full((2, 1, 3), -np.inf)
    # no history keys: the native output; no native keys: the lifted history
    assert np.array_equal(orc.lift_lse_combine(native, lse, low, lift, mix, ninf), native)
    got = orc.lift_lse_combine(native, ninf, low, lift, mix, lse)
    assert np.allclose(got[:1], np.einsum("bhqk,hko->bhqo", low[:1], lift), atol=1e-12)
    assert np.allclose(got[1:], low[1:] @ _expand_mix(mix[0]), atol=1e-12)


def test_finish_is_merge_at_the_group_heads():
    rng = np.random.default_rng(2)
    B, Hn, S, D = 2, 5, 6, 16
    heads = np.array([3, 0, 4])
    native = rng.normal(size=(B, Hn, S, D))
    nlse = rng.normal(size=(B, Hn, S))
    lifted = rng.normal(size=(B, 3, S, D))
    llse = rng.normal(size=(B, 3, S))
    result = rng.normal(size=(B, Hn, S, D))
    got = orc.finish(native, nlse, lifted, llse, heads, result)
    for g, hd in enumerate(heads):
        ref, _ = orc.merge(native[:, hd], nlse[:, hd], lifted[:, g], llse[:, g])
        assert np.allclose(got[:, hd], ref, atol=1e-12)
    untouched = [h for h in range(Hn) if h not in heads]
    assert np.array_equal(got[:, untouched], result[:, untouched])
    # the value-mean correction merges lifted + mean - projected
    mean = rng.normal(size=(B, Hn, 1, D))
    proj = rng.normal(size=(B, 3, 1, D))
    got_c = orc.finish(native, nlse, lifted, llse, heads, result, mean, proj)
    for g, hd in enumerate(heads):
        ref, _ = orc.merge(native[:, hd], nlse[:, hd], lifted[:, g] + mean[:, hd] - proj[:, g],
                           llse[:, g])
        assert np.allclose(got_c[:, hd], ref, atol=1e-12)
    # projected equal to the mean of each group head's native head changes nothing
    same = orc.finish(native, nlse, lifted, llse, heads, result, mean, mean[:, heads])
    assert np.abs(same - got).max() < 1e-12


def test_finish_infinite_lse():
    """Both partitions empty (x = z = -inf): the reference keeps l = -inf and
    the origin 0, so the row is 0."""
    native = np.ones((1, 1, 2, 4))
    lifted = np.ones((1, 1, 2, 4))
    ninf = np.full((1, 1, 2), -np.inf)
    got = orc.finish(native, ninf, lifted, ninf, [0], np.full((1, 1, 2, 4), 7.0))
    assert np.array_equal(got, np.zeros((1, 1, 2, 4)))
