"""Pins of the oracle's low_native segment (oracle.fast_attend(native_low=...),
restating MG35:241-249, 324-347) by what the mathematics fixes:
- LSE-merging two attention partitions equals one softmax over the union of
  their keys, so moving current tokens out of the native partition into the
  segment of an identity reader group (identity affine maps) leaves each
  head's output as it was, up to the bf16 rounding of the extra merge;
- a selection reader (q_reduce and k_affine keeping the same d of D dims)
  scores the moved tokens on those dims only: the merged output equals one
  softmax over [native keys at full width; moved keys on the kept dims];
- a segment whose tokens no query sees merges with weight zero: the output
  equals the call without the segment, bit for bit."""
import numpy as np

import oracle.oracle as orc

D = 64


def _bits(x):
    return orc.f32_to_bf16(np.asarray(x, np.float32))


def _problem(seed, H=2, Q=9, Nc=12):
    rng = np.random.default_rng(seed)
    q = _bits(rng.standard_normal((Q, H, D)) / D ** 0.5)
    kc = _bits(rng.standard_normal((Nc, H, D)))
    vc = _bits(rng.standard_normal((Nc, H, D)))
    return rng, q, kc, vc


def _group(heads, d, sel=None):
    """A reader group dict of the oracle: identity maps, or (sel) q_reduce and
    k_affine that keep dims sel of each head; values at full width."""
    nh = len(heads)
    eye = np.eye(D, dtype=np.float32)
    g = {"heads": heads, "q_reduce": None, "k_affine": None, "v_affine": None, "lift": None,
         "k_read": np.zeros((nh, d, 8), np.uint16), "v_read": np.zeros((nh, D, 8), np.uint16)}
    if sel is not None:
        pick = _bits(eye[:, sel])
        g["q_reduce"] = np.stack([pick] * nh)
        g["k_affine"] = np.stack([pick] * nh)
    return g


def _fast(q, kc, vc, groups, mask=None, native_low=None):
    out, lse = orc.fast_attend(q, kc, vc, None, None, [], [], groups, D ** -0.5, D=D,
                               cur_mask=mask, native_low=native_low)
    return out, lse


def test_moving_tokens_to_an_identity_reader_changes_nothing():
    rng, q, kc, vc = _problem(1)
    Q, Nc = q.shape[0], kc.shape[0]
    moved = np.zeros(Nc, bool)
    moved[[1, 4, 5, 10]] = True
    ref, ref_lse = _fast(q, kc, vc, [_group([0, 1], D)])
    keep = np.ones((Q, Nc), bool) & ~moved[None]
    got, got_lse = _fast(q, kc, vc, [_group([0, 1], D)], mask=keep,
                         native_low={"k_pre_bf16": kc[moved], "v_pre_bf16": vc[moved],
                                     "mask": None})
    np.testing.assert_allclose(got, ref, atol=2 ** -7 * max(1.0, np.abs(ref).max()), rtol=0)
    np.testing.assert_allclose(got_lse, ref_lse, atol=1e-6, rtol=0)


def test_selection_reader_scores_moved_tokens_on_the_kept_dims():
    rng, q, kc, vc = _problem(2, H=1)
    Q, Nc = q.shape[0], kc.shape[0]
    moved = np.zeros(Nc, bool)
    moved[[0, 3, 7, 8]] = True
    sel = np.sort(rng.choice(D, 32, replace=False))
    keep = np.ones((Q, Nc), bool) & ~moved[None]
    got, _ = _fast(q, kc, vc, [_group([0], 32, sel)], mask=keep,
                   native_low={"k_pre_bf16": kc[moved], "v_pre_bf16": vc[moved], "mask": None})
    qf, kf, vf = (orc.bf16_to_f32(t)[:, 0].astype(np.float64) for t in (q, kc, vc))
    s = np.concatenate([qf @ kf[~moved].T, qf[:, sel] @ kf[moved][:, sel].T], 1) * D ** -0.5
    p = np.exp(s - s.max(1, keepdims=True))
    want = (p @ np.concatenate([vf[~moved], vf[moved]], 0)) / p.sum(1, keepdims=True)
    np.testing.assert_allclose(got[:, 0], want, atol=2 ** -7 * max(1.0, np.abs(want).max()), rtol=0)


def test_an_unseen_segment_merges_with_weight_zero():
    rng, q, kc, vc = _problem(3)
    Q, Nc = q.shape[0], kc.shape[0]
    moved = np.zeros(Nc, bool)
    moved[[2, 6]] = True
    keep = np.ones((Q, Nc), bool) & ~moved[None]
    base, base_lse = _fast(q, kc, vc, [_group([0, 1], D)], mask=keep)
    got, got_lse = _fast(q, kc, vc, [_group([0, 1], D)], mask=keep,
                         native_low={"k_pre_bf16": kc[moved], "v_pre_bf16": vc[moved],
                                     "mask": np.zeros((Q, int(moved.sum())), bool)})
    assert np.array_equal(got, base)
    assert np.array_equal(got_lse, base_lse)
