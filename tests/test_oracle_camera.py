"""Pins of the oracle's camera PRoPE transform (oracle.camera_vectors /
camera_apply) by checks that do not restate it:

* the reference's own rearrange + einsum of both layouts
  (_apply_tiled_projmat prope_attention.py:120-130, _apply_contiguous_projmat
  :133-176) run in fp64 on bf16-rounded matrices (camera_kernel.py:21-24),
  element for element;
* identity matrices leave x unchanged; a permutation matrix moves dims
  exactly; P then P^-1 (in fp64) returns x to bf16 rounding;
* the MG fused layout of camera_kernel.py:15-19 (d = g*8 + 2*i + r, sub-frame
  g % 4) names the same 4-vectors as the full layout at D = 128.
"""
import numpy as np
import pytest
import torch
from einops import rearrange

import oracle.oracle as orc


def _bf16(x):
    return x.to(torch.float32).to(torch.bfloat16).to(torch.float64)


def _ref_full(feats, matrix):
    """_apply_tiled_projmat (prope_attention.py:120-130) in fp64."""
    feat_pc = rearrange(feats, "b h (s t) (p q j r) -> b h s t r p q j", s=matrix.shape[1],
                        p=4, q=4, j=4)
    out_pc = torch.einsum("bscij,bhstrpcj->bhstrpci", matrix, feat_pc)
    return rearrange(out_pc, "b h s t r p q j -> b h (s t) (p q j r)")


def _ref_sf13(feats, matrix):
    """_apply_contiguous_projmat (prope_attention.py:133-176), sub-frames
    (1, 3), 16 dims each, in fp64."""
    cam, rest = feats[..., :32], feats[..., 32:]
    cam = rearrange(cam, "b h (s t) (n f j) -> b h s t n f j", s=matrix.shape[1], n=2, f=4, j=4)
    m_sel = matrix.index_select(2, torch.tensor([1, 3]))
    out = torch.einsum("bsnij,bhstnfj->bhstnfi", m_sel, cam)
    return torch.cat([rearrange(out, "b h s t n f j -> b h (s t) (n f j)"), rest], dim=-1)


def _bits(x):
    return x.to(torch.float32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("layout,D", [("full", 128), ("full", 64), ("full", 192),
                                      ("sf13", 128), ("sf13", 48)])
def test_camera_matches_reference_einsum(layout, D):
    g = torch.Generator().manual_seed(D)
    F, T, H = 3, 5, 2
    mats = torch.eye(4).expand(1, F, 4, 4, 4) + 0.4 * torch.randn(1, F, 4, 4, 4, generator=g)
    x = (torch.randn(1, H, F * T, D, generator=g) * 3).to(torch.bfloat16)
    ref_fn = _ref_full if layout == "full" else _ref_sf13
    ref = ref_fn(x.double(), _bf16(mats))
    rows = np.repeat(np.arange(F), T)
    got = orc.camera_apply(_bits(x[0].transpose(0, 1)), mats[0].numpy()[rows], layout)
    assert np.array_equal(got, _bits(ref[0].transpose(0, 1)))


def test_camera_identity_permutation_and_inverse():
    rng = np.random.default_rng(0)
    S, H, D = 6, 2, 128
    x = orc.f32_to_bf16((rng.standard_normal((S, H, D)) * 2).astype(np.float32))
    eye = np.broadcast_to(np.eye(4, dtype=np.float32), (S, 4, 4, 4)).copy()
    for layout in ("full", "sf13"):
        assert np.array_equal(orc.camera_apply(x, eye, layout), x)
    # a permutation matrix moves dims of each vector exactly
    perm = np.eye(4, dtype=np.float32)[[2, 0, 3, 1]]
    pm = np.broadcast_to(perm, (S, 4, 4, 4)).copy()
    y = orc.camera_apply(x, pm, "full")
    for dims, _ in orc.camera_vectors("full", D):
        assert np.array_equal(y[:, :, dims], x[:, :, np.array(dims)[[2, 0, 3, 1]]])
    # P then P^-1 (both exactly representable in bf16: scaled permutations)
    p = (2.0 * perm).astype(np.float32)
    pinv = np.linalg.inv(p.astype(np.float64)).astype(np.float32)
    y = orc.camera_apply(orc.camera_apply(x, np.broadcast_to(p, (S, 4, 4, 4)).copy(), "sf13"),
                         np.broadcast_to(pinv, (S, 4, 4, 4)).copy(), "sf13")
    assert np.array_equal(y, x)
    # a general P, P^-1 pair round-trips to within bf16 rounding
    P = (np.eye(4) + 0.2 * rng.standard_normal((4, 4))).astype(np.float32)
    P = orc.bf16_to_f32(orc.f32_to_bf16(P))
    Pi = np.linalg.inv(P.astype(np.float64)).astype(np.float32)
    y = orc.camera_apply(orc.camera_apply(x, np.broadcast_to(P, (S, 4, 4, 4)).copy()),
                         np.broadcast_to(Pi, (S, 4, 4, 4)).copy())
    xf, yf = orc.bf16_to_f32(x), orc.bf16_to_f32(y)
    assert np.abs(yf - xf).max() <= 0.05 * np.abs(xf).max()


def test_camera_full_layout_is_mg_block_layout():
    """camera_kernel.py:15-19: d = g*8 + 2*i + r, 4-vector over i (j there),
    sub-frame cams[g] = g % 4 (mg35.py:60) -- the full layout at D = 128."""
    mg = sorted(([g * 8 + 2 * i + r for i in range(4)], g % 4) for g in range(16) for r in range(2))
    assert sorted(orc.camera_vectors("full", 128)) == mg


def test_camera_rejects_bad_layouts():
    with pytest.raises(ValueError):
        orc.camera_vectors("full", 96)
    with pytest.raises(ValueError):
        orc.camera_vectors("sf13", 16)


def _ref_selected(x, matrix, cams):
    """camera_selected (CN/core.py:125-137) for one head: x [S, W] reader dims
    in whole 8-dim blocks, matrix [S, 4, 4, 4], block j on sub-frame
    cams[j]; the reference's einsum "bhfgij,bhftgjr->bhftgir" with one frame
    per row (f = S, t = 1), in fp64."""
    S, W = x.shape
    selected = matrix[:, torch.as_tensor(cams)][None, None]       # b h f g i j
    values = x.reshape(1, 1, S, 1, W // 8, 4, 2)                   # b h f t g j r
    out = torch.einsum("bhfgij,bhftgjr->bhftgir", selected, values)
    return out.reshape(S, W)


@pytest.mark.parametrize("W", [32, 64, 128])
def test_camera_blocks_match_reference_camera_selected(W):
    g = torch.Generator().manual_seed(W + 1)
    S = 7
    mats = torch.eye(4).expand(S, 4, 4, 4) + 0.4 * torch.randn(S, 4, 4, 4, generator=g)
    x = (torch.randn(S, W, generator=g) * 2).to(torch.bfloat16)
    cams = torch.randint(0, 4, (W // 8,), generator=g)
    ref = _ref_selected(x.double(), _bf16(mats), cams)
    got = orc.camera_blocks_apply(_bits(x), mats.numpy(), cams.numpy())
    assert np.array_equal(got, _bits(ref))


def test_camera_blocks_j_mod_4_is_the_full_layout_at_128():
    g = torch.Generator().manual_seed(5)
    S = 6
    mats = torch.eye(4).expand(S, 4, 4, 4) + 0.3 * torch.randn(S, 4, 4, 4, generator=g)
    x = torch.randn(S, 128, generator=g).to(torch.bfloat16)
    a = orc.camera_blocks_apply(_bits(x), mats.numpy(), np.arange(16) % 4)
    b = orc.camera_apply(_bits(x)[:, None, :], mats.numpy(), "full")[:, 0]
    assert np.array_equal(a, b)
