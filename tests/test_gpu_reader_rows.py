"""nkv_reader_rows (ops.reader_rows) against the oracle: rows of a
[B, S, H, D] tensor read through a reader group -- projection by the group's
matrix, RoPE on the retained pairs at each row's position, the camera on the
reader's 8-dim blocks -- as MG's low_native segment reads the moved tokens
(mg35.py:241-249, 324-336).  The identity read is bit-exact; a projection
matches the fp64 product rounded to bf16 within one bf16 step (fp32
accumulation), and the transforms of the GPU's own projected rows are
bit-exact; the padding columns are zero."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import ops
from tests._helpers import u16

pytestmark = pytest.mark.gpu

B, S, H, D = 2, 50, 3, 128
TPF = 10  # rows per camera frame


def _inputs(dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, H, 2 * D, generator=g).to(torch.bfloat16)[..., :D]  # strided view
    ang = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6.0
    freqs = torch.polar(torch.ones_like(ang), ang)
    P = (torch.eye(4).expand(1, 5, 4, 4, 4) + 0.2 * torch.randn(1, 5, 4, 4, 4, generator=g))
    frame_mat = torch.tensor([3, 1, 4, 0, 2], dtype=torch.int32)
    cam = ops.Camera(P.contiguous().to(dev), frame_mat.to(dev), TPF)
    rows_mats = P[0].numpy()[np.repeat(frame_mat.numpy(), TPF)]          # [S, 4, 4, 4]
    return g, x, freqs, cam, rows_mats


def _oracle_transform(bits, freqs, pairs, mats, blocks):
    """bits [S, E] of one head: RoPE on pairs, then the camera on blocks."""
    y = orc.rope_apply(bits[:, None, :], freqs[:, pairs])[:, 0]
    return orc.camera_blocks_apply(y, mats, blocks)


@pytest.mark.parametrize("E,out_width", [(32, 128), (64, 64)])
def test_reader_rows_projection_rope_camera(dev, E, out_width):
    g, x, freqs, cam, mats = _inputs(dev, seed=E)
    heads = torch.tensor([2, 0], dtype=torch.int32)
    nh = 2
    w = (torch.randn(nh, D, E, generator=g) / D ** 0.5).to(torch.bfloat16)
    pairs = torch.stack([torch.randperm(D // 2, generator=g)[:E // 2] for _ in range(nh)]).int()
    blocks = torch.randint(0, 4, (nh, E // 8), generator=g, dtype=torch.int32)
    xd = x.to(dev)
    rope = ops.RopeTable.from_freqs(freqs, dev)
    plain = ops.reader_rows(xd, heads.to(dev), w.to(dev), out_width=out_width)
    full = ops.reader_rows(xd, heads.to(dev), w.to(dev), rope=rope, pairs=pairs.to(dev),
                           camera=cam, blocks=blocks.to(dev), out_width=out_width)
    assert plain.shape == (B, S, nh, out_width)
    assert not bool(plain[..., E:].any()) and not bool(full[..., E:].any())
    fnp = freqs.numpy()
    for b in range(B):
        for i in range(nh):
            xb = orc.bf16_to_f32(u16(x[b, :, int(heads[i])])).astype(np.float64)
            want = orc.bf16_to_f32(orc.f32_to_bf16((xb @ orc.bf16_to_f32(u16(w[i])).astype(np.float64))
                                                   .astype(np.float32)))
            got = plain[b, :, i, :E].float().cpu().numpy()
            # fp32 accumulation against the fp64 product: within one bf16 step
            assert np.all(np.abs(got - want) <= 2 ** -7 * np.maximum(np.abs(want), 2 ** -60)), (b, i)
            ref = _oracle_transform(u16(plain[b, :, i, :E]), fnp, pairs[i].numpy(), mats,
                                    blocks[i].numpy())
            assert np.array_equal(u16(full[b, :, i, :E]), ref), (b, i)


def test_reader_rows_identity_is_exact(dev):
    g, x, freqs, cam, mats = _inputs(dev, seed=7)
    heads = torch.tensor([1, 2, 0], dtype=torch.int32)
    pairs = torch.stack([torch.randperm(D // 2, generator=g) for _ in range(3)]).int()
    xd = x.to(dev)
    rope = ops.RopeTable.from_freqs(freqs, dev)
    copy = ops.reader_rows(xd, heads.to(dev))
    assert torch.equal(copy, xd[:, :, heads.long()])
    full = ops.reader_rows(xd, heads.to(dev), rope=rope, pairs=pairs.to(dev), camera=cam)
    fnp = freqs.numpy()
    blocks = np.arange(D // 8) % 4
    for b in range(B):
        for i in range(3):
            ref = _oracle_transform(u16(x[b, :, int(heads[i])]), fnp, pairs[i].numpy(), mats, blocks)
            assert np.array_equal(u16(full[b, :, i]), ref), (b, i)
