"""Camera PRoPE on the GPU (nkv_camera_apply, nkv_attend with camera) against
the oracle: bit-exact for the standalone transform, the fused attention within
the attention bar (max-abs 2e-2, cosine 0.9995, |dlse| < 2e-3), and the fused
path against the unfused GPU path (decode, rotate, transform, attend
uncompressed)."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import _lib, ops
from tests._helpers import Scenario, max_abs_cos, u16

pytestmark = pytest.mark.gpu


def _camera(dev, batches, n_mats, frame_mat, tpf, layout="full", seed=0):
    g = torch.Generator().manual_seed(seed)
    mats = torch.eye(4).expand(batches, n_mats, 4, 4, 4) + 0.3 * torch.randn(
        batches, n_mats, 4, 4, 4, generator=g)
    cam = ops.Camera(mats.contiguous().to(dev), torch.tensor(frame_mat, dtype=torch.int32).to(dev),
                     tpf, layout)
    return cam, mats


def _row_mats(mats_b, frame_mat, tpf, rows):
    """[len(rows), 4, 4, 4] matrices of codec rows (frame index clamped)."""
    f = np.minimum(np.asarray(rows) // tpf, len(frame_mat) - 1)
    return mats_b.numpy()[np.asarray(frame_mat)[f]]


@pytest.mark.parametrize("layout,D", [("full", 128), ("full", 64), ("sf13", 128), ("sf13", 36)])
def test_camera_apply_bitexact(dev, layout, D):
    frame_mat, tpf = [2, 0, 0, 1], 7
    cam, mats = _camera(dev, 2, 3, frame_mat, tpf, layout, seed=D)
    S = len(frame_mat) * tpf
    x = (torch.randn(2, S, 3, D, generator=torch.Generator().manual_seed(1)) * 3).to(torch.bfloat16)
    got = ops.camera_apply(x.to(dev), cam)
    torch.cuda.synchronize()
    for b in range(2):
        ref = orc.camera_apply(u16(x[b]), _row_mats(mats[b], frame_mat, tpf, np.arange(S)), layout)
        assert np.array_equal(u16(got[b].cpu()), ref), f"batch {b}"


def test_camera_apply_rows_strides_in_place_broadcast(dev):
    frame_mat, tpf = [1, 1, 0], 4
    cam, mats = _camera(dev, 1, 2, frame_mat, tpf, seed=5)
    rows = torch.tensor([11, 0, 5, 5, 9, 30], dtype=torch.int32)  # 30: past the frames, clamped
    buf = torch.randn(2, 6, 5, 136, generator=torch.Generator().manual_seed(2)).to(
        torch.bfloat16).to(dev)
    before = buf.clone()
    x = buf[:, :, 1:4, 4:132]
    ops.camera_apply(x, cam, rows=rows.to(dev), out=x)
    torch.cuda.synchronize()
    for b in range(2):
        ref = orc.camera_apply(u16(before[b, :, 1:4, 4:132]),
                               _row_mats(mats[0], frame_mat, tpf, rows.numpy()))
        assert np.array_equal(u16(x[b]), ref)
    mask = torch.ones_like(buf, dtype=torch.bool)
    mask[:, :, 1:4, 4:132] = False
    assert torch.equal(buf[mask], before[mask])


@pytest.mark.parametrize("B,N,Q,Nc,tpf,layout,with_rope", [
    (1, 300, 100, 64, 50, "full", False),     # Q within one query tile: AUTO takes key chunks
    (2, 777, 40, 100, 37, "full", True),      # ragged last chunk, per-batch matrices, RoPE first
    (1, 600, 300, 0, 100, "sf13", False),     # no current keys, the sf13 layout
])
def test_attend_camera_matches_oracle(dev, B, N, Q, Nc, tpf, layout, with_rope):
    sc = Scenario(B=B, H=3, N=N, Q=Q, Nc=Nc, rK=128, rV=128, G=32, C=8, seed=N)
    key, value = sc.codecs(dev)
    frames = -(-N // tpf)
    frame_mat = [(3 * f) % 4 for f in range(frames)]
    cam, mats = _camera(dev, B, 4, frame_mat, tpf, layout, seed=N)
    rope, freqs = None, None
    if with_rope:
        gh, gw = 1, tpf
        bands = ops.rope_bands(128, 64)
        rope = ops.Rope.from_bands(bands, list(range(frames)), gh, gw, dev)
        t, h, w = (torch.view_as_complex(x.cpu()).numpy() for x in (rope.cs_t, rope.cs_h,
                                                                    rope.cs_w))
        freqs = orc.kv_freqs((t, h, w), rope.frame_pos.cpu().numpy(), gh, gw)[:N]
    kc = None if sc.k_cur is None else sc.k_cur.to(dev)
    vc = None if sc.v_cur is None else sc.v_cur.to(dev)
    out, lse = ops.attend(sc.q.to(dev), kc, vc, key, value, rope=rope, camera=cam)
    torch.cuda.synchronize()
    for b in range(B):
        ref, ref_lse = orc.decode_attend(
            u16(sc.q[b]), None if kc is None else u16(sc.k_cur[b]),
            None if vc is None else u16(sc.v_cur[b]), sc.hist[b]["k"], sc.hist[b]["v"], sc.scale,
            key_freqs=freqs, key_cam=(_row_mats(mats[b], frame_mat, tpf, np.arange(N)), layout))
        diff, cos = max_abs_cos(out[b].float().cpu().numpy(), ref)
        assert diff <= 2e-2 and cos >= 0.9995, (b, diff, cos)
        assert np.abs(lse[b].cpu().numpy() - ref_lse).max() < 2e-3
    plain, _ = ops.attend(sc.q.to(dev), kc, vc, key, value, rope=rope)
    assert (plain.float() - out.float()).abs().max().item() > 1e-3


def test_attend_camera_equals_unfused_gpu_path(dev):
    """decode -> rope -> camera (K and V) -> attend over uncompressed keys gives
    the fused result up to the attention's own rounding (identical bf16 rows)."""
    sc = Scenario(H=2, N=520, Q=300, Nc=40, rK=384, rV=256, G=32, C=16, with_mean=True, seed=3)
    key, value = sc.codecs(dev)
    bands = ops.rope_bands(128, 64)
    rope = ops.Rope.from_bands(bands, [3, 1], 13, 20, dev)
    cam, _ = _camera(dev, 1, 2, [1, 0], 260, seed=9)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    fused, flse = ops.attend(q, kc, vc, key, value, rope=rope, camera=cam)
    kd = ops.decode(key, 2 * 128).reshape(1, sc.N, 2, 128)
    vd = ops.decode(value, 2 * 128).reshape(1, sc.N, 2, 128)
    kr = ops.camera_apply(ops.rope_apply(kd, rope), cam)
    vr = ops.camera_apply(vd, cam)
    unfused, ulse = ops.attend(q, torch.cat([kr, kc], 1), torch.cat([vr, vc], 1),
                               schedule="key_chunks")
    torch.cuda.synchronize()
    assert (fused.float() - unfused.float()).abs().max().item() < 1e-2
    assert (flse - ulse).abs().max().item() < 1e-4


def test_attend_camera_rejects_query_tiles_and_bad_layout(dev):
    sc = Scenario(H=1, N=100, Q=20, Nc=0, rK=64, rV=64, G=32, C=4)
    key, value = sc.codecs(dev)
    cam, _ = _camera(dev, 1, 1, [0], 100)
    with pytest.raises(_lib.NanoKVError, match="key-chunk schedule"):
        ops.attend(sc.q.to(dev), None, None, key, value, camera=cam, schedule="query_tiles")
    x = torch.zeros(1, 4, 1, 96, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.NanoKVError, match="D % 64"):
        ops.camera_apply(x, cam)
