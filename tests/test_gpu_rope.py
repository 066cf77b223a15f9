"""Read-time RoPE on the GPU (nkv_rope_apply, nkv_attend with rope) against
the oracle: bit-exact for the standalone rotation, the fused attention within
the attention bar (max-abs 2e-2, cosine 0.9995, |dlse| < 2e-3), and the fused
path against the unfused GPU path (decode, rotate, attend uncompressed)."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import _lib, ops
from tests._helpers import Scenario, max_abs_cos, u16

pytestmark = pytest.mark.gpu


def _rope(dev, D, positions, gh, gw, end=64, disable_t=False):
    bands = ops.rope_bands(D, end)
    rope = ops.Rope.from_bands(bands, positions, gh, gw, dev, disable_t=disable_t)
    # the oracle's per-token frequencies from the very tables the GPU reads
    t = torch.view_as_complex(rope.cs_t.cpu()).numpy()
    h = torch.view_as_complex(rope.cs_h.cpu()).numpy()
    w = torch.view_as_complex(rope.cs_w.cpu()).numpy()
    fpos = rope.frame_pos.cpu().numpy()
    freqs = orc.kv_freqs((t, h, w), fpos, gh, gw)
    return rope, freqs


def test_rope_apply_rejects_incomplete_bands(dev):
    """D = 64: the reference's band split gives 11 + 10 + 10 = 31 pairs for 32
    (64 // 3 is odd), so its rope_apply cannot run either; the library refuses."""
    bands = ops.rope_bands(64, 8)
    rope = ops.Rope.from_bands(bands, [0], 2, 2, dev)
    x = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.NanoKVError, match="D / 2 pairs"):
        ops.rope_apply(x, rope)


@pytest.mark.parametrize("D", [128, 96, 12])
def test_rope_apply_bitexact(dev, D):
    gh, gw = 6, 7
    rope, freqs = _rope(dev, D, [5, 9, 0, 63], gh, gw)
    S = freqs.shape[0]
    g = torch.Generator().manual_seed(D)
    x = (torch.randn(2, S, 3, D, generator=g) * 4).to(torch.bfloat16)
    got = ops.rope_apply(x.to(dev), rope)
    torch.cuda.synchronize()
    for b in range(2):
        ref = orc.rope_apply(u16(x[b]), freqs)
        assert np.array_equal(u16(got[b].cpu()), ref), f"batch {b}"


def test_rope_apply_rows_strides_in_place(dev):
    """Row list, padded strides and an 8-byte offset (the one-pair path), in place."""
    D, gh, gw = 128, 4, 5
    rope, freqs = _rope(dev, D, [2, 30, 7], gh, gw)
    rows = torch.tensor([59, 0, 17, 17, 40, 3], dtype=torch.int32)
    g = torch.Generator().manual_seed(1)
    buf = torch.randn(1, 6, 7, 136, generator=g).to(torch.bfloat16).to(dev)
    before = buf.clone()
    x = buf[:, :, 1:6, 4:132]  # [1, S, H, D] with padded strides
    ops.rope_apply(x, rope, rows=rows.to(dev), out=x)
    torch.cuda.synchronize()
    ref = orc.rope_apply(u16(before[0, :, 1:6, 4:132]), freqs[rows.numpy()])
    assert np.array_equal(u16(x[0]), ref)
    # everything outside the view is untouched
    mask = torch.ones_like(buf, dtype=torch.bool)
    mask[:, :, 1:6, 4:132] = False
    assert torch.equal(buf[mask], before[mask])


def test_rope_disable_t_band(dev):
    D, gh, gw = 128, 3, 3
    rope, freqs = _rope(dev, D, [11, 4], gh, gw, disable_t=True)
    assert np.all(freqs[:, :22] == 1.0)
    x = torch.randn(1, 18, 2, D, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    got = ops.rope_apply(x.to(dev), rope)
    torch.cuda.synchronize()
    assert np.array_equal(u16(got[0].cpu()), orc.rope_apply(u16(x[0]), freqs))
    # the temporal dims pass through unchanged
    assert torch.equal(got[0, :, :, :44].cpu(), x[0, :, :, :44])


@pytest.mark.parametrize("N,Q,Nc,gh,gw,positions", [
    (300, 100, 64, 10, 10, [4, 9, 1]),        # Q within one query tile: AUTO still takes key chunks
    (600, 300, 0, 20, 15, [0, 33]),           # no current keys
    (777, 40, 100, 7, 37, [7, 6, 5]),         # ragged last chunk
])
def test_attend_rope_matches_oracle(dev, N, Q, Nc, gh, gw, positions):
    sc = Scenario(H=3, N=N, Q=Q, Nc=Nc, rK=128, rV=128, G=32, C=8, seed=N)
    key, value = sc.codecs(dev)
    rope, freqs = _rope(dev, 128, positions, gh, gw)
    kc = None if sc.k_cur is None else sc.k_cur.to(dev)
    vc = None if sc.v_cur is None else sc.v_cur.to(dev)
    out, lse = ops.attend(sc.q.to(dev), kc, vc, key, value, rope=rope)
    torch.cuda.synchronize()
    ref, ref_lse = orc.decode_attend(u16(sc.q[0]), None if kc is None else u16(sc.k_cur[0]),
                                     None if vc is None else u16(sc.v_cur[0]),
                                     sc.hist[0]["k"], sc.hist[0]["v"], sc.scale,
                                     key_freqs=freqs[:N])
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3
    # RoPE moved the result: the same call without it differs
    plain, _ = ops.attend(sc.q.to(dev), kc, vc, key, value)
    assert (plain.float() - out.float()).abs().max().item() > 1e-3


def test_attend_rope_equals_unfused_gpu_path(dev):
    """decode -> nkv_rope_apply -> attend over uncompressed keys gives the fused
    result up to the attention's own rounding (identical bf16 keys)."""
    sc = Scenario(H=2, N=520, Q=300, Nc=40, rK=384, rV=256, G=32, C=16, with_mean=True, seed=3)
    key, value = sc.codecs(dev)
    rope, _ = _rope(dev, 128, [3, 1], 13, 20)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    fused, flse = ops.attend(q, kc, vc, key, value, rope=rope)
    kd = ops.decode(key, 2 * 128).reshape(1, sc.N, 2, 128)
    vd = ops.decode(value, 2 * 128).reshape(1, sc.N, 2, 128)
    kr = ops.rope_apply(kd, rope)
    k_all = torch.cat([kr, kc], 1)
    v_all = torch.cat([vd, vc], 1)
    unfused, ulse = ops.attend(q, k_all, v_all, schedule="key_chunks")
    torch.cuda.synchronize()
    assert (fused.float() - unfused.float()).abs().max().item() < 1e-2
    assert (flse - ulse).abs().max().item() < 1e-4


def test_attend_rope_rejects_query_tiles_and_short_frames(dev):
    sc = Scenario(H=1, N=100, Q=20, Nc=0, rK=64, rV=64, G=32, C=4)
    key, value = sc.codecs(dev)
    rope, _ = _rope(dev, 128, [0, 1], 5, 10)
    with pytest.raises(_lib.NanoKVError, match="key-chunk schedule"):
        ops.attend(sc.q.to(dev), None, None, key, value, rope=rope, schedule="query_tiles")
    short, _ = _rope(dev, 128, [0], 5, 10)  # 50 rows for 100 history tokens
    with pytest.raises(_lib.NanoKVError) as e:
        ops.attend(sc.q.to(dev), None, None, key, value, rope=short)
    assert e.value.code == _lib.NKV_ERR_INVALID
