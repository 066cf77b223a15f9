"""NanoKV-Fast with the camera PRoPE, current-key visibility masks and segment
tables, against the oracle's fast_attend (which follows the reference's
order: camera_selected on the reader query, keys and values, P on each
partition's output before the lift, then the LSE merge; CN/mg35.py:253-347).
The kernel leaves P to the caller, so the test applies P to its output with
nkv_camera_apply."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, nanokv_codec as nc, ops, synth
from tests._helpers import Scenario, max_abs_cos, oracle_codec, oracle_groups, u16

pytestmark = pytest.mark.gpu

MAX_ABS, MIN_COS = 2e-2, 0.9995


def _mats(n, seed, amp=0.2):
    g = torch.Generator().manual_seed(seed)
    return (torch.eye(4).expand(1, n, 4, 4, 4) + amp * torch.randn(1, n, 4, 4, 4, generator=g))


@pytest.mark.parametrize("d", [32, 64])
def test_fast_camera_against_oracle(dev, d):
    """Identity readers on head 0, d-wide readers on the others; 4 history
    frames of 60 rows with cameras 0..3, queries in 2 frames of cameras 4, 5;
    the last frame protected."""
    sc = Scenario(H=3, D=128, N=240, Q=64, Nc=64, rK=128, rV=128, G=32, C=8, seed=d)
    F, tpf = 4, 60
    P = _mats(6, 1).contiguous()
    P_T = P.transpose(-1, -2).contiguous()
    P_inv = torch.linalg.inv(P).contiguous()
    hist_frames = [0, 1, 2, 3]
    q_frames = [4, 5]
    cam_k = ops.Camera(P_inv.to(dev), torch.tensor(hist_frames, dtype=torch.int32, device=dev), tpf)
    cam_q = ops.Camera(P_T.to(dev), torch.tensor(q_frames, dtype=torch.int32, device=dev), 32)
    cam_o = ops.Camera(P.to(dev), torch.tensor(q_frames, dtype=torch.int32, device=dev), 32)
    # the current keys live in the query frames: P^-1 of frames 4, 5
    cam_c = ops.Camera(P_inv.to(dev), torch.tensor(q_frames, dtype=torch.int32, device=dev), 32)
    q_pre = sc.q.to(dev)
    q_nat = ops.camera_apply(q_pre, cam_q)
    kc = ops.camera_apply(sc.k_cur.to(dev), cam_c)
    vc = ops.camera_apply(sc.v_cur.to(dev), cam_c)
    payload = synth.make_readers(sc.shape, sc.layer, full_heads=(0,), d=d)
    reader = codec_native.ReaderLayer(payload, dev)
    key, value = sc.codecs(dev)
    protect = torch.arange(sc.N, device=dev) >= 180
    pr = torch.nonzero(protect).flatten().to(torch.int32)
    lr = torch.nonzero(~protect).flatten().to(torch.int32)
    out, lse = ops.fast_attend(q_nat, kc, vc, key, value, pr, lr,
                               [g.tensors(camera=True) for g in reader.groups],
                               q_pre=q_pre, camera=cam_k, q_camera=cam_q)
    out = ops.camera_apply(out, cam_o)
    rows_k = np.repeat(np.array(hist_frames), tpf)
    rows_q = np.repeat(np.array(q_frames), 32)
    ref, ref_lse = orc.fast_attend(u16(q_nat[0]), u16(kc[0]), u16(vc[0]), sc.hist[0]["k"],
                                   sc.hist[0]["v"], pr.cpu().numpy(), lr.cpu().numpy(),
                                   oracle_groups(payload), sc.scale, D=sc.D,
                                   q_pre_bf16=u16(q_pre[0]), key_cam=P_inv[0].numpy()[rows_k],
                                   q_cam=P_T[0].numpy()[rows_q], out_cam=P[0].numpy()[rows_q])
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (d, diff, cos)
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3


def test_fast_visibility_mask_against_oracle(dev):
    """A current-key mask applies to the native partition of every head."""
    sc = Scenario(H=2, D=128, N=300, Q=80, Nc=96, rK=128, rV=128, G=32, C=8, seed=2)
    mask = np.random.default_rng(1).random((sc.Q, sc.Nc)) > 0.4
    mask[3] = False
    vis = ops.Visibility.from_bool(torch.from_numpy(mask), dev)
    payload = synth.make_readers(sc.shape, sc.layer, full_heads=(1,), d=32)
    reader = codec_native.ReaderLayer(payload, dev)
    key, value = sc.codecs(dev)
    protect = torch.zeros(sc.N, dtype=torch.bool, device=dev)
    protect[200:] = True
    pr = torch.nonzero(protect).flatten().to(torch.int32)
    lr = torch.nonzero(~protect).flatten().to(torch.int32)
    out, lse = ops.fast_attend(sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value, pr,
                               lr, [g.tensors() for g in reader.groups], visibility=vis)
    ref, ref_lse = orc.fast_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]),
                                   sc.hist[0]["k"], sc.hist[0]["v"], pr.cpu().numpy(),
                                   lr.cpu().numpy(), oracle_groups(payload), sc.scale, D=sc.D,
                                   cur_mask=mask)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)


def test_fast_over_segments_with_own_tables(dev):
    """fast_history_attention over a segment list whose segments have their
    own C64 center tables: the reader tables of every segment are projected
    in one launch and the low rows read row center_base + id."""
    H, D, layer_id = 2, 128, 31
    sh = synth.Shape("fseg", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=64)
    lay = synth.make_layer(sh, seed=8)
    nc.register_operator("k", layer_id, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev))
    nc.register_operator("v", layer_id, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev))
    nc.register_centers("k", layer_id, None)
    nc.register_centers("v", layer_id, None)
    cache_k = cache_v = None
    for c in range(4):
        k = synth.history_rows(sh, lay.centers_k, 80, seed=10 + c).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, 80, seed=20 + c).to(dev)[None].to(torch.bfloat16)
        cache_k = nc.concat_values(cache_k, nc.encode_tensor("k", layer_id, k))
        cache_v = nc.concat_values(cache_v, nc.encode_tensor("v", layer_id, v))
    payload = synth.make_readers(sh, lay, full_heads=(0,), d=64)
    reader = codec_native.ReaderLayer(payload, dev)
    g = torch.Generator().manual_seed(12)
    q = (torch.randn(1, H, 48, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, H, 16, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, H, 16, D, generator=g).to(torch.bfloat16).to(dev)
    protect = torch.arange(320, device=dev) >= 240
    out, lse = codec_native.fast_history_attention(q, cache_k, cache_v, kc, vc, reader, protect,
                                                   return_lse=True)
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    assert key.segments is not None
    sname = "bf16" if key.scale_dtype == torch.bfloat16 else "fp16"
    prot = torch.nonzero(protect).flatten().cpu().numpy()
    low = torch.nonzero(~protect).flatten().cpu().numpy()
    ref, ref_lse = orc.fast_attend(u16(q[0].permute(1, 0, 2)), u16(kc[0].permute(1, 0, 2)),
                                   u16(vc[0].permute(1, 0, 2)), oracle_codec(key, 0, sname),
                                   oracle_codec(value, 0, sname), prot, low,
                                   oracle_groups(payload), D ** -0.5, D=D)
    diff, cos = max_abs_cos(out[0].permute(1, 0, 2).float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)


def _split_groups(payload, parts):
    """The payload's reader group 1 split into `parts` groups of its heads."""
    g = payload["groups"][1]
    n = len(g["heads"])
    cuts = [round(i * n / parts) for i in range(parts + 1)]
    split = [{k: v[a:b] for k, v in g.items()} for a, b in zip(cuts[:-1], cuts[1:])]
    return dict(payload, groups=[payload["groups"][0]] + split)


@pytest.mark.parametrize("parts", [1, 3])
def test_fast_out_camera_equals_separate_apply(dev, parts):
    """o_camera: the call's P on the merged output gives the bits of
    nkv_camera_apply on the output of the call without it -- on the one
    staged launch (2 groups, P in its combine) and on the per-group path
    (4 groups, one partition more than one launch holds)."""
    sc = Scenario(H=5, D=128, N=300, Q=96, Nc=32, rK=128, rV=128, G=32, C=8, seed=4 + parts)
    P = _mats(6, 3).contiguous()
    P_T = P.transpose(-1, -2).contiguous()
    P_inv = torch.linalg.inv(P).contiguous()
    tpf = 60
    qf = torch.tensor([4, 5], dtype=torch.int32, device=dev)
    cam_k = ops.Camera(P_inv.to(dev), torch.tensor([0, 1, 2, 3, 0], dtype=torch.int32,
                                                   device=dev), tpf)
    cam_q = ops.Camera(P_T.to(dev), qf, 48)
    cam_o = ops.Camera(P.to(dev), qf, 48)
    payload = _split_groups(synth.make_readers(sc.shape, sc.layer, full_heads=(0,), d=32), parts)
    reader = codec_native.ReaderLayer(payload, dev)
    assert len(reader.groups) == 1 + parts
    key, value = sc.codecs(dev)
    protect = torch.arange(sc.N, device=dev) >= 240
    pr = torch.nonzero(protect).flatten().to(torch.int32)
    lr = torch.nonzero(~protect).flatten().to(torch.int32)
    q_pre = sc.q.to(dev)
    q = ops.camera_apply(q_pre, cam_q)
    args = (q, sc.k_cur.to(dev), sc.v_cur.to(dev), key, value, pr, lr,
            [g.tensors(camera=True) for g in reader.groups])
    kw = dict(q_pre=q_pre, camera=cam_k, q_camera=cam_q)
    raw, lse = ops.fast_attend(*args, **kw)
    fused, lse_f = ops.fast_attend(*args, **kw, out_camera=cam_o)
    torch.cuda.synchronize()
    assert torch.equal(fused, ops.camera_apply(raw, cam_o))
    assert torch.equal(lse, lse_f)
    assert not torch.equal(fused, raw)
