"""The maybe_attention drop-in (nanokv_amd.mg35) end to end on the GPU, with
the reference hook's call signature: a segment-list cache written by the
hook's own commit (per-segment C64 tables), a manifest binding a reader
checkpoint to the operator file by SHA-256, per-token RoPE tables, the camera
PRoPE, a mosaic hole mask and chunk-id visibility.  The result is checked
against the oracle's fast_attend fed in the reference's order
(MG35:192-347): routing, RoPE, camera, masks, partitions and merge."""
import hashlib
import json
import types

import numpy as np
import pytest
import torch

import oracle.oracle as orc
from tests._mg35_ref import keep_reference, route_reference
from nanokv_amd import codec_native, mg35, nanokv_codec as nc, ops, synth
from tests._helpers import max_abs_cos, oracle_codec, oracle_groups, u16

pytestmark = pytest.mark.gpu

MAX_ABS, MIN_COS = 2e-2, 0.9995
H, D, LAYER, GH, GW = 2, 128, 5, 5, 8
TF = GH * GW  # tokens per frame


def _setup(dev, tmp_path, monkeypatch, policy):
    monkeypatch.setenv("MG35_KVCODEC_C64_CLUSTERS", "16")
    for k in ("NANOKV_SCALE_GROUP", "NANOKV_SCALE_DTYPE", "NANOKV_QUANT_MODE"):
        monkeypatch.delenv(k, raising=False)
    sh = synth.Shape("mg35", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=128, C=16)
    lay = synth.make_layer(sh, seed=LAYER)
    nc.register_operator("k", LAYER, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev))
    nc.register_operator("v", LAYER, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev))
    nc.register_centers("k", LAYER, None)
    nc.register_centers("v", LAYER, None)
    payload = synth.make_readers(sh, lay, full_heads=(0,), d=64)
    reader_file = tmp_path / "layer.pt"
    torch.save(payload, reader_file)
    op = tmp_path / "codec.pt"
    op.write_bytes(b"frozen operator")
    manifest = {"format": "codec_native_manifest_v1", "model": "matrix-game-3.5",
                "codec_operator_sha256": hashlib.sha256(op.read_bytes()).hexdigest(),
                "policy": policy,
                "layers": {f"0:{LAYER}": {"sha256": hashlib.sha256(reader_file.read_bytes())
                                          .hexdigest(), "calibrated": True, "path": "layer.pt"}}}
    mf = tmp_path / "manifest.json"
    mf.write_text(json.dumps(manifest))
    monkeypatch.setenv("MG35_CODEC_NATIVE_ENABLE", "1")
    monkeypatch.setenv("MG35_KVCODEC_MODE", "worldplay_method")
    monkeypatch.setenv("MG35_KVCODEC_PREPACKED_OPERATOR_PATH", str(op))
    monkeypatch.setenv("MG35_CODEC_NATIVE_MANIFEST", str(mf))
    codec_native._READER_BANKS.clear()  # the manifest is read once per path
    return sh, lay, payload


def _attn(disable_t=False):
    return types.SimpleNamespace(o=lambda x: x, prope_camera_layout="full", use_prope=True,
                                 prope_disable_native_rope=False, prope_disable_t_rope=disable_t,
                                 rope_t_pairs=22)


def _freqs(positions):
    bands = ops.rope_bands(D, 64)
    bands_np = tuple(b.numpy() for b in bands)
    return orc.kv_freqs(bands_np, positions, GH, GW)  # [frames * TF, D/2] complex128


@pytest.mark.parametrize("camera,disable_t", [(False, False), (True, False), (True, True)])
def test_maybe_attention_against_oracle(dev, tmp_path, monkeypatch, camera, disable_t):
    _hook_case(dev, tmp_path, monkeypatch, camera, disable_t, "none")


@pytest.mark.parametrize("low_native,camera,disable_t", [("all", True, False), ("mosaic", False, False),
                                                         ("current", True, True)])
def test_maybe_attention_low_native(dev, tmp_path, monkeypatch, low_native, camera, disable_t):
    """MG's low_native extension (MG35:171-175, 241-249, 324-347): the mosaic
    and / or current tokens leave the native partition and are read by each
    reader group through its affine maps, with their own RoPE, P^-1 and
    visibility, merged after the codec low rows; against the oracle's
    native_low segment."""
    _hook_case(dev, tmp_path, monkeypatch, camera, disable_t, low_native)


def _hook_case(dev, tmp_path, monkeypatch, camera, disable_t, low_native):
    policy = {"recent_native_frames": 2, "anchor_stride": 2, "sink_native_frames": 1,
              "low_native": low_native}
    sh, lay, payload = _setup(dev, tmp_path, monkeypatch, policy)
    g = torch.Generator().manual_seed(11)
    # history: 7 frames committed in 4 chunks (4 segments), chunk ids per frame
    cache = {}
    chunks = [([0, 1], [-1, -1]), ([2, 3], [0, 0]), ([4], [1]), ([5, 6], [0, 0])]
    for frames, ids in chunks:
        n = len(frames) * TF
        k = (torch.randn(1, n, H * D, generator=g)).to(torch.bfloat16).to(dev)
        v = (torch.randn(1, n, H * D, generator=g)).to(torch.bfloat16).to(dev)
        mg35._commit(cache, k, v, layer_idx=LAYER, cur_frames=frames, cur_positions=None,
                     cur_cache_chunk_ids=ids)
    assert len(nc.segments_of(cache["k"])) == 4 and cache["frames"] == list(range(7))
    N = 7 * TF
    M, S = TF, 2 * TF                      # one mosaic frame, two current frames
    mosaic_frames, cur_frames = [7], [8, 9]
    cache_freqs = _freqs(list(range(7)))
    freqs_cur = _freqs([7, 8, 9])
    q_pre = (torch.randn(1, M + S, H * D, generator=g) / D ** 0.5).to(torch.bfloat16)
    k_pre = torch.randn(1, M + S, H * D, generator=g).to(torch.bfloat16)
    v_raw = torch.randn(1, M + S, H * D, generator=g).to(torch.bfloat16)
    # the hook gets the native (rotated) q and k, as causal_self_attention_kv
    # builds them (wan_video_dit.py:414-422)
    rf = freqs_cur.copy()
    if disable_t:
        rf[:, :22] = 1
    q_nat = orc.rope_apply(u16(q_pre[0].view(M + S, H, D)), rf)
    k_nat = orc.rope_apply(u16(k_pre[0].view(M + S, H, D)), rf)

    def dev_bits(bits, shape):
        return torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).reshape(shape).to(dev)
    q_native = dev_bits(q_nat, (1, M + S, H * D))
    k_native = dev_bits(k_nat, (1, M + S, H * D))
    hole_keep = torch.rand(M, generator=g) > 0.3
    cam_info = None
    if camera:
        P = (torch.eye(4).expand(1, 10, 4, 4, 4) +
             0.2 * torch.randn(1, 10, 4, 4, 4, generator=g)).contiguous()
        P_inv = torch.linalg.inv(P).contiguous()
        P_T = P.transpose(-1, -2).contiguous()
        cam_info = (None, (P.to(dev), P_T.to(dev), P_inv.to(dev)))
    out = mg35.maybe_attention(
        _attn(disable_t), q_pre.to(dev), q_native, k_native, v_raw.to(dev),
        k_pre[:, M:].to(dev), torch.from_numpy(freqs_cur)[:, None], cam_info,
        layer_idx=LAYER, num_heads=H, mosaic_tokens=M, cur_frames=cur_frames,
        cur_positions=None, mosaic_frames=mosaic_frames, cache=cache,
        cache_freqs=torch.from_numpy(cache_freqs)[:, None], cache_frames=cache["frames"],
        cache_read_chunk_id=0, cur_cache_chunk_ids=[-1, 0], write_cache=False,
        hole_keep=hole_keep.to(dev), a1_pass=None, all_k_pre=k_pre.to(dev))
    assert out is not None and out.shape == (1, M + S, H * D)
    assert bool((out[:, :M] == 0).all())
    # ---- oracle, in the reference's order
    # routing and visibility from the independent restatements of
    # MG35:155-170 and MG35:258-283, not from the hook's own helpers
    r_prot, r_low = route_reference(cache["frames"], cache["chunk_ids"], 0, N, 2, 2, 1, False)
    prot = torch.nonzero(r_prot).flatten().numpy()
    low = torch.nonzero(r_low).flatten().numpy()
    assert prot.size and low.size
    keep = keep_reference(S, M, S, len(cur_frames), hole_keep, [-1, 0]).numpy()
    key, value = nc.history_codecs(cache["k"], cache["v"], dev)
    sname = "bf16" if key.scale_dtype == torch.bfloat16 else "fp16"
    qn = q_nat[M:]
    kc, vc = k_nat, u16(v_raw[0].view(M + S, H, D))
    kw = {}
    kf = cache_freqs.copy()
    qf = freqs_cur[M:].copy()
    if disable_t:
        kf[:, :22] = 1
        qf[:, :22] = 1
    if camera:
        rows_k = np.repeat(np.array(cache["frames"]), TF)
        rows_q = np.repeat(np.array(cur_frames), TF)
        rows_c = np.repeat(np.array(mosaic_frames + cur_frames), TF)
        qn = orc.camera_apply(qn, P_T[0].numpy()[rows_q], "full")
        kc = orc.camera_apply(kc, P_inv[0].numpy()[rows_c], "full")
        vc = orc.camera_apply(vc, P_inv[0].numpy()[rows_c], "full")
        kw = dict(key_cam=P_inv[0].numpy()[rows_k], q_cam=P_T[0].numpy()[rows_q],
                  out_cam=P[0].numpy()[rows_q])
    # low_native: the moved tokens leave the native partition's visibility
    moved = np.zeros(M + S, bool)
    if low_native in ("all", "mosaic"):
        moved[:M] = True
    if low_native in ("all", "current"):
        moved[M:] = True
    if moved.any():
        lf = freqs_cur[moved].copy()
        if disable_t:
            lf[:, :22] = 1
        lm = keep[:, moved]
        kw["native_low"] = {
            "k_pre_bf16": u16(k_pre[0].view(M + S, H, D))[moved],
            "v_pre_bf16": u16(v_raw[0].view(M + S, H, D))[moved],
            "freqs": lf,
            "cam": P_inv[0].numpy()[rows_c][moved] if camera else None,
            "mask": None if lm.all() else lm}
        keep = keep & ~moved[None, :]
    ref, _ = orc.fast_attend(qn, kc, vc, oracle_codec(key, 0, sname), oracle_codec(value, 0, sname),
                             prot, low, oracle_groups(payload), D ** -0.5, D=D, key_freqs=kf,
                             q_pre_bf16=u16(q_pre[0, M:].view(S, H, D)), q_freqs=qf,
                             cur_mask=keep, **kw)
    got = out[0, M:].view(S, H, D).float().cpu().numpy()
    diff, cos = max_abs_cos(got, ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (camera, disable_t, low_native, diff, cos)


def test_maybe_attention_returns_none_and_commits(dev, tmp_path, monkeypatch):
    """All active history protected: no low rows, so None (MG35:187-190);
    with low rows and write_cache the chunk is committed as a new segment
    with its frames, positions and chunk ids (MG35:73-97, 349-356)."""
    _setup(dev, tmp_path, monkeypatch, {"recent_native_frames": 8})
    g = torch.Generator().manual_seed(3)
    cache = {}
    for frames in ([0, 1], [2, 3]):
        k = torch.randn(1, 2 * TF, H * D, generator=g).to(torch.bfloat16).to(dev)
        mg35._commit(cache, k, k.clone(), layer_idx=LAYER, cur_frames=frames, cur_positions=None,
                     cur_cache_chunk_ids=None)
    S = TF
    x = (torch.randn(1, S, H * D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    freqs_cur = torch.from_numpy(_freqs([4]))[:, None]
    cache_freqs = torch.from_numpy(_freqs([0, 1, 2, 3]))[:, None]
    args = (_attn(), x, x, x, x, x, freqs_cur, None)
    kw = dict(layer_idx=LAYER, num_heads=H, mosaic_tokens=0, cur_frames=[4], cur_positions=[40],
              mosaic_frames=[], cache=cache, cache_freqs=cache_freqs,
              cache_frames=cache["frames"], cache_read_chunk_id=None, cur_cache_chunk_ids=[2],
              write_cache=True, hole_keep=None, a1_pass=None)
    assert mg35.maybe_attention(*args, **kw) is None
    assert len(nc.segments_of(cache["k"])) == 2  # the native path commits, not the hook
    # one protected frame only: frames 0..2 are low, the hook answers and commits
    _setup(dev, tmp_path, monkeypatch, {"recent_native_frames": 1})
    out = mg35.maybe_attention(*args, **kw)
    assert out is not None and out.shape == (1, S, H * D)
    assert len(nc.segments_of(cache["k"])) == 3 and len(nc.segments_of(cache["v"])) == 3
    assert cache["frames"] == [0, 1, 2, 3, 4]
    assert cache["positions"] == [0, 1, 2, 3, 40]
    assert cache["chunk_ids"] == [-1, -1, -1, -1, 2]
