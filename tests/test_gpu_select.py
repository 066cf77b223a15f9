"""Parity of the history selection features of nkv_attend against the oracle:
segment tables (per-segment center tables read in place, no concatenation),
history row lists, current-key visibility masks (attention_lse masks,
attention_grouped_mask, the hook's keep masks) and per-row RoPE tables.
All calls go through the C ABI (ops -> libnanokv_hip.so)."""
import os

import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, nanokv_codec as nc, ops, synth
from tests._helpers import Scenario, max_abs_cos, oracle_codec, u16

pytestmark = pytest.mark.gpu

MAX_ABS, MIN_COS = 2e-2, 0.9995


def _segmented_cache(dev, layer_id, sh, lay, lengths, seed):
    """A paired K/V segment list encoded by encode_tensor with per-segment
    C64 centers (no shared table registered): every segment has its own
    center table, as the reference's cache does."""
    nc.register_operator("k", layer_id, encoder=lay.w_enc_k.to(dev), decoder=lay.w_dec_k.to(dev))
    nc.register_operator("v", layer_id, encoder=lay.w_enc_v.to(dev), decoder=lay.w_dec_v.to(dev))
    nc.register_centers("k", layer_id, None)
    nc.register_centers("v", layer_id, None)
    cache_k = cache_v = None
    for i, n in enumerate(lengths):
        k = synth.history_rows(sh, lay.centers_k, n, seed=seed + i).to(dev)[None].to(torch.bfloat16)
        v = synth.history_rows(sh, lay.centers_v, n, seed=seed + 50 + i).to(dev)[None]
        cache_k = nc.concat_values(cache_k, nc.encode_tensor("k", layer_id, k))
        cache_v = nc.concat_values(cache_v, nc.encode_tensor("v", layer_id, v.to(torch.bfloat16)))
    return cache_k, cache_v


def _flat(cd):
    """The same codec as one flat array: codes, scales and ids concatenated,
    tables concatenated with each segment's ids offset (int16)."""
    segs = cd.segments.segments
    ids, tables, base = [], [], 0
    for sg in segs:
        ids.append(sg.ids.to(torch.int32) + base)
        tables.append(sg.centers)
        base += int(sg.centers.shape[1])
    return ops.Codec(packed=torch.cat([s.packed for s in segs], 1).contiguous(),
                     scales=torch.cat([s.scales for s in segs], 1).contiguous(),
                     w_dec=cd.w_dec, group=cd.group, mean=cd.mean,
                     ids=torch.cat(ids, 1).to(torch.int16).contiguous(),
                     centers=torch.cat(tables, 1).contiguous())


def test_segment_table_equals_concatenated_codec(dev):
    """A 5-segment cache with per-segment C64 tables: the fused call over the
    segment table equals, bit for bit, the call over the concatenated codec
    (ids offset into the concatenated tables), and meets the bar against the
    oracle's decode-then-attend."""
    H, D, layer_id = 2, 128, 21
    sh = synth.Shape("seg", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=64)
    lay = synth.make_layer(sh, seed=3)
    os.environ.pop("NANOKV_SCALE_GROUP", None)
    cache_k, cache_v = _segmented_cache(dev, layer_id, sh, lay, [100, 260, 96, 300, 70], seed=70)
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    assert key.segments is not None and len(key.segments.segments) == 5
    tables = {sg.centers.data_ptr() for sg in key.segments.segments}
    assert len(tables) == 5  # every segment has its own table
    # the table is remembered for the same segment list
    assert nc.history_codecs(cache_k, cache_v, dev)[0] is key
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(1, 300, H, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, 40, H, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, 40, H, D, generator=g).to(torch.bfloat16).to(dev)
    out_s, lse_s = ops.attend(q, kc, vc, key, value)
    out_f, lse_f = ops.attend(q, kc, vc, _flat(key), _flat(value), schedule="key_chunks")
    torch.cuda.synchronize()
    assert torch.equal(out_s.view(torch.int16), out_f.view(torch.int16))
    assert torch.equal(lse_s, lse_f)
    sname = "bf16" if key.scale_dtype == torch.bfloat16 else "fp16"
    ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), oracle_codec(key, 0, sname),
                                     oracle_codec(value, 0, sname), D ** -0.5)
    diff, cos = max_abs_cos(out_s[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse_s[0].cpu().numpy() - ref_lse).max() < 2e-3


def test_codec_history_attention_over_segments(dev):
    """The payload API reads a segment list through the segment table and
    meets the bar against the oracle over the same payload bits."""
    H, D, layer_id = 3, 128, 22
    sh = synth.Shape("seg2", H=H, D=D, N=0, Q=0, Nc=0, rK=256, rV=128, G=32, C=64)
    lay = synth.make_layer(sh, seed=4)
    cache_k, cache_v = _segmented_cache(dev, layer_id, sh, lay, [128, 128, 200], seed=90)
    g = torch.Generator().manual_seed(6)
    q = (torch.randn(1, H, 64, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    out, lse = codec_native.codec_history_attention(q, cache_k, cache_v, return_lse=True)
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    sname = "bf16" if key.scale_dtype == torch.bfloat16 else "fp16"
    ref, ref_lse = orc.decode_attend(u16(q[0].permute(1, 0, 2)), None, None,
                                     oracle_codec(key, 0, sname), oracle_codec(value, 0, sname),
                                     D ** -0.5)
    diff, cos = max_abs_cos(out[0].permute(1, 0, 2).float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)


@pytest.mark.parametrize("rows", ["frames", "scattered", "empty"])
def test_history_row_list(dev, rows):
    """hist_rows attends only the listed codec rows (the chunk-id frame filter
    of wan_video_dit.py:509-530)."""
    sc = Scenario(H=2, N=600, Q=90, Nc=50, rK=384, rV=256, G=32, C=16, seed=4)
    if rows == "frames":
        sel = np.concatenate([np.arange(0, 150), np.arange(300, 450)])
    elif rows == "scattered":
        sel = np.sort(np.random.default_rng(2).choice(600, 333, replace=False))
    else:
        sel = np.array([], np.int64)
    key, value = sc.codecs(dev)
    hr = torch.from_numpy(sel.astype(np.int32)).to(dev)
    out, lse = ops.attend(sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value,
                          hist_rows=hr)
    ref, ref_lse = sc.reference(0, hist_rows=sel)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (rows, diff, cos)
    assert np.abs(lse[0].cpu().numpy() - ref_lse).max() < 2e-3


@pytest.mark.parametrize("Nc", [64, 300])
def test_current_key_visibility_mask(dev, Nc):
    """A random boolean visibility of the current keys per query (including a
    query that sees no current key, and one that sees all), with and
    without history: attention over the visible keys only."""
    for N in (0, 260):
        sc = Scenario(H=2, N=N, Q=70, Nc=Nc, rK=128, rV=128, G=32, C=8, seed=N + Nc)
        rng = np.random.default_rng(Nc)
        mask = rng.random((sc.Q, Nc)) > 0.5
        mask[0] = False
        mask[1] = True
        vis = ops.Visibility.from_bool(torch.from_numpy(mask), dev)
        key, value = sc.codecs(dev)
        out, lse = ops.attend(sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value,
                              visibility=vis)
        ref, ref_lse = sc.reference(0, cur_mask=mask)
        got = out[0].float().cpu().numpy()
        diff, cos = max_abs_cos(got, ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (N, Nc, diff, cos)
        gl, rl = lse[0].cpu().numpy(), ref_lse
        assert np.array_equal(np.isneginf(gl), np.isneginf(rl))
        fin = np.isfinite(rl)
        assert np.abs(gl[fin] - rl[fin]).max() < 2e-3
        if N == 0:  # the query that sees nothing gets (0, -inf)
            assert np.all(got[0] == 0) and np.all(np.isneginf(gl[:, 0]))


def test_attention_lse_mask_and_grouped_mask(dev):
    """codec_native.attention_lse with a [1, 1, Q, N] boolean mask and
    attention_grouped_mask with chunk-id query groups (CN/core.py:45-72,
    94-103) against the oracle's masked attention."""
    g = torch.Generator().manual_seed(8)
    B, H, Qn, N, D = 1, 3, 96, 200, 128
    q = (torch.randn(B, H, Qn, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    k = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev)
    mask = torch.rand(Qn, N, generator=g) > 0.3
    out, lse = codec_native.attention_lse(q, k, v, mask[None, None].to(dev), scale=D ** -0.5)

    def ref_of(m):
        o, l = orc.attention(orc.bf16_to_f32(u16(q[0])), orc.bf16_to_f32(u16(k[0])),
                             orc.bf16_to_f32(u16(v[0])), D ** -0.5, mask=m)
        return o, l
    ro, rl = ref_of(mask.numpy())
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ro)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse[0].cpu().numpy() - rl).max() < 2e-3
    # chunk-id groups: queries of group i see keys of group i and anchors
    q_ids = torch.arange(Qn) // 32 - 1          # -1 (anchor), 0, 1
    k_ids = torch.arange(N) * 3 // N - 1
    keep = torch.where((q_ids < 0)[:, None], (k_ids < 0)[None].expand(Qn, N),
                       (q_ids[:, None] == k_ids[None]) | (k_ids < 0)[None])
    out2, lse2 = codec_native.attention_grouped_mask(q, k, v, keep[None, None].to(dev),
                                                     q_ids.to(dev), scale=D ** -0.5)
    ro2, rl2 = ref_of(keep.numpy())
    diff, cos = max_abs_cos(out2[0].float().cpu().numpy(), ro2)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse2[0].cpu().numpy() - rl2).max() < 2e-3


def test_rope_table_equals_rope_bands(dev):
    """The per-row RoPE table (the reference's cache_freqs form) rotates the
    history keys exactly as the factored frame bands do."""
    sc = Scenario(H=2, N=4 * 60, Q=40, Nc=20, rK=128, rV=128, G=32, C=8, seed=9)
    rope_b = ops.Rope.from_bands(ops.rope_bands(128, 64), [3, 7, 11, 15], 6, 10, dev)
    # the reference's per-token table [240, 1, 64] from the very bands the GPU reads
    t, h, w = (torch.view_as_complex(x.cpu()).numpy() for x in (rope_b.cs_t, rope_b.cs_h,
                                                                rope_b.cs_w))
    freqs = orc.kv_freqs((t, h, w), rope_b.frame_pos.cpu().numpy(), 6, 10)
    rope_t = ops.RopeTable.from_freqs(torch.from_numpy(freqs)[:, None], dev)
    key, value = sc.codecs(dev)
    args = (sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value)
    out_b, lse_b = ops.attend(*args, rope=rope_b)
    out_t, lse_t = ops.attend(*args, rope=rope_t)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), out_t.view(torch.int16))
    ref, _ = sc.reference(0, key_freqs=freqs)
    diff, cos = max_abs_cos(out_t[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
