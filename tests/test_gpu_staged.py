"""GPU parity of nkv_attend's staged schedule (decode the history into tile
images once, then flash attention over them with key splits and the LSE
combine), which the key-chunk decomposition runs at D = 128:
every decode variant (the decode GEMM's register epilogue: bias, centers of
1/2/4-byte ids, no centers, scale groups, bf16 scales, segment tables; the
in-LDS decode for read-time RoPE and camera), history row lists, current-key
visibility masks, ragged and empty tiles, against the oracle's
decode-then-attend: max-abs <= 2e-2, cosine >= 0.9995, |dlse| < 2e-3."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import ops
from tests._helpers import Scenario, max_abs_cos, u16

pytestmark = pytest.mark.gpu

MAX_ABS, MIN_COS = 2e-2, 0.9995


def _check(sc, dev, **kw):
    key, value = sc.codecs(dev)
    kc = None if sc.k_cur is None else sc.k_cur.to(dev)
    vc = None if sc.v_cur is None else sc.v_cur.to(dev)
    ref_kw = kw.pop("ref_kw", {})
    out, lse = ops.attend(sc.q.to(dev), kc, vc, key, value, **kw)
    out = out.float().cpu().numpy()
    lse = lse.cpu().numpy()
    for b in range(sc.B):
        ref, ref_lse = sc.reference(b, **ref_kw)
        diff, cos = max_abs_cos(out[b], ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (b, diff, cos)
        assert np.array_equal(np.isneginf(lse[b]), np.isneginf(ref_lse))
        fin = np.isfinite(ref_lse)
        if fin.any():
            assert np.abs(lse[b][fin] - ref_lse[fin]).max() < 2e-3
    return out, lse


# history ending inside a 32-key step, a 128-key tile and a 256-key chunk;
# one history key; no history; no current keys; one current key; a last
# query block of 1..31 queries; two batch items
@pytest.mark.parametrize("B,N,Nc,Q", [(1, 700, 300, 1040), (1, 256, 0, 1024), (1, 1, 129, 1100),
                                      (1, 0, 400, 1030), (1, 1000, 1, 1536), (2, 383, 77, 1057)])
def test_staged_shapes(dev, B, N, Nc, Q):
    _check(Scenario(B=B, H=2, N=N, Q=Q, Nc=Nc, rK=384, rV=256, G=32, C=16, seed=N + Q), dev)


@pytest.mark.parametrize("G,scale_dtype,with_mean,id_dtype,centers", [
    (384, torch.bfloat16, False, torch.uint8, True),
    (32, torch.float16, True, torch.int16, True),
    (64, torch.bfloat16, True, torch.int32, True),
    (32, torch.float16, True, torch.uint8, False),
])
def test_staged_codec_variants(dev, G, scale_dtype, with_mean, id_dtype, centers):
    _check(Scenario(H=2, N=600, Q=1030, Nc=90, rK=384, rV=384, G=G, C=40, scale_dtype=scale_dtype,
                    with_mean=with_mean, id_dtype=id_dtype, centers=centers, seed=G), dev)


def test_staged_ranks(dev):
    """Different K and V ranks (64 and 256: one and four decoder slices)
    through the decode GEMM."""
    _check(Scenario(H=3, N=530, Q=1100, Nc=60, rK=64, rV=256, G=32, C=8, seed=5), dev)


def test_staged_ranks_at_resident_limit(dev):
    """K at the largest rank the decode kernel holds in LDS (384, six
    slices) and V at one slice, in two launches."""
    _check(Scenario(H=2, N=600, Q=1030, Nc=50, rK=384, rV=64, G=64, C=8, seed=15), dev)


def test_staged_multi_tile_ranges(dev):
    """Blocks of the resident-decoder kernel that decode several pairs of
    tiles: 16 heads of 63 tiles in equal ranges per codec, so that ranges of
    odd tile counts cross head boundaries, and a ragged last tile."""
    _check(Scenario(H=16, N=8000, Q=1024, Nc=40, rK=384, rV=384, G=32, C=16, seed=16), dev)


def test_staged_ranges_across_heads_and_current_batches(dev):
    """Two batch items of 3 heads with 37 history tiles each (ranges of one
    or two tiles, some across a head boundary) and 6 current tiles per head,
    built by the current-key blocks in batches of 4 with a partial last
    batch."""
    _check(Scenario(B=2, H=3, N=37 * 128 - 5, Q=1030, Nc=700, rK=384, rV=384, G=32, C=16,
                    seed=17), dev)


@pytest.mark.parametrize("rows", ["scattered", "empty"])
def test_staged_history_rows(dev, rows):
    sc = Scenario(H=2, N=800, Q=1050, Nc=70, rK=128, rV=128, G=32, C=16, seed=6)
    sel = (np.sort(np.random.default_rng(3).choice(800, 411, replace=False)) if rows == "scattered"
           else np.array([], np.int64))
    hr = torch.from_numpy(sel.astype(np.int32)).to(dev)
    _check(sc, dev, hist_rows=hr, ref_kw={"hist_rows": sel})


def test_staged_visibility_mask(dev):
    """The flash kernel's masked instance: random visibility of the current
    keys per query, a query that sees no current key and one that sees all."""
    for N in (0, 300):
        sc = Scenario(H=2, N=N, Q=1040, Nc=290, rK=128, rV=128, G=32, C=8, seed=N + 1)
        mask = np.random.default_rng(N).random((sc.Q, sc.Nc)) > 0.4
        mask[0] = False
        mask[1] = True
        vis = ops.Visibility.from_bool(torch.from_numpy(mask), dev)
        out, lse = _check(sc, dev, visibility=vis, ref_kw={"cur_mask": mask})
        if N == 0:
            assert np.all(out[0][0] == 0) and np.all(np.isneginf(lse[0][:, 0]))


def _rope(dev, positions, gh, gw):
    rope = ops.Rope.from_bands(ops.rope_bands(128, 64), positions, gh, gw, dev)
    t, h, w = (torch.view_as_complex(x.cpu()).numpy() for x in (rope.cs_t, rope.cs_h, rope.cs_w))
    return rope, orc.kv_freqs((t, h, w), rope.frame_pos.cpu().numpy(), gh, gw)


def test_staged_rope(dev):
    sc = Scenario(H=2, N=777, Q=1030, Nc=100, rK=128, rV=128, G=32, C=8, seed=7)
    rope, freqs = _rope(dev, [7, 6, 5], 7, 37)
    _check(sc, dev, rope=rope, ref_kw={"key_freqs": freqs[:sc.N]})


def test_staged_camera(dev):
    """Camera P^-1 of the history keys and values (full layout), per batch
    item, with RoPE first, through the in-LDS decode."""
    from tests.test_gpu_camera import _camera, _row_mats
    B, N, tpf = 2, 500, 100
    sc = Scenario(B=B, H=2, N=N, Q=1040, Nc=50, rK=128, rV=128, G=32, C=8, seed=8)
    frame_mat = [(3 * f) % 4 for f in range(N // tpf)]
    cam, mats = _camera(dev, B, 4, frame_mat, tpf, "full", seed=8)
    rope, freqs = _rope(dev, list(range(N // tpf)), 10, tpf // 10)
    key, value = sc.codecs(dev)
    out, lse = ops.attend(sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value,
                          rope=rope, camera=cam)
    for b in range(B):
        ref, ref_lse = sc.reference(b, key_freqs=freqs[:N],
                                    key_cam=(_row_mats(mats[b], frame_mat, tpf, np.arange(N)),
                                             "full"))
        diff, cos = max_abs_cos(out[b].float().cpu().numpy(), ref)
        assert diff <= MAX_ABS and cos >= MIN_COS, (b, diff, cos)
        assert np.abs(lse[b].cpu().numpy() - ref_lse).max() < 2e-3


def test_staged_segments(dev):
    """A segment table (per-segment center tables) through the decode GEMM:
    equal to the flat codec it concatenates, and against the oracle."""
    from tests.test_gpu_select import _flat, _segmented_cache
    from nanokv_amd import nanokv_codec as nc, synth
    from tests._helpers import oracle_codec
    H, D = 2, 128
    sh = synth.Shape("seg", H=H, D=D, N=0, Q=0, Nc=0, rK=128, rV=128, G=32, C=64)
    lay = synth.make_layer(sh, seed=4)
    cache_k, cache_v = _segmented_cache(dev, 31, sh, lay, [300, 260, 96, 400], seed=90)
    key, value = nc.history_codecs(cache_k, cache_v, dev)
    g = torch.Generator().manual_seed(6)
    q = (torch.randn(1, 1100, H, D, generator=g) / D ** 0.5).to(torch.bfloat16).to(dev)
    kc = torch.randn(1, 70, H, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(1, 70, H, D, generator=g).to(torch.bfloat16).to(dev)
    out_s, lse_s = ops.attend(q, kc, vc, key, value)
    out_f, lse_f = ops.attend(q, kc, vc, _flat(key), _flat(value))
    torch.cuda.synchronize()
    assert torch.equal(out_s.view(torch.int16), out_f.view(torch.int16))
    assert torch.equal(lse_s, lse_f)
    sname = "bf16" if key.scale_dtype == torch.bfloat16 else "fp16"
    ref, ref_lse = orc.decode_attend(u16(q[0]), u16(kc[0]), u16(vc[0]), oracle_codec(key, 0, sname),
                                     oracle_codec(value, 0, sname), D ** -0.5)
    diff, cos = max_abs_cos(out_s[0].float().cpu().numpy(), ref)
    assert diff <= MAX_ABS and cos >= MIN_COS, (diff, cos)
    assert np.abs(lse_s[0].cpu().numpy() - ref_lse).max() < 2e-3


def test_staged_workspace_and_repeat(dev):
    """The workspace size query covers the staged path; a caller workspace
    reused across calls of different sizes gives the allocated-call result."""
    big = Scenario(H=2, N=900, Q=1100, Nc=100, rK=128, rV=128, G=32, C=8, seed=10)
    small = Scenario(H=2, N=300, Q=1024, Nc=40, rK=128, rV=128, G=32, C=8, seed=11)
    kb, vb = big.codecs(dev)
    ws = torch.empty(ops.attend_workspace_size(big.q.to(dev), big.N, big.Nc, kb, vb),
                     dtype=torch.uint8, device=dev)
    for sc in (big, small):
        key, value = sc.codecs(dev)
        args = (sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value)
        a, la = ops.attend(*args)
        b_, lb = ops.attend(*args, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int16), b_.view(torch.int16))
        assert torch.equal(la, lb)


def test_staged_kernel_events(dev):
    """Kernel events stamped by the flash launch itself: the output is
    bit-identical to a call without events, and the bracketed time is
    positive and inside the call's own."""
    sc = Scenario(H=2, N=900, Q=1100, Nc=100, rK=128, rV=128, G=32, C=8, seed=12)
    key, value = sc.codecs(dev)
    args = (sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev), key, value)
    plain, lp = ops.attend(*args)
    kb, ke = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cb, ce = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    kb.record()  # torch creates the underlying events on their first record
    ke.record()
    torch.cuda.synchronize()
    assert kb.cuda_event and ke.cuda_event
    cb.record()
    timed, lt = ops.attend(*args, kernel_events=(kb.cuda_event, ke.cuda_event))
    ce.record()
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16), timed.view(torch.int16))
    assert torch.equal(lp, lt)
    kms, cms = kb.elapsed_time(ke), cb.elapsed_time(ce)
    assert 0.0 < kms <= cms, (kms, cms)
