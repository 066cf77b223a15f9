"""Host logic of the maybe_attention drop-in (nanokv_amd.mg35) on the CPU:
its None / error contract (MG35:107-130), the frame routing against the
reference's own tensor formulation of it (MG35:155-170, independent of the
set-based restatement under test), and the hole / chunk-id keep mask
(MG35:258-283, wan_video_dit.py:454-520)."""
import hashlib
import itertools
import json
import types

import pytest
import torch

from tests._mg35_ref import keep_reference, route_reference
from nanokv_amd import codec_native, mg35


def _attn():
    return types.SimpleNamespace(o=lambda x: x, prope_camera_layout="full", use_prope=True,
                                 prope_disable_native_rope=False, prope_disable_t_rope=False,
                                 rope_t_pairs=22)


def _call(**over):
    kw = dict(layer_idx=0, num_heads=2, mosaic_tokens=0, cur_frames=[0], cur_positions=None,
              mosaic_frames=[], cache=None, cache_freqs=None, cache_frames=[],
              cache_read_chunk_id=None, cur_cache_chunk_ids=None, write_cache=False,
              hole_keep=None, a1_pass=None)
    kw.update(over)
    x = torch.zeros(1, 4, 256)
    return mg35.maybe_attention(_attn(), x, x, x, x, x, None, None, **kw)


def test_disabled_returns_none(monkeypatch):
    monkeypatch.delenv("MG35_CODEC_NATIVE_ENABLE", raising=False)
    assert _call() is None


def test_wrong_mode_and_a1_pass_raise(monkeypatch):
    monkeypatch.setenv("MG35_CODEC_NATIVE_ENABLE", "1")
    monkeypatch.setenv("MG35_KVCODEC_MODE", "pca_int4")
    with pytest.raises(RuntimeError, match="worldplay_method"):
        _call()
    monkeypatch.setenv("MG35_KVCODEC_MODE", "worldplay_method")
    with pytest.raises(RuntimeError, match="A1"):
        _call(a1_pass=object())


def test_unlisted_layer_returns_none(monkeypatch, tmp_path):
    op = tmp_path / "codec.pt"
    op.write_bytes(b"operator")
    manifest = {"format": "codec_native_manifest_v1", "model": "matrix-game-3.5",
                "codec_operator_sha256": hashlib.sha256(b"operator").hexdigest(),
                "policy": {"recent_native_frames": 1}, "layers": {}}
    mf = tmp_path / "manifest.json"
    mf.write_text(json.dumps(manifest))
    monkeypatch.setenv("MG35_CODEC_NATIVE_ENABLE", "1")
    monkeypatch.setenv("MG35_KVCODEC_MODE", "worldplay_method")
    monkeypatch.setenv("MG35_KVCODEC_PREPACKED_OPERATOR_PATH", str(op))
    monkeypatch.setenv("MG35_CODEC_NATIVE_MANIFEST", str(mf))
    assert _call(layer_idx=3) is None
    # a manifest for another model is refused (CN/core.py:237-239)
    manifest["model"] = "hy-worldplay"
    mf2 = tmp_path / "m2.json"
    mf2.write_text(json.dumps(manifest))
    monkeypatch.setenv("MG35_CODEC_NATIVE_MANIFEST", str(mf2))
    with pytest.raises(ValueError, match="manifest/model"):
        _call(layer_idx=3)


def test_route_matches_reference_formulation():
    cases = 0
    for n in range(0, 7):
        for recent, stride, sink, native in itertools.product(range(0, 4), range(0, 3),
                                                              range(0, 2), (False, True)):
            for chunks in ([], [-1] * n, [(i % 3) - 1 for i in range(n)]):
                for read in (None, 0, 1):
                    tokens = 3 * n
                    r = mg35.route(list(range(10, 10 + n)), chunks, read, tokens, recent,
                                   stride, sink, native)
                    p, lo = route_reference(list(range(n)), chunks, read, tokens, recent,
                                               stride, sink, native)
                    assert torch.equal(r["protect"], p), (n, recent, stride, sink, chunks, read)
                    assert torch.equal(r["low"], lo)
                    assert r["low_count"] == int(lo.sum())
                    cases += 1
    assert cases > 1000


def test_route_rejects_ragged_frames():
    with pytest.raises(ValueError, match="equal-sized frames"):
        mg35.route([0, 1, 2], [], None, 10, 1, 0, 0, False)


def test_visibility_keep():
    # no hole, no chunk ids: everything visible -> None
    assert mg35.visibility_keep(4, 2, 4, [0, 1], None, None) is None
    hole = torch.tensor([True, False])
    keep = mg35.visibility_keep(4, 2, 4, [0, 1], hole, None)
    assert keep.shape == (4, 6) and torch.equal(keep[:, :2], hole[None].expand(4, 2))
    assert bool(keep[:, 2:].all())
    # chunk ids: current frames of chunks -1 (anchor) and 3
    keep = mg35.visibility_keep(4, 2, 4, [0, 1], None, [-1, 3])
    q_ids = torch.tensor([-1, -1, 3, 3])
    k_ids = torch.tensor([-1, -1, 3, 3])
    want = torch.where(q_ids[:, None] < 0, (k_ids < 0)[None].expand(4, 4),
                       (q_ids[:, None] == k_ids[None]) | (k_ids < 0)[None])
    assert torch.equal(keep[:, 2:], want) and bool(keep[:, :2].all())
    with pytest.raises(RuntimeError, match="divisible"):
        mg35.visibility_keep(5, 0, 4, [0, 1], None, [0, 1])


def test_visibility_keep_matches_per_key_rule():
    """visibility_keep against the per-(query, key) statement of MG35:258-283
    over frame counts, chunk-id patterns (anchors, one chunk, mixed) and hole
    masks."""
    g = torch.Generator().manual_seed(3)
    cases = 0
    for F in (1, 2, 3, 4):
        for ids in (None, [-1] * F, [0] * F, [(i % 3) - 1 for i in range(F)],
                    [i for i in range(F)], [-1] + [2] * (F - 1)):
            for M in (0, 3):
                for hole in (None, torch.rand(M, generator=g) > 0.4):
                    if hole is not None and M == 0:
                        continue
                    for qpf, kpf in ((1, 1), (2, 3), (4, 2)):
                        Q, K = qpf * F, kpf * F
                        got = mg35.visibility_keep(Q, M, K, list(range(F)), hole, ids)
                        want = keep_reference(Q, M, K, F, hole, ids)
                        if want is None:
                            assert got is None, (F, ids, M, qpf, kpf)
                        else:
                            assert got is not None and torch.equal(got, want), (F, ids, M, qpf, kpf)
                        cases += 1
    assert cases > 200
