"""Host-side logic of the codec API (payload dicts, segment lists, policy),
exercised on CPU tensors without any kernel launch."""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import codec_native, nanokv_codec as nc


def _fake_payload(kind, S, r=64, hd=128, B=1, group=32):
    return {"codec": nc.CODEC, "kind": kind, "layer": 0, "shape": (B, S, hd),
            "latent_shape": (B, S, r), "latent_numel": B * S * r,
            "packed_codes": torch.zeros(B * S * r // 2, dtype=torch.uint8),
            "scale": torch.ones(B, S, r // group, dtype=torch.float16),
            "centers": torch.zeros(B, 4, hd, dtype=torch.bfloat16),
            "ids": torch.zeros(B, S, dtype=torch.uint8), "semantic": True,
            "source_dtype": "bfloat16", "scale_group": group, "scale_dtype": "fp16"}


def test_concat_and_shapes():
    a, b = _fake_payload("k", 10), _fake_payload("k", 7)
    assert nc.concat_values(None, a) is a and nc.concat_values(a, None) is a
    seg = nc.concat_values(a, b)
    assert seg["codec"] == nc.SEGMENTS and len(seg["segments"]) == 2
    seg3 = nc.concat_values(seg, _fake_payload("k", 3))
    assert len(seg3["segments"]) == 3
    assert nc.value_shape(seg3) == (1, 20, 128)
    assert nc.value_shape(None) is None
    assert nc.value_shape(torch.zeros(1, 5, 8)) == (1, 5, 8)
    with pytest.raises(RuntimeError):
        nc.concat_values(a, torch.zeros(1))


def test_payload_bytes_counts_resident_tensors():
    p = _fake_payload("k", 10)
    expect = 10 * 32 + 10 * 2 * 2 + 4 * 128 * 2 + 10
    assert nc.payload_bytes(p) == expect
    assert nc.payload_bytes(nc.concat_values(p, p)) == 2 * expect


def test_pairs_validation():
    k, v = _fake_payload("k", 10), _fake_payload("v", 10)
    assert len(nc._pairs(k, v)) == 1
    with pytest.raises(RuntimeError):
        nc._pairs(k, _fake_payload("k", 10))
    with pytest.raises(ValueError):
        nc._pairs(nc.concat_values(k, k), v)


def test_select_value_raw_tensor():
    t = torch.arange(2 * 6 * 4).reshape(2, 6, 4)
    out = nc.select_value(t, torch.tensor([1, 4]), kind="k", layer=0, dtype=torch.float32,
                          device="cpu")
    assert torch.equal(out, t[:, [1, 4]])


def test_select_value_keeps_whole_segments():
    a, b = _fake_payload("k", 4), _fake_payload("k", 3)
    seg = nc.concat_values(a, b)
    assert nc.select_value(seg, torch.arange(4, 7), kind="k", layer=0, dtype=torch.bfloat16,
                           device="cpu") is b
    both = nc.select_value(seg, torch.arange(0, 7), kind="k", layer=0, dtype=torch.bfloat16,
                           device="cpu")
    assert both["segments"] == [a, b]
    with pytest.raises(RuntimeError):
        nc.select_value(seg, torch.tensor([5, 1]), kind="k", layer=0, dtype=torch.bfloat16,
                        device="cpu")


def test_register_operator_shape_checks():
    with pytest.raises(ValueError):
        nc.register_operator("k", 0, encoder=torch.zeros(64, 128), decoder=torch.zeros(64, 128))
    with pytest.raises(ValueError):
        nc.register_operator("x", 0, encoder=torch.zeros(64, 128), decoder=torch.zeros(128, 64))
    nc.register_operator("k", 99, encoder=torch.zeros(64, 128), decoder=torch.zeros(128, 64))
    assert nc._OPERATORS[("k", 99)]["encoder"].dtype == torch.bfloat16
    with pytest.raises(RuntimeError):
        nc._operator("v", 98, torch.device("cpu"))


def test_env_settings(monkeypatch):
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "32")
    monkeypatch.setenv("NANOKV_SCALE_DTYPE", "fp16")
    assert nc._scale_group(384) == 32 and nc._scale_dtype() == torch.float16
    monkeypatch.setenv("NANOKV_SCALE_GROUP", "0")
    assert nc._scale_group(384) == 384
    monkeypatch.setenv("MG35_KVCODEC_TARGET", "bogus")
    with pytest.raises(ValueError):
        nc._target_enabled("k")


def test_protected_tokens_matches_oracle_policy():
    for count in range(0, 9):
        for recent in range(0, 4):
            for stride in range(0, 4):
                for sink in range(0, 3):
                    frames = torch.arange(count).repeat_interleave(3)
                    got = codec_native.protected_tokens(frames, recent, stride, sink)
                    ref = np.repeat(orc.protected_frames(count, recent, stride, sink), 3)
                    assert got.tolist() == ref.tolist()
    # repeated frame ids form one run (CN:142-145)
    frames = torch.tensor([5, 5, 7, 7, 5, 5])
    assert codec_native.protected_tokens(frames, 1, 0).tolist() == [False] * 4 + [True] * 2


def test_codec_history_attention_refuses_short_camera_frames():
    """The camera's frames must cover the cached rows exactly (complete
    equal-sized frames, as mg35.py _expand_frames and camera_kernel.py:64
    require); refused before any device work."""
    import torch
    from nanokv_amd import codec_native, nanokv_codec, ops
    payload = {"codec": nanokv_codec.CODEC, "kind": "k", "layer": 0, "shape": (1, 120, 256)}
    cam = ops.Camera(torch.zeros(1, 2, 4, 4, 4), torch.tensor([0, 1], dtype=torch.int32), 50)
    q = torch.zeros(1, 2, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="frames must cover exactly"):
        codec_native.codec_history_attention(q, payload, payload, camera=cam)


def test_history_codecs_cache_releases_dropped_payloads():
    """history_codecs remembers the segment table of a paired segment list, but
    only while the payloads live: dropping them (as select_value or a cache
    reset does) removes the entry, and the codes' memory is freed."""
    import gc
    import weakref

    nc.register_operator("k", 0, encoder=torch.zeros(64, 128), decoder=torch.zeros(128, 64))
    nc.register_operator("v", 0, encoder=torch.zeros(64, 128), decoder=torch.zeros(128, 64))
    nc._HISTORY_TABLES.clear()
    k = nc.concat_values(_fake_payload("k", 10), _fake_payload("k", 6))
    v = nc.concat_values(_fake_payload("v", 10), _fake_payload("v", 6))
    first = nc.history_codecs(k, v, torch.device("cpu"))
    assert len(nc._HISTORY_TABLES) == 1
    again = nc.history_codecs(k, v, torch.device("cpu"))
    assert again[0] is first[0] and again[1] is first[1]     # the remembered tables
    codes = weakref.ref(k["segments"][0]["packed_codes"])
    storage = weakref.ref(k["segments"][0]["packed_codes"].untyped_storage())
    del first, again, k, v
    gc.collect()
    assert len(nc._HISTORY_TABLES) == 0
    assert codes() is None
    # a fresh list of new payloads builds a new entry
    k2 = nc.concat_values(_fake_payload("k", 4), _fake_payload("k", 4))
    v2 = nc.concat_values(_fake_payload("v", 4), _fake_payload("v", 4))
    nc.history_codecs(k2, v2, torch.device("cpu"))
    assert len(nc._HISTORY_TABLES) == 1
    del storage
