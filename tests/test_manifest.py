"""Manifest-bound reader loading (codec_native.get_layer, CN/core.py:229-275)
on the CPU: the manifest must name the model and carry the SHA-256 of the
deployed codec operator file; reader checkpoints must match their recorded
SHA-256; uncalibrated readers are refused unless explicitly allowed."""
import hashlib
import json

import pytest
import torch

from nanokv_amd import codec_native, synth


def _sha(path):
    return hashlib.sha256(path.read_bytes()).hexdigest()


@pytest.fixture
def bank(tmp_path, monkeypatch):
    sh = synth.Shape("m", H=4, D=128, N=0, Q=0, Nc=0, rK=64, rV=64, G=32, C=4)
    layer = synth.make_layer(sh, seed=1)
    payload = synth.make_readers(sh, layer, full_heads=(0,), d=32)
    torch.save(payload, tmp_path / "reader_07.pt")
    op = tmp_path / "codec.pt"
    op.write_bytes(b"frozen operator bytes")
    manifest = {"format": "codec_native_manifest_v1", "model": "mg35",
                "codec_operator_sha256": _sha(op),
                "layers": {"0:7": {"path": "reader_07.pt", "sha256": _sha(tmp_path / "reader_07.pt"),
                                   "calibrated": True},
                           "0:8": {"path": "reader_07.pt", "sha256": _sha(tmp_path / "reader_07.pt"),
                                   "calibrated": False}}}
    (tmp_path / "manifest.json").write_text(json.dumps(manifest))
    monkeypatch.setenv("MG35_CODEC_NATIVE_ENABLE", "1")
    monkeypatch.setenv("MG35_CODEC_NATIVE_MANIFEST", str(tmp_path / "manifest.json"))
    codec_native._READER_BANKS.clear()
    return tmp_path, op, manifest


def _get(op, layer=7, heads=4, model="mg35"):
    return codec_native.get_layer("MG35_CODEC_NATIVE", model, layer, device="cpu", heads=heads,
                                  native_dim=128, operator_path=str(op))


def test_loads_bound_reader(bank):
    _, op, manifest = bank
    reader, m = _get(op)
    assert isinstance(reader, codec_native.ReaderLayer) and m == manifest
    assert [len(g.heads) for g in reader.groups] == [1, 3]
    assert _get(op, layer=3) == (None, manifest)  # a layer the manifest does not list


def test_refusals(bank, monkeypatch):
    tmp, op, _ = bank
    with pytest.raises(RuntimeError, match="initialization-only"):
        _get(op, layer=8)
    monkeypatch.setenv("MG35_CODEC_NATIVE_ALLOW_UNCALIBRATED", "1")
    assert _get(op, layer=8)[0] is not None
    with pytest.raises(ValueError, match="layout mismatch"):
        _get(op, heads=8)
    codec_native._READER_BANKS.clear()
    with pytest.raises(ValueError, match="manifest/model"):
        _get(op, model="hy")
    other = tmp / "other.pt"
    other.write_bytes(b"a different operator")
    with pytest.raises(ValueError, match="not bound"):
        _get(other)
    codec_native._READER_BANKS.clear()
    torch.save({"tampered": torch.zeros(1)}, tmp / "reader_07.pt")
    with pytest.raises(ValueError, match="checksum"):
        _get(op)
    monkeypatch.setenv("MG35_CODEC_NATIVE_ENABLE", "0")
    assert _get(op) == (None, None)
