"""Refusals of preload_operator_weights on the CPU (MG:56-66, 186-212,
257-279): a prepacked operator file must record this runtime's center
storage and rung, and each entry the deployment's artifact directories
(unless NANOKV_PORTABLE_CODEC_SHA256 vouches for the file); every refusal
happens before any operator reaches a device."""
import hashlib

import pytest
import torch

from nanokv_amd import nanokv_codec as nc


def _write(tmp_path, **over):
    entry = {"basis_dir": str(tmp_path / "basis"), "decoder_dir": str(tmp_path / "dec_k"),
             "qat_dir": "", "mean": torch.zeros(4),
             "encoder": {"qweight": torch.zeros(2, 4, dtype=torch.int8),
                         "scale": torch.ones(2, 1, dtype=torch.bfloat16), "group_size": 4},
             "decoder": {"qweight": torch.zeros(4, 2, dtype=torch.int8),
                         "scale": torch.ones(4, 1, dtype=torch.bfloat16), "group_size": 2}}
    payload = {"format": nc.PREPACKED_FORMAT, "rung": "full", "center_storage": "bf16",
               "center_block_size": 64, "entries": {"k:03": entry}}
    payload.update(over)
    path = tmp_path / "codec.pt"
    torch.save(payload, path)
    return path


@pytest.fixture
def env(tmp_path, monkeypatch):
    for name in ("basis", "dec_k", "qat_v"):
        (tmp_path / name).mkdir()
    monkeypatch.setenv("MG35_KVCODEC_BASIS_DIR", str(tmp_path / "basis"))
    monkeypatch.setenv("MG35_KVCODEC_DECODER_DIR_K", str(tmp_path / "dec_k"))
    monkeypatch.setenv("MG35_KVCODEC_DECODER_DIR_V", str(tmp_path / "qat_v"))
    for k in ("MG35_WORLDPLAY_RUNG", "MG35_KVCODEC_CENTER_STORAGE", "NANOKV_PORTABLE_CODEC_SHA256",
              "MG35_KVCODEC_CENTER_BLOCK_SIZE"):
        monkeypatch.delenv(k, raising=False)
    return tmp_path


def _load(path):
    # the checks pass when loading reaches the device step, which needs a GPU
    nc.preload_operator_weights(torch.device("cpu"), str(path))


def test_accepted_file_reaches_the_device_step(env):
    with pytest.raises(ValueError, match="GPU tensors"):
        _load(_write(env))


def test_center_provenance_mismatch(env, monkeypatch):
    with pytest.raises(RuntimeError, match="center provenance mismatch"):
        _load(_write(env, center_storage="int8_block"))
    with pytest.raises(RuntimeError, match="center provenance mismatch"):
        _load(_write(env, center_block_size=32))
    # the pca rung has no centers: provenance none/0
    monkeypatch.setenv("MG35_WORLDPLAY_RUNG", "pca")
    with pytest.raises(RuntimeError, match="center provenance mismatch"):
        _load(_write(env, rung="pca"))
    entry_pca = _write(env, rung="pca", center_storage="none", center_block_size=0)
    with pytest.raises(RuntimeError, match="K operator provenance"):
        _load(entry_pca)  # pca expects no decoder dir for K


def test_rung_mismatch(env, monkeypatch):
    monkeypatch.setenv("MG35_WORLDPLAY_RUNG", "c64")
    with pytest.raises(RuntimeError, match="operator rung=full runtime=c64"):
        _load(_write(env))
    monkeypatch.setenv("MG35_WORLDPLAY_RUNG", "bogus")
    with pytest.raises(ValueError, match="MG35_WORLDPLAY_RUNG"):
        _load(_write(env))


def test_artifact_directory_mismatch_and_portable_codec(env, monkeypatch):
    other = env / "elsewhere"
    other.mkdir()
    monkeypatch.setenv("MG35_KVCODEC_BASIS_DIR", str(other))
    path = _write(env)
    with pytest.raises(RuntimeError, match="K operator provenance mismatch L3"):
        _load(path)
    # a portable codec vouched for by its SHA-256 may carry other paths
    monkeypatch.setenv("NANOKV_PORTABLE_CODEC_SHA256",
                       hashlib.sha256(path.read_bytes()).hexdigest())
    with pytest.raises(ValueError, match="GPU tensors"):
        _load(path)
    monkeypatch.setenv("NANOKV_PORTABLE_CODEC_SHA256", "0" * 64)
    with pytest.raises(ValueError, match="checksum mismatch"):
        _load(path)
