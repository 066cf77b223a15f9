"""Pins of the oracle's INT8 operator storage (oracle.int8_pack /
int8_dequant, _pack_operator MG:108-131, unpack_int8_weight
nanokv_codec_kernels.py:64-82) by checks that do not restate it:

* hand-computed codes and scales (zero rows and the 1e-12 floor, half ties
  to even, the amax element at +-127);
* brute force: every code is the integer in [-127, 127] nearest to w / s
  (ties to even), s = max(amax, 1e-12) / 127 of its group;
* torch's tensor ops of the reference's packer and of its bf16 dequant
  product (the library routines the reference runs).
"""
import numpy as np
import pytest
import torch

import oracle.oracle as orc


def _bf16_bits(x: float) -> int:
    return int(torch.tensor([x], dtype=torch.float32).to(torch.bfloat16).view(torch.int16)[0]) & 0xFFFF


def test_int8_known_answers():
    w = np.array([[127.0, -63.5, 1.0, 0.5, 2.5, -2.5, 126.5, -127.0],
                  [0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = orc.int8_pack(w, group=8)
    # amax 127 -> s = 1: codes are the values rounded half to even
    assert q[0].tolist() == [127, -64, 1, 0, 2, -2, 126, -127]
    assert s[0, 0] == _bf16_bits(1.0)
    # a zero row: s = 1e-12 / 127 (the floor), codes 0
    assert q[1].tolist() == [0] * 8
    assert s[1, 0] == _bf16_bits(np.float32(1e-12) / np.float32(127.0))
    # two groups of 4 scale independently
    q2, s2 = orc.int8_pack(np.array([[1, 2, 3, 4, 100, 50, -25, 0]], np.float32), group=4)
    assert q2[0, :4].tolist() == [32, 64, 95, 127]   # 1 / (4 / 127) = 31.75 -> 32, 2 -> 63.5 -> 64
    assert q2[0, 4:].tolist() == [127, 64, -32, 0]   # 50 / (100 / 127) = 63.5 -> 64 (even)
    assert s2[0].tolist() == [_bf16_bits(4 / 127), _bf16_bits(100 / 127)]


def test_int8_brute_force_nearest_code():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((16, 96)) * np.exp(rng.uniform(-4, 4, (16, 1)))).astype(np.float32)
    w[3, 5] = 0.0
    for group in (96, 32, 8):
        q, _ = orc.int8_pack(w, group)
        g = w.reshape(16, -1, group)
        s = np.maximum(np.abs(g).max(axis=2), np.float32(1e-12)).astype(np.float32) / np.float32(127)
        x = (g / s[:, :, None]).astype(np.float32).reshape(16, -1)
        cand = np.arange(-127, 128)[None, None, :]
        dist = np.abs(x[:, :, None] - cand)
        best = dist.min(axis=2, keepdims=True)
        ties = np.where(dist == best, cand, 1000)
        even = np.where((ties % 2 == 0) & (ties != 1000), ties, 1000).min(axis=2)
        nearest = np.where(even != 1000, even, ties.min(axis=2))
        assert np.array_equal(q.astype(np.int64), nearest), group


@pytest.mark.parametrize("group", [0, 64])
def test_int8_pack_matches_torch_ops(group):
    g = torch.Generator().manual_seed(group + 1)
    weight = torch.randn(40, 256, generator=g) * 0.05
    q, s = orc.int8_pack(weight.numpy(), group)
    gs = group or 256
    grouped = weight.reshape(40, -1, gs)
    scale = grouped.abs().amax(dim=2).clamp_min(1e-12) / 127.0
    ref_q = (grouped / scale[:, :, None]).round().clamp(-127, 127).to(torch.int8).reshape(40, 256)
    ref_s = scale.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(q, ref_q.numpy())
    assert np.array_equal(s, ref_s)


def test_int8_dequant_matches_torch_bf16_product():
    g = torch.Generator().manual_seed(7)
    q = torch.randint(-127, 128, (24, 96), generator=g, dtype=torch.int8)
    scale = (torch.rand(24, 3, generator=g) * 0.1).to(torch.bfloat16)
    got = orc.int8_dequant(q.numpy(), scale.view(torch.int16).numpy().view(np.uint16), 32)
    ref = (q.reshape(24, 3, 32).to(torch.bfloat16) * scale[:, :, None]).reshape(24, 96)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
