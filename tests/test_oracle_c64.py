"""Pins of the oracle's C64 fit (oracle.c64_fit, semantic_residual
MG:301-330) by checks that do not restate it:

* the labels of the last round against exact rational distances
  (fractions.Fraction) to the centers that round started from;
* the centers against the closed-form mean of each cluster's rows;
* zero rounds leave the drawn rows and zero labels;
* the reference's own torch loop on the CPU (fp32 bmm distances, one-hot
  mean update) gives the same labels and the centers to fp32 rounding.
"""
from fractions import Fraction

import numpy as np
import torch

import oracle.oracle as orc


def _data(B, S, HD, seed):
    rng = np.random.default_rng(seed)
    base = rng.standard_normal((5, HD)).astype(np.float32) * 3
    x = base[rng.integers(0, 5, (B, S))] + rng.standard_normal((B, S, HD)).astype(np.float32)
    return x.astype(np.float32)


def test_zero_rounds_keep_the_drawn_rows():
    x = _data(2, 30, 8, 0)
    init = [7, 0, 29, 3]
    c, lab = orc.c64_fit(x, init, iterations=0)
    assert np.array_equal(c, x[:, init]) and not lab.any()


def test_labels_exact_and_centers_are_cluster_means():
    x = _data(1, 40, 6, 1)
    init = [3, 17, 25]
    c1, _ = orc.c64_fit(x, init, iterations=1)      # centers the second round starts from
    c2, lab = orc.c64_fit(x, init, iterations=2)
    for i in range(40):
        exact = [sum((Fraction(float(a)) - Fraction(float(b))) ** 2 for a, b in zip(x[0, i], c1[0, k]))
                 for k in range(3)]
        best = min(exact)
        assert lab[0, i] == exact.index(best)
    for k in range(3):
        rows = x[0][lab[0] == k]
        if len(rows):
            mean = rows.astype(np.float64).mean(0)
            np.testing.assert_allclose(c2[0, k], mean, rtol=2 ** -22, atol=1e-7)
        else:
            assert np.array_equal(c2[0, k], c1[0, k])


def test_matches_reference_torch_loop():
    x = _data(2, 300, 64, 2)
    C, iters = 16, 2
    draw = torch.Generator(device="cpu").manual_seed(20260804 + 5)
    init = torch.randperm(300, generator=draw)[:C]
    c, lab = orc.c64_fit(x, init.numpy(), iters)
    # the reference's loop, CPU fp32 (MG:301-330)
    rows = torch.from_numpy(x)
    centers = rows.index_select(1, init).clone()
    row_norm = rows.square().sum(-1, keepdim=True)
    for _ in range(iters):
        dist = row_norm + centers.square().sum(-1).unsqueeze(1) - 2.0 * torch.bmm(
            rows, centers.transpose(1, 2))
        labels = dist.argmin(-1)
        onehot = torch.nn.functional.one_hot(labels, num_classes=C).transpose(1, 2).float()
        counts = onehot.sum(-1)
        updated = torch.bmm(onehot, rows) / counts.clamp_min(1.0).unsqueeze(-1)
        centers = torch.where((counts > 0).unsqueeze(-1), updated, centers)
    assert np.array_equal(lab, labels.numpy())
    np.testing.assert_allclose(c, centers.numpy(), rtol=1e-5, atol=1e-5)
