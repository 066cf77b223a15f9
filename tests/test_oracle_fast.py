"""Pins of the oracle's NanoKV-Fast restatement (oracle.fast_attend,
reader_tables, reader_read) by invariants that do not restate its formula:

* identity readers (q_reduce = k_affine = v_affine = lift = I, k_read /
  v_read = the head's decoder rows) make the low partition the full decode,
  so for ANY split of the history into protected / low rows the hybrid
  result equals plain decode-then-attend over all rows (CN/core.py:258-262);
* all rows protected leaves only the native partition;
* projected tables / biases against an explicit torch computation.
"""
import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import synth
from tests._helpers import Scenario, max_abs_cos, oracle_groups, u16


def _identity_payload(sc):
    return synth.make_readers(sc.shape, sc.layer, full_heads=tuple(range(sc.H)))


@pytest.mark.parametrize("split", ["recent", "anchors", "none", "all"])
def test_identity_readers_equal_full_decode(split):
    sc = Scenario(H=2, D=32, N=90, Q=12, Nc=10, rK=64, rV=64, G=32, C=6, with_mean=True)
    N = sc.N
    if split == "recent":
        prot = np.arange(60, N)
    elif split == "anchors":
        prot = np.array([0, 1, 2, 30, 31, 50, 88, 89])
    elif split == "none":
        prot = np.array([], np.int64)
    else:
        prot = np.arange(N)
    low = np.setdiff1d(np.arange(N), prot)
    groups = oracle_groups(_identity_payload(sc))
    for g in groups:  # identity readers carry no projection matrices
        assert g["q_reduce"] is None and g["k_affine"] is None and g["v_affine"] is None
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    out, lse = orc.fast_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val, prot,
                               low, groups, sc.scale, D=sc.D)
    ref, ref_lse = sc.reference(0)
    diff, cos = max_abs_cos(out, ref)
    # the hybrid result is rounded to bf16 twice (partition outputs, merge)
    assert diff < 2e-2 and cos > 0.9999, (split, diff, cos)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-4)


def test_reader_tables_against_torch():
    g = torch.Generator().manual_seed(3)
    C, HD, D, d = 5, 8, 4, 3
    centers = torch.randn(C, HD, generator=g).to(torch.bfloat16)
    mean = torch.randn(HD, generator=g)
    aff = torch.randn(D, d, generator=g).to(torch.bfloat16)
    h = 1
    table, bias = orc.reader_tables(u16(centers), mean.numpy(), h, u16(aff), D=D)
    ref_t = (centers[:, h * D:(h + 1) * D].double() @ aff.double()).float().to(torch.bfloat16)
    assert np.array_equal(table, u16(ref_t))
    ref_b = (mean[h * D:(h + 1) * D].to(torch.bfloat16).double() @ aff.double()).float()
    np.testing.assert_array_equal(bias, ref_b.to(torch.bfloat16).float().numpy())
    # identity affine: the head's center columns and bf16(mean)
    table, bias = orc.reader_tables(u16(centers), mean.numpy(), h, None, D=D)
    assert np.array_equal(table, u16(centers[:, h * D:(h + 1) * D].contiguous()))
    np.testing.assert_array_equal(bias, mean[h * D:(h + 1) * D].to(torch.bfloat16).float().numpy())


def test_reader_read_against_torch_linear():
    # F.linear(latent, read, bias) rounded to bf16, plus the table row (CN:188-200)
    sc = Scenario(H=2, D=32, N=20, Q=1, Nc=0, rK=64, rV=64, G=32, C=4)
    key = sc.hist[0]["k"]
    g = torch.Generator().manual_seed(5)
    read = torch.randn(8, 64, generator=g).to(torch.bfloat16)
    table = torch.randn(4, 8, generator=g).to(torch.bfloat16)
    bias = torch.randn(8, generator=g).to(torch.bfloat16).float()
    rows = np.array([3, 0, 19, 7])
    got = orc.bf16_to_f32(orc.reader_read(key, rows, u16(read), u16(table), bias.numpy()))
    latent = torch.from_numpy(orc.bf16_to_f32(orc.unpack_latent(
        key["packed"], key["scales"], 64, 32, "fp16", rows)))
    lin = (latent.double() @ read.double().T + bias.double()).float().to(torch.bfloat16)
    ids = torch.from_numpy(np.asarray(key["ids"], np.int64)[rows])
    ref = (lin.float() + table[ids].float()).to(torch.bfloat16).float()
    np.testing.assert_array_equal(got, ref.numpy())


def test_lift_applies_to_the_low_output():
    """With no native rows the hybrid result is the low partition alone; a lift
    L then gives bf16(out_without_lift . L) up to the bf16 rounding of the
    unlifted output (a transposed or misplaced lift fails this)."""
    sc = Scenario(H=2, D=32, N=70, Q=9, Nc=0, rK=64, rV=64, G=32, C=5, with_mean=True)
    payload = _identity_payload(sc)
    groups = oracle_groups(payload)
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    low = np.arange(sc.N)
    none = np.array([], np.int64)
    base, _ = orc.fast_attend(u16(sc.q[0]), None, None, key, val, none, low, groups, sc.scale, D=sc.D)
    g = torch.Generator().manual_seed(4)
    L = (torch.randn(2, 32, 32, generator=g) / 32 ** 0.5).to(torch.bfloat16)
    lifted_groups = [dict(gr, lift=u16(L[[h for h in gr["heads"]]])) for gr in groups]
    out, _ = orc.fast_attend(u16(sc.q[0]), None, None, key, val, none, low, lifted_groups,
                             sc.scale, D=sc.D)
    for h in range(2):
        ref = base[:, h] @ L[h].float().numpy()
        np.testing.assert_allclose(out[:, h], ref, rtol=2e-2, atol=2e-2)
        # not the transpose
        assert np.abs(out[:, h] - base[:, h] @ L[h].float().numpy().T).max() > 5e-2


def test_identity_readers_with_camera_equal_full_decode():
    """With identity readers (block sub-frames j % 4) the camera path of
    fast_attend is the full decode with P^-1 on the history keys / values and
    P on the output (CN/mg35.py:253-257, 310-347), for a recent-frames split."""
    sc = Scenario(H=2, D=128, N=60, Q=12, Nc=10, rK=64, rV=64, G=32, C=6)
    g = torch.Generator().manual_seed(9)
    kinv = (torch.eye(4).expand(sc.N, 4, 4, 4) + 0.2 * torch.randn(sc.N, 4, 4, 4, generator=g)).numpy()
    qt = (torch.eye(4).expand(sc.Q, 4, 4, 4) + 0.2 * torch.randn(sc.Q, 4, 4, 4, generator=g)).numpy()
    p = (torch.eye(4).expand(sc.Q, 4, 4, 4) + 0.2 * torch.randn(sc.Q, 4, 4, 4, generator=g)).numpy()
    prot, low = np.arange(40, sc.N), np.arange(40)
    groups = oracle_groups(_identity_payload(sc))
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    # the native query is the transformed one; the readers start from q_pre
    q_native = orc.camera_apply(u16(sc.q[0]), qt, "full")
    out, lse = orc.fast_attend(q_native, u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val, prot,
                               low, groups, sc.scale, D=sc.D, q_pre_bf16=u16(sc.q[0]),
                               key_cam=kinv, q_cam=qt, out_cam=p)
    ref, ref_lse = orc.decode_attend(q_native, u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val,
                                     sc.scale, D=sc.D, key_cam=(kinv, "full"))
    ref = orc.bf16_to_f32(orc.camera_apply(orc.f32_to_bf16(ref.astype(np.float32)), p, "full"))
    diff, cos = max_abs_cos(out, ref)
    assert diff < 3e-2 and cos > 0.9999, (diff, cos)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-4)


def test_identity_readers_with_mask_equal_full_decode():
    """A current-key mask reaches only the native partition: with identity
    readers fast_attend equals decode_attend under the same mask."""
    sc = Scenario(H=2, D=32, N=50, Q=14, Nc=12, rK=64, rV=64, G=32, C=5)
    mask = np.random.default_rng(4).random((sc.Q, sc.Nc)) > 0.4
    prot, low = np.arange(30, sc.N), np.arange(30)
    groups = oracle_groups(_identity_payload(sc))
    key, val = sc.hist[0]["k"], sc.hist[0]["v"]
    out, lse = orc.fast_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val, prot,
                               low, groups, sc.scale, D=sc.D, cur_mask=mask)
    ref, ref_lse = orc.decode_attend(u16(sc.q[0]), u16(sc.k_cur[0]), u16(sc.v_cur[0]), key, val,
                                     sc.scale, D=sc.D, cur_mask=mask)
    diff, cos = max_abs_cos(out, ref)
    assert diff < 2e-2 and cos > 0.9999, (diff, cos)
    np.testing.assert_allclose(lse, ref_lse, atol=1e-4)
