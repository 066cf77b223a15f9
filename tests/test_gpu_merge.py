"""GPU parity of the HY and LingBot partition merges against the oracle:
nkv_lift_lse_combine (HY's Main/PRoPE value lift fused with the LSE merge),
lse_combine_split (already lifted halves) and nkv_finish (LingBot's merge
with the value-mean correction and head scatter).  The GPU sums each lift in
fp32 where the oracle uses fp64, so outputs agree to one bf16 rounding: at
most one bf16 unit in the last place of the reference value (2^-7 relative)
plus 1e-6 absolute."""
import ctypes

import numpy as np
import pytest
import torch

import oracle.oracle as orc
from nanokv_amd import _lib, ops
from tests._helpers import u16

pytestmark = pytest.mark.gpu


def _f(t):
    return orc.bf16_to_f32(u16(t)).astype(np.float64) if t.dtype == torch.bfloat16 \
        else t.detach().cpu().double().numpy()


def _close_bf16(got, ref):
    got = orc.bf16_to_f32(u16(got)).astype(np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = np.abs(ref) * 2.0 ** -7 + 1e-6
    assert np.all(err <= bound), float((err - bound).max())


def _inputs(dev, B, H, Q, Dl, seed, strided=False):
    g = torch.Generator().manual_seed(seed)
    native = torch.randn(2 * B, H, Q, 128, generator=g).to(torch.bfloat16)
    if strided:  # [2B, Q, H, 128] storage seen as [2B, H, Q, 128]
        native = native.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    low = torch.randn(2 * B, H, Q, Dl, generator=g).to(torch.bfloat16)
    lift = (torch.randn(H, Dl, 128, generator=g) / Dl ** 0.5).to(torch.bfloat16)
    mix = (torch.randn(H, Dl // 4, 32, generator=g) / 4).to(torch.bfloat16)
    nl = torch.randn(2 * B, H, Q, generator=g) * 3
    hl = torch.randn(2 * B, H, Q, generator=g) * 3
    return [t.to(dev) for t in (native, nl, low, lift, mix, hl)]


@pytest.mark.parametrize("Dl", [32, 64, 96])
@pytest.mark.parametrize("B,H,Q,strided", [(1, 2, 64, False), (2, 3, 97, True)])
def test_lift_lse_combine(dev, Dl, B, H, Q, strided):
    native, nl, low, lift, mix, hl = _inputs(dev, B, H, Q, Dl, seed=Dl + Q, strided=strided)
    out = ops.lift_lse_combine(native, nl, low, lift, mix, hl)
    assert out.is_contiguous() and out.shape == native.shape
    ref = orc.lift_lse_combine(_f(native), _f(nl), _f(low), _f(lift), _f(mix), _f(hl))
    _close_bf16(out, ref)


def test_lift_lse_combine_empty_partitions(dev):
    native, nl, low, lift, mix, hl = _inputs(dev, 1, 2, 40, 64, seed=5)
    nl[:, :, :10] = -float("inf")     # no native keys: the lifted history
    hl[:, :, 10:20] = -float("inf")   # no history keys: the native output
    out = ops.lift_lse_combine(native, nl, low, lift, mix, hl)
    ref = orc.lift_lse_combine(_f(native), _f(nl), _f(low), _f(lift), _f(mix), _f(hl))
    _close_bf16(out, ref)
    assert torch.equal(out[:, :, 10:20].view(torch.int16), native[:, :, 10:20].view(torch.int16))


def test_lift_lse_combine_rejections(dev):
    native, nl, low, lift, mix, hl = _inputs(dev, 1, 2, 8, 64, seed=6)
    with pytest.raises(ValueError, match="D32/D64/D96"):
        ops.lift_lse_combine(native, nl, low[..., :48], lift[:, :48], mix[:, :12], hl)
    with pytest.raises(ValueError, match="PRoPE lift"):
        ops.lift_lse_combine(native, nl, low, lift, mix[:, :8], hl)
    # the C ABI refuses an unsupported width itself
    a = _lib.NkvLiftCombineArgs()
    a.B, a.H, a.Q, a.low_dim = 1, 2, 8, 48
    code = _lib.lib().nkv_lift_lse_combine(None, ctypes.byref(a))
    assert code == _lib.NKV_ERR_UNSUPPORTED


def test_lse_combine_split(dev):
    native, nl, _, _, _, hl = _inputs(dev, 2, 3, 50, 64, seed=7)
    g = torch.Generator().manual_seed(8)
    main = torch.randn(2, 3, 50, 128, generator=g).to(torch.bfloat16).to(dev)
    prope = torch.randn(2, 3, 50, 128, generator=g).to(torch.bfloat16).to(dev)
    out = ops.lse_combine_split(native, nl, main, prope, hl)
    hist = np.concatenate([_f(main), _f(prope)], 0)
    ref, _ = orc.merge(_f(native), _f(nl), hist, _f(hl))
    _close_bf16(out, ref)


@pytest.mark.parametrize("correct", [False, True])
def test_finish(dev, correct):
    g = torch.Generator().manual_seed(9 + correct)
    B, Hn, S, D = 2, 5, 70, 128
    heads = torch.tensor([3, 0, 4])
    native = torch.randn(B, Hn, S, D, generator=g).to(torch.bfloat16).to(dev)
    nlse = (torch.randn(B, Hn, S, generator=g) * 2).to(dev)
    # a strided group output: [B, S, h, D] storage
    lifted = torch.randn(B, S, 3, D, generator=g).to(torch.bfloat16).to(dev).permute(0, 2, 1, 3)
    llse = (torch.randn(B, 3, S, generator=g) * 2).to(dev)
    llse[0, 1, :5] = -float("inf")
    result = torch.randn(B, Hn, S, D, generator=g).to(torch.bfloat16).to(dev)
    before = result.clone()
    mean = proj = None
    if correct:
        mean = torch.randn(B, Hn, 1, D, generator=g).to(dev)
        proj = torch.randn(B, 3, 1, D, generator=g).to(dev)
    got = ops.finish(native, nlse, lifted, llse, heads.to(dev), result, mean, proj)
    assert got is result
    ref = orc.finish(_f(native), _f(nlse), _f(lifted), _f(llse), heads.numpy(), _f(before),
                     None if mean is None else _f(mean), None if proj is None else _f(proj))
    _close_bf16(result[:, heads.tolist()], ref[:, heads.numpy()])
    untouched = [1, 2]
    assert torch.equal(result[:, untouched].view(torch.int16), before[:, untouched].view(torch.int16))


def test_finish_in_place_and_bad_head(dev):
    """result may be native itself; a head index outside the native heads
    writes nothing."""
    g = torch.Generator().manual_seed(11)
    native = torch.randn(1, 3, 20, 64, generator=g).to(torch.bfloat16).to(dev)
    nlse = torch.randn(1, 3, 20, generator=g).to(dev)
    lifted = torch.randn(1, 2, 20, 64, generator=g).to(torch.bfloat16).to(dev)
    llse = torch.randn(1, 2, 20, generator=g).to(dev)
    ref = orc.finish(_f(native), _f(nlse), _f(lifted), _f(llse), [2, 0], _f(native))
    ops.finish(native, nlse, lifted, llse, torch.tensor([2, 0], device=dev), native)
    _close_bf16(native, ref)
    before = native.clone()
    ops.finish(native, nlse, lifted, llse, torch.tensor([7, -1], device=dev), native)
    assert torch.equal(native.view(torch.int16), before.view(torch.int16))
