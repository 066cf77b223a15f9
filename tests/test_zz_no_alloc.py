"""nkv_attend_static, the allocation-free nkv_attend, through the C ABI: the
same results as nkv_attend (bit for bit: the same kernels read the same
inputs) on two calls in a row, the second smaller; a call that needs more
scratch than the static array holds is refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from nanokv_amd import _lib, ops
from tests._helpers import Scenario, max_abs_cos

pytestmark = pytest.mark.gpu


def _both(sc, dev, **kw):
    key, value = sc.codecs(dev)
    q, kc, vc = sc.q.to(dev), sc.k_cur.to(dev), sc.v_cur.to(dev)
    ref_out, ref_lse = ops.attend(q, kc, vc, key, value, **kw)
    out = torch.empty_like(ref_out)
    lse = torch.empty_like(ref_lse)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(dev)
    got_out, got_lse = ops.attend_static(q, kc, vc, key, value, out=out, lse=lse, **kw)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated(dev) == before  # nothing allocated for the call
    assert got_out is out and got_lse is lse
    return ref_out, ref_lse, out, lse


def test_static_scratch_matches_nkv_attend_twice(dev):
    # 1: key-chunk schedule (staged at 10 query blocks), tiles and partials in the static scratch
    big = Scenario(H=2, N=600, Q=300, Nc=64, rK=384, rV=256, G=32, C=16, seed=1)
    need = ops.attend_workspace_size(big.q, big.N, big.Nc, *big.codecs(dev))
    assert 0 < need <= _lib.NKV_STATIC_SCRATCH_BYTES
    r_out, r_lse, out, lse = _both(big, dev)
    assert torch.equal(out.view(torch.int16), r_out.view(torch.int16))
    assert torch.equal(lse, r_lse)
    ref, _ = big.reference(0)
    diff, cos = max_abs_cos(out[0].float().cpu().numpy(), ref)
    assert diff <= 2e-2 and cos >= 0.9995, (diff, cos)
    # 2: a smaller call right after (query tiles with split-K partials); the
    # scratch still holds the first call's partials and is overwritten
    small = Scenario(H=2, N=200, Q=90, Nc=30, rK=128, rV=128, G=32, C=8, seed=2)
    r_out, r_lse, out, lse = _both(small, dev, schedule="query_tiles")
    assert torch.equal(out.view(torch.int16), r_out.view(torch.int16))
    assert torch.equal(lse, r_lse)
    r_out, r_lse, out, lse = _both(small, dev, schedule="key_chunks")
    assert torch.equal(out.view(torch.int16), r_out.view(torch.int16))


def test_static_scratch_refuses_oversize_calls(dev):
    """A config-1-sized key-chunk call (206 MB of tiles and partials) is refused with
    NKV_ERR_WORKSPACE before anything is launched.  The size query (host
    arithmetic) already exceeds the static array; every pointer of the call is a
    real device buffer of its declared shape, so no launch could read outside
    memory even if the refusal came later."""
    B, H, D, Q, N, Nc, r, G = 1, 24, 128, 1560, 12480, 1560, 384, 32
    args = _lib.NkvAttendArgs()
    args.B, args.H, args.D, args.Q, args.N, args.Nc = B, H, D, Q, N, Nc
    args.softmax_scale = D ** -0.5
    for c in (args.key, args.value):
        c.r, c.group, c.scale_dtype = r, G, _lib.NKV_DTYPE_FP16
    bf = dict(dtype=torch.bfloat16, device=dev)
    q = torch.zeros(B, Q, H, D, **bf)
    out = torch.empty(B, Q, H, D, **bf)
    k_cur = torch.zeros(B, Nc, H, D, **bf)
    v_cur = torch.zeros(B, Nc, H, D, **bf)
    keep = [q, out, k_cur, v_cur]
    args.q, args.out = q.data_ptr(), out.data_ptr()
    args.k_cur, args.v_cur = k_cur.data_ptr(), v_cur.data_ptr()
    for t in (q, out, k_cur, v_cur):
        assert t.is_contiguous()
    args.q_sb, args.q_st, args.q_sh = Q * H * D, H * D, D
    args.o_sb, args.o_st, args.o_sh = Q * H * D, H * D, D
    args.k_sb, args.k_st, args.k_sh = Nc * H * D, H * D, D
    args.v_sb, args.v_st, args.v_sh = Nc * H * D, H * D, D
    for c in (args.key, args.value):
        packed = torch.zeros(B, N, r // 2, dtype=torch.uint8, device=dev)
        scales = torch.zeros(B, N, r // G, dtype=torch.float16, device=dev)
        w_dec = torch.zeros(H * D, r, **bf)
        keep += [packed, scales, w_dec]
        c.packed, c.scales, c.w_dec = packed.data_ptr(), scales.data_ptr(), w_dec.data_ptr()
    need = _lib.lib().nkv_attend_workspace_size(ctypes.byref(args))
    assert need > _lib.NKV_STATIC_SCRATCH_BYTES
    torch.cuda.synchronize()
    rc = _lib.lib().nkv_attend_static(None, ctypes.byref(args))
    assert rc == _lib.NKV_ERR_WORKSPACE
    assert b"nkv_attend_static holds" in _lib.lib().nkv_last_error()
    torch.cuda.synchronize()
    del keep
