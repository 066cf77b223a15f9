"""The staged schedule's workspace plan against the extents its kernels write
(host arithmetic of the library, no GPU).

Every staged call plans one workspace: per partition its tile images (K and
V^T per 128-key tile, at the partition's K/Q width), then its split partials.
nkv_plan_check runs the library's planner and checks, from the same tile
format the decode and flash kernels address the tiles with, that each
partition's last V^T image and its partials end inside its slice.  The same
check runs inside every staged call before any launch.  A decode that wrote
the V^T images of a 32- or 64-wide partition at the 128-wide tile stride
(a layout mistake that once faulted a GPU run) is caught here, on the CPU.
The same check holds the decode launch's block plan to what the kernel
assumes: per codec a multiple of 8 blocks with ranges of at most 24 tiles,
and current-key blocks whenever a partition has current tiles.
"""
import ctypes

import pytest

from nanokv_amd import _lib


def _check(parts, v_dk=0):
    lib = _lib.lib()
    fn = lib.nkv_plan_check
    fn.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_size_t)]
    fn.restype = ctypes.c_int
    flat = [v for p in parts for v in p]
    arr = (ctypes.c_int64 * len(flat))(*flat)
    total = ctypes.c_size_t(0)
    rc = fn(arr, len(parts), v_dk, ctypes.byref(total))
    return rc, lib.nkv_last_error().decode(), total.value


# (B, H, dk, Q, n_rows, Nc, rK, rV, camera)
CFG1 = (1, 24, 128, 1560, 12480, 1560, 384, 384, 0)
CFG2 = (1, 24, 128, 780, 49920, 780, 384, 256, 0)
CFG3_NATIVE = (1, 24, 128, 1560, 3120, 1560, 384, 384, 0)


def _tiles(H, dk, n_rows, Nc, B=1):
    chunks = -(-n_rows // 256) + -(-Nc // 256)
    return B * H * 2 * chunks * 128 * (dk + 128) * 2


@pytest.mark.parametrize("parts", [
    [CFG1],
    [CFG2],
    [(2, 3, 128, 100, 300, 0, 128, 64, 0)],          # last history tile empty (300 % 256 <= 128)
    [(1, 2, 128, 33, 1, 1, 64, 64, 1)],               # one key each, camera (stage8 decode)
    [CFG3_NATIVE, (1, 18, 32, 1560, 9360, 0, 384, 384, 0)],
    [CFG3_NATIVE, (1, 6, 128, 1560, 9360, 0, 384, 384, 0),
     (1, 6, 32, 1560, 9360, 0, 384, 384, 0), (1, 12, 64, 1560, 9360, 0, 384, 384, 0)],
    [(2, 4, 128, 1024, 700, 200, 256, 128, 0), (2, 4, 64, 1024, 1000, 0, 256, 128, 0)],
])
def test_plan_extents_fit(parts):
    rc, err, total = _check(parts)
    assert rc == _lib.NKV_OK, err
    # the plan holds at least every partition's tile images
    assert total >= sum(_tiles(p[1], p[2], p[4], p[5], p[0]) for p in parts)


def test_cfg1_workspace_is_the_documented_size():
    rc, err, total = _check([CFG1])
    assert rc == _lib.NKV_OK, err
    tiles = _tiles(24, 128, 12480, 1560)
    assert tiles == 24 * 112 * 64 * 1024          # 176.2 MB of tile images
    assert total - tiles == pytest.approx(29.8e6, rel=0.01)   # split partials


@pytest.mark.parametrize("dk", [32, 64])
def test_v_images_at_the_128_wide_stride_are_caught(dk):
    """The V^T images of a narrow partition addressed with the 128-wide tile
    format run past its tiles: the check names the last V^T image."""
    parts = [CFG3_NATIVE, (1, 18, dk, 1560, 9360, 0, 384, 384, 0)]
    rc, err, _ = _check(parts, v_dk=128)
    assert rc == _lib.NKV_ERR_INVALID
    assert "partition 1" in err and "last V^T image" in err
    # the partition's own width fits
    assert _check(parts, v_dk=dk)[0] == _lib.NKV_OK


def test_unstaged_partitions_are_refused():
    # a 32-wide reader with ranks above the resident decoder's 384 runs the
    # key-chunk kernel, not the staged plan; with the camera and ranks up to
    # 384 it is staged
    rc, err, _ = _check([(1, 4, 32, 64, 512, 0, 448, 128, 1)])
    assert rc == _lib.NKV_ERR_INVALID and "not staged" in err
    assert _check([(1, 4, 32, 64, 512, 0, 384, 128, 1)])[0] == _lib.NKV_OK


@pytest.mark.parametrize("B,H,n_rows,Nc,rK,rV", [
    (1, 24, 12480, 1560, 384, 384),    # cfg1
    (1, 24, 49920, 780, 384, 256),     # cfg2: K and V in two launches
    (1, 1, 1, 1, 64, 64),              # one tile of each
    (3, 5, 128 * 37 - 5, 700, 384, 384),
    (2, 64, 300, 5000, 128, 128),      # more current than history tiles
    (1, 8, 2_000_000, 0, 384, 384),    # ranges pinned at 24 tiles
    (1, 24, 0, 1560, 384, 384),        # current keys only
    (4, 40, 12480, 1560, 192, 320),
])
def test_decode_block_plan(B, H, n_rows, Nc, rK, rV):
    rc, err, _ = _check([(B, H, 128, 1024, n_rows, Nc, rK, rV, 0)])
    assert rc == _lib.NKV_OK, err
