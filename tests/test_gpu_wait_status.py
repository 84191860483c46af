"""The bounded waits of the one-pass scans and radix sorts report when they give
up (include/fastgs_hip.h: wait status), and the caller raises.  The give-up
is forced from the host with fgs_set_wait_spin_limit(0) (every wait gives up
at once, without polling); every kernel still runs to its end, the writes
stay in bounds, the status word says which wait gave up, rasterize_gaussians
raises WaitError, and once the limit is restored the same calls are exact
again.  The restored runs double as the GPU test of fgs_sort_pairs_u64 on
full 64-bit keys with ties (the reference's argsort + take,
binding.cpp:195-197) against numpy's stable argsort."""
import contextlib
import ctypes

import numpy as np
import pytest

from fastgs_core_amd import _lib
from fastgs_core_amd import synthetic as syn

from tests.helpers import IMAGE_ATOL, to_np, to_torch

pytestmark = pytest.mark.gpu

LOOK_BACK, SCAN = 2, 1


def _say(*a):
    print("[gpu-test] wait status", *a, flush=True)


@contextlib.contextmanager
def _spin_limit(n):
    lib = _lib.load()
    prev = lib.fgs_set_wait_spin_limit(n)
    try:
        yield
    finally:
        lib.fgs_set_wait_spin_limit(prev)


def _stream(torch, dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _sort(torch, keys, vals):
    lib = _lib.load()
    dev = torch.device("cuda")
    n = keys.size
    ki = torch.from_numpy(keys.view(np.int64)).to(dev)
    vi = torch.from_numpy(vals.view(np.int32)).to(dev)
    ko = torch.empty(n, dtype=torch.int64, device=dev)
    vo = torch.empty(n, dtype=torch.int32, device=dev)
    ws = torch.empty(int(lib.fgs_sort_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    status = torch.full((1,), -1, dtype=torch.int32, device=dev)
    _lib.check(lib.fgs_sort_pairs_u64(ki.data_ptr(), vi.data_ptr(), ko.data_ptr(), vo.data_ptr(),
                                      n, 0, 64, ws.data_ptr(), status.data_ptr(),
                                      _stream(torch, dev)))
    torch.cuda.synchronize()
    return to_np(ko).view(np.uint64), to_np(vo).view(np.uint32), int(status.item())


def test_sort_pairs_u64_full_keys_and_forced_give_up():
    import torch

    rng = np.random.default_rng(3)
    n = 1_500_000
    # 64-bit keys over every bit, with many ties (a few high words, random low)
    hi = rng.integers(0, 5, n, dtype=np.uint64) << np.uint64(61)
    keys = hi | rng.integers(0, 2**20, n, dtype=np.uint64) | (rng.integers(0, 3, n, dtype=np.uint64)
                                                               << np.uint64(40))
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    _say("sort, spin limit 0")
    with _spin_limit(0):
        _, _, status = _sort(torch, keys, vals)
    assert status == LOOK_BACK, status
    _say("sort, default spin limit")
    ko, vo, status = _sort(torch, keys, vals)
    assert status == 0
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(ko, keys[order])
    np.testing.assert_array_equal(vo, vals[order])


def test_scan_forced_give_up_then_exact():
    import torch

    lib = _lib.load()
    dev = torch.device("cuda")
    n = 1_000_003
    x = np.random.default_rng(4).integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    xin = torch.from_numpy(x.view(np.int32)).to(dev)
    out = torch.empty(n, dtype=torch.int32, device=dev)
    ws = torch.empty(int(lib.fgs_scan_workspace_bytes(n)), dtype=torch.uint8, device=dev)
    status = torch.full((1,), -1, dtype=torch.int32, device=dev)
    for limit, want in ((0, SCAN), (None, 0)):
        _say("scan, spin limit", limit)
        ctx = _spin_limit(limit) if limit is not None else contextlib.nullcontext()
        with ctx:
            _lib.check(lib.fgs_inclusive_scan_u32(xin.data_ptr(), out.data_ptr(), n,
                                                  ws.data_ptr(), status.data_ptr(),
                                                  _stream(torch, dev)))
            torch.cuda.synchronize()
        assert int(status.item()) == want
    np.testing.assert_array_equal(to_np(out).view(np.uint32),
                                  np.cumsum(x, dtype=np.uint64).astype(np.uint32))


@pytest.mark.parametrize("grid", ["two_level", "one_level"])
def test_binning_reports_the_depth_sort_give_up(oracle, grid):
    """fgs_binning_sorted writes the wait status of the depth order it runs (and
    of its own scan and tile sort on the one-level path) after them; with
    the waits restored the same call is bit-exact."""
    import torch

    from fastgs_core_amd import rasterizer
    from tests.helpers import scene_small

    if grid == "two_level":
        sc, cam = scene_small(31, 60_000, 0, 1920, 1080)
    else:
        sc, cam = scene_small(32, 30_000, 0, 4352, 2176)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    K = int(ref["rendered"])
    gx, gy = (cam.width + 15) // 16, (cam.height + 15) // 16
    dev = torch.device("cuda")
    g = {k: torch.from_numpy(np.ascontiguousarray(ref[k])).to(dev)
         for k in ("geom_means2d", "geom_depths", "geom_conic_opacity")}
    tiles = torch.from_numpy(ref["geom_tiles_touched"].view(np.int32)).to(dev)
    assert tiles.numel() > 2 * 4096 and K > 8 * 4096  # several chunks in every wait

    def run():
        out = rasterizer._binning_sorted(g["geom_means2d"], g["geom_depths"],
                                         g["geom_conic_opacity"], tiles, K, gx, gy, 1.0)
        torch.cuda.synchronize()
        return out

    _say("binning", grid, "spin limit 0")
    with _spin_limit(0):
        tbuf = run()[-1]
    status = int(tbuf[-1].item())
    assert status & LOOK_BACK, status
    if grid == "one_level":
        assert status == LOOK_BACK | SCAN, status
    _say("binning", grid, "default spin limit")
    keys, plist, ranges, _, boffs, tbuf = run()
    assert int(tbuf[-1].item()) == 0
    np.testing.assert_array_equal(to_np(keys).view(np.uint64), ref["point_list_keys"])
    np.testing.assert_array_equal(to_np(plist).view(np.uint32), ref["point_list"])
    np.testing.assert_array_equal(to_np(boffs).view(np.uint32), ref["bucket_offsets"])


def test_rasterize_gaussians_raises_when_a_wait_gives_up(oracle):
    import torch

    import fastgs_core
    from fastgs_core_amd import WaitError

    sc = syn.scene_config2(5, 40_000, 3)
    cam = syn.sphere_cameras(1, 9, 640, 480)[0]
    inp = syn.make_inputs(sc, cam)
    tin = to_torch(inp)
    _say("rasterize_gaussians, spin limit 0")
    with _spin_limit(0):
        with pytest.raises(WaitError, match="bounded wait gave up"):
            fastgs_core.rasterize_gaussians(tin, 640, 480, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
        torch.cuda.synchronize()
    _say("rasterize_gaussians, default spin limit")
    ref = oracle.render(inp, 640, 480, cam.tan_fovx, cam.tan_fovy, 3)
    out = fastgs_core.rasterize_gaussians(tin, 640, 480, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
    assert out["rendered"] == ref["rendered"]
    np.testing.assert_array_equal(to_np(out["point_list"]).view(np.uint32), ref["point_list"])
    np.testing.assert_allclose(to_np(out["out_color"]), ref["out_color"], atol=IMAGE_ATOL)
