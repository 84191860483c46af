"""The backward's optional tile order (fgs_raster_bwd_io.tile_order).

With the scratch set, fgs_rasterize_bwd first counting-sorts the tiles by
max_contrib (1024 buckets between 0 and the largest value, largest first) and
walks them in that order.  Checked through the C ABI on a rendered scene:
- the order is a permutation of the tiles;
- its buckets, recomputed on the host in float32 (the kernel's operations:
  one IEEE multiply, truncation), never decrease, so max_contrib never rises
  from one bucket to the next;
- the gradients equal those of the index-order walk up to the order of the
  float atomic adds (1e-5 relative plus 1e-6 of the largest magnitude).
"""
import ctypes

import numpy as np
import pytest

from fastgs_core_amd import _lib
from fastgs_core_amd import synthetic as syn

from tests.helpers import scene_small, to_np, to_torch


def _say(*a):
    print("[gpu-test]", *a, flush=True)


def _buckets(mc):
    mc = np.asarray(mc, np.uint32)
    mx = int(mc.max()) if mc.size else 0
    if mx == 0:
        return np.full(mc.shape, 1023, np.int64)
    sc = np.float32(1023.0) / np.float32(mx)
    q = (mc.astype(np.float32) * sc).astype(np.uint32).astype(np.int64)
    return 1023 - np.minimum(q, 1023)


@pytest.mark.gpu
def test_backward_tile_order_is_heaviest_first_and_result_invariant():
    import torch

    import fastgs_core

    sc, cam = scene_small(21, 20000, 3, 640, 480)
    _say("tile order", cam.width, cam.height)
    inp = syn.make_inputs(sc, cam)
    tin = to_torch(inp)
    out = fastgs_core.rasterize_gaussians(tin, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                          cam.tan_fovy, sc["degree"])
    W, H = cam.width, cam.height
    T = ((W + 15) // 16) * ((H + 15) // 16)
    P = out["geom_means2d"].shape[0]
    C = 3
    dev = out["out_color"].device
    rng = np.random.default_rng(3)
    dL = torch.from_numpy(rng.standard_normal((C, W * H)).astype(np.float32)).to(dev)
    bg = torch.zeros(C, dtype=torch.float32, device=dev)
    lib = _lib.load()

    def run(order):
        f32 = dict(dtype=torch.float32, device=dev)
        g = {k: torch.empty(s, **f32) for k, s in (("means2d", (P, 2)), ("colors", (P, C)),
                                                   ("conic", (P, 4)), ("vsp", (P, 4)))}
        prm = _lib.RasterParams(W, H, C, T, int(out["num_buckets"]), 0, 0, P,
                                int(out["point_list"].numel()))

        def p(t):
            return None if t is None else t.data_ptr()

        io = _lib.RasterBwdIO(
            p(out["ranges"]), p(out["point_list"]), p(out["geom_means2d"]), p(out["geom_rgb"]),
            p(out["geom_conic_opacity"]), p(bg), p(out["img_final_t"]), p(out["img_n_contrib"]),
            p(out["img_max_contrib"]), p(dL), p(g["means2d"]), p(g["colors"]), p(g["conic"]),
            p(g["vsp"]), p(order))
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(lib.fgs_rasterize_bwd(ctypes.byref(prm), ctypes.byref(io), stream))
        torch.cuda.synchronize()
        return {k: to_np(v).astype(np.float64) for k, v in g.items()}

    ref = run(None)
    order_t = torch.full((T,), -1, dtype=torch.int32, device=dev)
    got = run(order_t)
    order = to_np(order_t).astype(np.int64)
    np.testing.assert_array_equal(np.sort(order), np.arange(T))
    mc = to_np(out["img_max_contrib"]).astype(np.uint32)
    assert mc.max() > 0
    b = _buckets(mc)[order]
    assert np.all(np.diff(b) >= 0), "buckets must not decrease along the order"
    assert b[0] == 0 and _buckets(mc).min() == 0
    for k in ref:
        scale = np.abs(ref[k]).max()
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-5, atol=1e-6 * scale, err_msg=k)
