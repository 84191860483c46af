"""BASELINE configs[2] (cfg3) at its full size: 1,000,000 Gaussians, SH degree 3,
1920x1080, the first of the bench's seeded poses.

The oracle finishes this frame in a few seconds on the host, so the forward
is checked against it exactly as the small cases are (integer outputs and
the tile lists bit-exact, the image within 1e-4), and the gradients through
the three gates of tests.helpers.check_backward_stages (the rasterize
backward's outputs, the preprocess backward on identical inputs, and end to
end, each against the sum of its terms' magnitudes).  Size-free properties are
checked as well: K is the sum of the tile counts, each tile's keys are sorted
by depth, and the viewspace gradient's absolute-value terms bound its signed
terms.
"""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

from tests.helpers import (IMAGE_ATOL, capture_2d_gradients, check_backward_stages, to_np,
                           to_torch)


def _say(*a):
    print("[gpu-test]", *a, flush=True)


@pytest.mark.gpu
def test_cfg3_full_size_forward_and_backward(oracle):
    import torch

    import fastgs_core

    P, W, H = 1_000_000, 1920, 1080
    sc = syn.scene_config2(0, P, 3)
    cam = syn.sphere_cameras(20, 1, W, H)[0]
    _say("cfg3 full size", P, W, H)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, W, H, cam.tan_fovx, cam.tan_fovy, 3)
    req = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")
    tin = to_torch(inp, requires_grad=req)
    out = fastgs_core.rasterize_gaussians(tin, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
    K = out["rendered"]
    assert K == ref["rendered"] and K > 1_000_000
    for k in ("radii", "geom_tiles_touched", "point_offsets"):
        np.testing.assert_array_equal(to_np(out[k]).astype(np.int64),
                                      np.asarray(ref[k]).astype(np.int64), err_msg=k)
    keys = to_np(out["point_list_keys"]).view(np.uint64)
    np.testing.assert_array_equal(keys, ref["point_list_keys"], err_msg="point_list_keys")
    np.testing.assert_array_equal(to_np(out["point_list"]).view(np.uint32), ref["point_list"])
    np.testing.assert_array_equal(to_np(out["ranges"]).view(np.uint32), ref["ranges"])
    np.testing.assert_array_equal(to_np(out["img_n_contrib"]).view(np.uint32),
                                  ref["img_n_contrib"])
    np.testing.assert_allclose(to_np(out["out_color"]), ref["out_color"], rtol=0, atol=IMAGE_ATOL)
    # size-free properties of the binning
    tiles = to_np(out["geom_tiles_touched"]).astype(np.int64)
    assert int(tiles.sum()) == K
    assert np.all(keys[1:] >= keys[:-1]), "keys are sorted by (tile, depth bits)"

    rng = np.random.default_rng(11)
    dL = rng.standard_normal((3, W * H)).astype(np.float32)
    _say("cfg3 full size backward")
    rg = oracle.render_backward(inp, ref, dL, W, H, cam.tan_fovx, cam.tan_fovy, 3,
                                magnitude=True)
    seen = capture_2d_gradients(out)
    loss = (out["out_color"] * torch.from_numpy(dL).cuda()).sum()
    loss.backward()
    check_backward_stages(oracle, inp, ref, rg, tin, seen, W, H, cam, 3)
    vg = to_np(tin["viewspace_points"].grad).astype(np.float64)
    slack = 1e-5 * np.abs(vg).max()
    assert np.all(vg[:, 2] >= np.abs(vg[:, 0]) - slack)
    assert np.all(vg[:, 3] >= np.abs(vg[:, 1]) - slack)
