"""GPU parity of every hot-path stage against the CPU oracle (restatement of
the reference Metal kernels), through the fastgs_core API and C ABI.

Gates: radii / tiles_touched / sorted keys+values / ranges / bucket arrays /
n_contrib / max_contrib bit-exact; image within 1e-4 absolute; gradients
within 1e-3 of the sum of their terms' magnitudes (helpers.assert_grad_gate).
"""
import sys

import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn
from tests.helpers import (IMAGE_ATOL, assert_grad_gate, capture_2d_gradients,
                           check_backward_stages, scene_small, to_np, to_torch)

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-test]", *a, flush=True)
    sys.stdout.flush()


def _render_both(oracle, sc, cam, get_flag=False, metric_map=None, bg=(0.0, 0.0, 0.0)):
    import fastgs_core

    inp = syn.make_inputs(sc, cam, background=bg)
    if metric_map is not None:
        inp["metric_map"] = metric_map
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, sc["degree"],
                        get_flag=get_flag)
    tin = to_torch(inp)
    out = fastgs_core.rasterize_gaussians(tin, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                          cam.tan_fovy, sc["degree"], 1.0, 1.0, False, get_flag)
    return inp, ref, out


@pytest.mark.parametrize("case", ["cfg1", "sh3_small", "sh3_close", "hd_grid", "wide_grid",
                                  "uhd_grid"])
def test_forward_pipeline_parity(oracle, case):
    if case == "cfg1":
        sc = syn.scene_config1(0, 4096)
        cam = syn.config1_camera(96, 80)
    elif case == "sh3_small":
        sc, cam = scene_small(1, 3000, 3, 160, 112)
    elif case == "hd_grid":  # 120 x 68 tiles: 135 super-tiles of 8 x 8
        sc, cam = scene_small(3, 6000, 1, 1920, 1080)
    elif case == "wide_grid":  # 272 x 8 tiles: 34 x 1 super-tiles (two-level path)
        sc, cam = scene_small(8, 3000, 1, 4352, 128)
    elif case == "uhd_grid":  # 272 x 136 tiles: 578 super-tiles (one-level path)
        sc, cam = scene_small(9, 2000, 1, 4352, 2176)
    else:
        sc, cam = scene_small(2, 1500, 2, 128, 128, eye=(0.3, 0.5, -1.6))
    _say("forward pipeline", case, "P", sc["means3d"].shape[0], cam.width, cam.height)
    inp, ref, out = _render_both(oracle, sc, cam)
    assert out["rendered"] == ref["rendered"]
    assert out["num_buckets"] == ref["num_buckets"]
    # integer outputs: bit-exact
    for k in ("radii", "geom_tiles_touched", "point_offsets", "geom_clamped"):
        np.testing.assert_array_equal(to_np(out[k]).astype(np.int64),
                                      np.asarray(ref[k]).astype(np.int64), err_msg=k)
    # float preprocess outputs: identical operation order -> equal to 1e-6 rel
    for k in ("geom_means2d", "geom_depths", "geom_cov3d", "geom_rgb", "geom_conic_opacity",
              "viewspace_points"):
        np.testing.assert_allclose(to_np(out[k]), ref[k], rtol=1e-6, atol=1e-6, err_msg=k)
    if ref["rendered"] == 0:
        return
    np.testing.assert_array_equal(to_np(out["point_list_keys"]).view(np.uint64),
                                  ref["point_list_keys"], err_msg="point_list_keys")
    np.testing.assert_array_equal(to_np(out["point_list"]).view(np.uint32), ref["point_list"])
    np.testing.assert_array_equal(to_np(out["ranges"]).view(np.uint32), ref["ranges"])
    np.testing.assert_array_equal(to_np(out["bucket_count"]).view(np.uint32), ref["bucket_count"])
    np.testing.assert_array_equal(to_np(out["bucket_offsets"]).view(np.uint32),
                                  ref["bucket_offsets"])
    np.testing.assert_array_equal(to_np(out["sample_bucket_to_tile"]).view(np.uint32),
                                  ref["sample_bucket_to_tile"])
    np.testing.assert_array_equal(to_np(out["img_n_contrib"]).view(np.uint32),
                                  ref["img_n_contrib"])
    np.testing.assert_array_equal(to_np(out["img_max_contrib"]).view(np.uint32),
                                  ref["img_max_contrib"])
    np.testing.assert_allclose(to_np(out["out_color"]), ref["out_color"], rtol=0, atol=IMAGE_ATOL)
    np.testing.assert_allclose(to_np(out["img_pixel_colors"]), ref["img_pixel_colors"], rtol=0,
                               atol=IMAGE_ATOL)
    np.testing.assert_allclose(to_np(out["img_final_t"]), ref["img_final_t"], rtol=0, atol=1e-5)


def test_sampled_state_parity(oracle):
    """write_sampled: T (bit for bit: the blend decisions depend on it) and the
    accumulated colour (image tolerance) of every live pixel at each 32-splat
    bucket start (sample_t / sample_ar); dead pixels keep the zero fill."""
    import fastgs_core

    sc, cam = scene_small(7, 3000, 3, 112, 80)
    _say("sampled state", cam.width, cam.height)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, sc["degree"],
                        write_sampled=True)
    out = fastgs_core.rasterize_gaussians(to_torch(inp), cam.width, cam.height, 16, 16,
                                          cam.tan_fovx, cam.tan_fovy, sc["degree"],
                                          write_sampled=True)
    assert ref["num_buckets"] > 0 and ref["sample_t"].size == ref["num_buckets"] * 256
    np.testing.assert_array_equal(to_np(out["sample_t"]).reshape(-1),
                                  np.asarray(ref["sample_t"]).reshape(-1))
    np.testing.assert_allclose(to_np(out["sample_ar"]).reshape(-1),
                               np.asarray(ref["sample_ar"]).reshape(-1), rtol=0, atol=IMAGE_ATOL)
    assert (to_np(out["sample_ar"]) == 0).sum() == (np.asarray(ref["sample_ar"]) == 0).sum()
    np.testing.assert_array_equal(to_np(out["img_n_contrib"]).view(np.uint32),
                                  ref["img_n_contrib"])
    np.testing.assert_allclose(to_np(out["out_color"]), ref["out_color"], rtol=0, atol=IMAGE_ATOL)


def test_metric_count_parity(oracle):
    sc, cam = scene_small(3, 2000, 1, 96, 96)
    rng = np.random.default_rng(5)
    mm = (rng.random(cam.width * cam.height) < 0.5).astype(np.int32)
    _say("metric count get_flag")
    inp, ref, out = _render_both(oracle, sc, cam, get_flag=True, metric_map=mm)
    np.testing.assert_array_equal(to_np(out["metric_count"]), ref["metric_count"])
    assert int(ref["metric_count"].sum()) > 0


@pytest.mark.parametrize("case", ["cfg1", "sh3", "bg", "sh1", "sh3_deg1", "sh_rows10"])
def test_backward_parity(oracle, case):
    """Gradients of every input against the oracle. The SH cases cover each
    LDS-staged row length (3, 8 and 15 rest coefficients), a degree below the
    buffer's (progressive SH training) and a row of 10 coefficients, which the
    library reads directly instead of staging."""
    import fastgs_core
    import torch

    bg = (0.0, 0.0, 0.0)
    if case == "cfg1":
        sc = syn.scene_config1(1, 3000)
        cam = syn.config1_camera(80, 64)
    elif case == "sh3":
        sc, cam = scene_small(4, 2500, 3, 128, 96)
    elif case == "sh1":
        sc, cam = scene_small(12, 2000, 1, 96, 80)
    elif case == "sh3_deg1":
        sc, cam = scene_small(13, 2000, 3, 96, 80)
    elif case == "sh_rows10":
        sc, cam = scene_small(14, 1999, 3, 112, 80)
        sc["sh"] = np.ascontiguousarray(sc["sh"][:, :10])
        sc["degree"] = 2
    else:
        sc, cam = scene_small(5, 2000, 2, 96, 112)
        bg = (0.2, 0.5, 0.9)
    degree = 1 if case == "sh3_deg1" else sc["degree"]
    _say("backward", case)
    inp = syn.make_inputs(sc, cam, background=bg)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, degree)
    rng = np.random.default_rng(11)
    dL = rng.standard_normal((3, cam.width * cam.height)).astype(np.float32)
    rg = oracle.render_backward(inp, ref, dL, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy,
                                degree, magnitude=True)
    req = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")
    tin = to_torch(inp, requires_grad=req)
    out = fastgs_core.rasterize_gaussians(tin, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                          cam.tan_fovy, degree)
    seen = capture_2d_gradients(out)
    loss = (out["out_color"] * torch.from_numpy(dL).cuda()).sum()
    loss.backward()
    check_backward_stages(oracle, inp, ref, rg, tin, seen, cam.width, cam.height, cam, degree)
    # the viewspace dummy carries (x, y) = dL/dmeans2d exactly
    assert_grad_gate("viewspace (x, y) vs dL/dmeans2d", to_np(tin["viewspace_points"].grad)[:, :2],
                     rg["raster"]["means2d"], rg["raster"]["mag_terms"]["means2d"])


def _assert_nonfinite_pattern_and_close(name, got, ref, mag):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin, err_msg=f"{name}: non-finite pattern")
    assert_grad_gate(name, np.where(fin, got, 0.0), np.where(fin, ref, 0.0),
                     np.where(fin, mag, 0.0))


def test_rasterize_backward_nonfinite_inputs(oracle):
    """NaN loss gradients at a few pixels and an infinite splat colour reach
    exactly the gradient entries the per-(pixel, splat) definition sends them
    to; every other entry still matches the oracle (the kernel's fast form is
    used only where all operands are finite)."""
    import torch

    import fastgs_core

    sc, cam = scene_small(6, 2500, 3, 128, 96)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, sc["degree"])
    pre, r = ref["pre"], ref["raster"]
    W, H = cam.width, cam.height
    rng = np.random.default_rng(21)
    dL = rng.standard_normal((3, W * H)).astype(np.float32)
    dL[:, [5 * W + 7, 40 * W + 64, 90 * W + 100]] = np.nan  # three pixels, three tiles
    colors = pre["rgb"].astype(np.float32).copy()
    hot = int(np.flatnonzero(pre["radii"] > 0)[len(np.flatnonzero(pre["radii"] > 0)) // 2])
    colors[hot, 1] = np.inf
    _say("rasterize backward non-finite inputs, inf colour on", hot)
    g = oracle.rasterize_bwd(ref["ranges"], ref["point_list"], pre["xys"], colors,
                             pre["conic_opacity"], inp["background"], r["final_t"], r["n_contrib"],
                             dL, W, H, magnitude=True)
    assert np.isnan(g["means2d"]).any() and np.isfinite(g["means2d"]).any()
    dev = torch.device("cuda")
    P = pre["xys"].shape[0]
    m2 = torch.from_numpy(pre["xys"].astype(np.float32)).to(dev).requires_grad_(True)
    col = torch.from_numpy(colors).to(dev).requires_grad_(True)
    co = torch.from_numpy(pre["conic_opacity"].astype(np.float32)).to(dev).requires_grad_(True)
    vsp = torch.zeros((P, 4), dtype=torch.float32, device=dev, requires_grad=True)
    T = ref["ranges"].shape[0]
    out = fastgs_core.rasterize_forward(
        ref["ranges"], ref["point_list"], ref["bucket_offsets"], m2, col, co, inp["background"],
        pre["radii"], None, None, vsp, W, H, 16, 16, 3, T, int(ref["bucket_offsets"][-1]), False)
    np.testing.assert_array_equal(to_np(out["n_contrib"]).view(np.uint32), r["n_contrib"])
    out["out_color"].backward(torch.from_numpy(dL).to(dev))
    for name, t, rk in (("means2d", m2, "means2d"), ("colors", col, "colors"),
                        ("conic_opacity", co, "conic_opacity"),
                        ("viewspace", vsp, "viewspace_points")):
        _assert_nonfinite_pattern_and_close(name, to_np(t.grad), g[rk], g["mag_terms"][rk])


def test_rasterize_forward_standalone_closed_form():
    """Reference rasterize_smoke.py fixture: one splat at (8,8), conic (1,0,1)."""
    import fastgs_core
    import torch

    _say("rasterize_forward closed form")
    o = 0.9
    out = fastgs_core.rasterize_forward(
        np.array([[0, 1]], np.uint32), np.array([0], np.uint32), np.array([1], np.uint32),
        np.array([[8.0, 8.0]], np.float32), np.array([[1.0, 0.0, 0.0]], np.float32),
        np.array([[1.0, 0.0, 1.0, o]], np.float32), np.zeros(3, np.float32),
        np.array([1], np.int32), np.zeros(256, np.int32), np.zeros(1, np.int32),
        np.zeros((1, 4), np.float32), 16, 16, 16, 16, 3, 1, 1, False)
    y, x = np.mgrid[0:16, 0:16]
    alpha = np.minimum(0.99, o * np.exp(-0.5 * ((8 - x) ** 2 + (8 - y) ** 2)))
    alpha = np.where(alpha >= 1 / 255, alpha, 0.0)
    img = to_np(out["out_color"]).reshape(3, 16, 16)
    np.testing.assert_allclose(img[0], alpha, atol=1e-6)
    np.testing.assert_allclose(img[1:], 0.0, atol=0)
    np.testing.assert_allclose(to_np(out["final_t"]).reshape(16, 16), 1 - alpha, atol=1e-6)
    np.testing.assert_array_equal(to_np(out["n_contrib"]).reshape(16, 16), (alpha > 0).astype(int))
    assert int(to_np(out["max_contrib"])[0]) == 1
    assert torch.is_tensor(out["out_color"])


def test_tile_prep_and_binning_kats():
    """Reference tile_prep_smoke.py / binning_smoke.py fixtures."""
    import fastgs_core

    _say("tile_prep + binning KATs")
    keys = np.array([(0 << 32) | 1, (0 << 32) | 2, (1 << 32) | 1, (1 << 32) | 2, (1 << 32) | 3,
                     (3 << 32) | 1, (3 << 32) | 2, (3 << 32) | 3], np.uint64)
    out = fastgs_core.tile_prep_forward(keys, 8, 4)
    np.testing.assert_array_equal(to_np(out["ranges"]), [[0, 2], [2, 5], [0, 0], [5, 8]])
    np.testing.assert_array_equal(to_np(out["bucket_count"]), [1, 1, 0, 1])
    p = 8
    out = fastgs_core.binning_forward(np.zeros((p, 2), np.float32), np.arange(p, dtype=np.float32),
                                      np.arange(1, p + 1, dtype=np.uint32),
                                      np.ones((p, 4), np.float32), np.ones(p, np.uint32), 1.0, 4,
                                      4, 1, p)
    np.testing.assert_array_equal(to_np(out["point_list_keys_unsorted"]), np.zeros(p))
    np.testing.assert_array_equal(to_np(out["point_list_unsorted"]), np.zeros(p))


def test_binning_forward_matches_oracle(oracle):
    import fastgs_core

    sc, cam = scene_small(6, 3000, 0, 128, 128)
    _say("binning_forward vs oracle")
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    gx, gy = (cam.width + 15) // 16, (cam.height + 15) // 16
    out = fastgs_core.binning_forward(ref["geom_means2d"], ref["geom_depths"],
                                      ref["point_offsets"], ref["geom_conic_opacity"],
                                      ref["geom_tiles_touched"], 1.0, gx, gy, 1, ref["rendered"])
    np.testing.assert_array_equal(to_np(out["point_list_keys_unsorted"]).view(np.uint64),
                                  ref["point_list_keys_unsorted"])
    np.testing.assert_array_equal(to_np(out["point_list_unsorted"]).view(np.uint32),
                                  ref["point_list_unsorted"])
    tp = fastgs_core.tile_prep_forward(ref["point_list_keys"], ref["rendered"], gx * gy)
    np.testing.assert_array_equal(to_np(tp["ranges"]).view(np.uint32), ref["ranges"])
    np.testing.assert_array_equal(to_np(tp["bucket_count"]).view(np.uint32), ref["bucket_count"])


@pytest.mark.parametrize("grid", ["two_level", "one_level"])
def test_binning_sorted_depth_order_entry(oracle, grid):
    """fgs_binning_sorted with the depth order sorted inside the call
    (depth_order NULL) and with it from a separate fgs_depth_order call: both
    give the oracle's sorted keys, values, ranges and bucket arrays bit for
    bit, on a grid of at most 256 super-tiles (two-level binning) and on one
    of 578 (the one-level fallback)."""
    import torch

    from fastgs_core_amd import _lib, rasterizer

    if grid == "two_level":
        sc, cam = scene_small(15, 2500, 0, 320, 176)
    else:
        sc, cam = scene_small(9, 2000, 0, 4352, 2176)
    _say("binning_sorted depth order", grid)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    K = int(ref["rendered"])
    assert K > 0
    gx, gy = (cam.width + 15) // 16, (cam.height + 15) // 16
    dev = torch.device("cuda")
    g = {k: torch.from_numpy(np.ascontiguousarray(ref[k])).to(dev)
         for k in ("geom_means2d", "geom_depths", "geom_conic_opacity")}
    tiles = torch.from_numpy(ref["geom_tiles_touched"].view(np.int32)).to(dev)
    P = tiles.numel()
    lib = _lib.load()
    dws = torch.empty(int(lib.fgs_depth_order_workspace_bytes(P)), dtype=torch.uint8, device=dev)
    _lib.check(lib.fgs_depth_order(P, g["geom_depths"].data_ptr(), tiles.data_ptr(),
                                   dws.data_ptr(), rasterizer._stream(dev)))
    for depth_ws in (None, dws):
        keys, plist, ranges, bcount, boffs, tbuf = rasterizer._binning_sorted(
            g["geom_means2d"], g["geom_depths"], g["geom_conic_opacity"], tiles, K, gx, gy, 1.0,
            depth_ws)
        assert int(tbuf[-1].item()) == 0  # wait status: every wait completed
        np.testing.assert_array_equal(to_np(keys).view(np.uint64), ref["point_list_keys"])
        np.testing.assert_array_equal(to_np(plist).view(np.uint32), ref["point_list"])
        np.testing.assert_array_equal(to_np(ranges).view(np.uint32).reshape(-1, 2),
                                      np.asarray(ref["ranges"]).reshape(-1, 2))
        np.testing.assert_array_equal(to_np(bcount).view(np.uint32), ref["bucket_count"])
        np.testing.assert_array_equal(to_np(boffs).view(np.uint32), ref["bucket_offsets"])


def test_empty_scene():
    import fastgs_core

    _say("empty scene")
    sc = syn.scene_config1(0, 256)
    cam = syn.config1_camera(64, 64)
    sc["means3d"] = sc["means3d"] - np.array([0, 0, 10], np.float32)  # all behind the camera
    out = fastgs_core.rasterize_gaussians(to_torch(syn.make_inputs(sc, cam)), 64, 64, 16, 16,
                                          cam.tan_fovx, cam.tan_fovy, 0)
    assert out["rendered"] == 0 and out["num_buckets"] == 0
    assert out["out_color"].numel() == 0
    assert int(out["radii"].abs().sum()) == 0


def test_preprocess_forward_standalone_kat():
    """Reference preprocess_smoke.py fixture (colour path fixed): all means at the
    origin with an identity view -> z = 0 <= 0.2 -> every output zero."""
    import fastgs_core

    _say("preprocess_forward KAT")
    n = 8
    inputs = {
        "means3d": np.zeros((n, 3), np.float32), "opacities": np.ones((n, 1), np.float32),
        "cov3d_precomp": np.ones((n, 6), np.float32),
        "colors_precomp": np.ones((n, 3), np.float32), "viewmat": np.eye(4, dtype=np.float32),
        "projmat": np.eye(4, dtype=np.float32), "cam_pos": np.zeros(3, np.float32),
        "viewspace_points": np.zeros((n, 4), np.float32),
    }
    out = fastgs_core.preprocess_forward(inputs, 16, 16)
    for k, v in out.items():
        assert float(to_np(v).astype(np.float64).__abs__().sum()) == 0.0, k


def test_preprocess_backward_validation_kat():
    """Reference preprocess_backward_validation.py: loss = sum(xys) + 0.1 sum(depths)
    + 0.01 sum(viewspace_points) -> d_viewspace == 0.01 on every visible row."""
    import fastgs_core
    import torch

    _say("preprocess backward KAT")
    n = 8
    m = torch.tensor([[0.1, 0.2, 1.0], [0.2, 0.1, 1.1], [0.3, 0.0, 1.2], [0.0, 0.3, 1.3],
                      [0.1, 0.1, 1.4], [0.2, 0.2, 1.5], [0.3, 0.3, 1.6], [0.4, 0.2, 1.7]],
                     device="cuda", requires_grad=True)
    vsp = torch.zeros((n, 4), device="cuda", requires_grad=True)
    inputs = {
        "means3d": m, "opacities": torch.ones((n, 1), device="cuda"),
        "cov3d_precomp": torch.ones((n, 6), device="cuda"),
        "colors_precomp": torch.ones((n, 3), device="cuda"),
        "viewmat": torch.eye(4, device="cuda"), "projmat": torch.eye(4, device="cuda"),
        "cam_pos": torch.zeros(3, device="cuda"), "viewspace_points": vsp,
    }
    out = fastgs_core.preprocess_forward(inputs, 16, 16)
    loss = out["xys"].sum() + 0.1 * out["depths"].sum() + 0.01 * out["viewspace_points"].sum()
    loss.backward()
    vis = to_np(out["radii"]) > 0
    g = to_np(vsp.grad)
    np.testing.assert_array_equal(g[vis], np.float32(0.01))
    np.testing.assert_array_equal(g[~vis], 0.0)
    assert np.isfinite(to_np(m.grad)).all()


def test_cov3d_precomp_colors_path_backward(oracle):
    """Precomputed-covariance / precomputed-colour path through the full backward."""
    import fastgs_core
    import torch

    sc, cam = scene_small(7, 1500, 0, 96, 96)
    _say("precomp path backward")
    rng = np.random.default_rng(3)
    P = sc["means3d"].shape[0]
    inp = syn.make_inputs(sc, cam)
    from oracle.oracle import Oracle  # noqa: F401
    pre = oracle.preprocess_fwd(inp["means3d"], inp["opacities"], inp["viewmatrix"],
                                inp["projmatrix"], inp["campos"], inp["viewspace_points"],
                                cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0,
                                scales=inp["scales"], rotations=inp["rotations"],
                                colors_precomp=np.zeros((P, 3), np.float32))
    for k in ("scales", "rotations", "dc", "sh"):
        del inp[k]
    inp["cov3d_precomp"] = pre["cov3d"]
    inp["colors_precomp"] = rng.uniform(0, 1, (P, 3)).astype(np.float32)
    ref = oracle.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    dL = rng.standard_normal((3, cam.width * cam.height)).astype(np.float32)
    rg = oracle.render_backward(inp, ref, dL, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0,
                                magnitude=True)
    tin = to_torch(inp, requires_grad=("means3d", "colors_precomp", "opacities", "cov3d_precomp"))
    out = fastgs_core.rasterize_gaussians(tin, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                          cam.tan_fovy, 0)
    np.testing.assert_allclose(to_np(out["out_color"]), ref["out_color"], atol=IMAGE_ATOL)
    (out["out_color"] * torch.from_numpy(dL).cuda()).sum().backward()
    assert_grad_gate("means3d", to_np(tin["means3d"].grad), rg["means3d"], rg["mag_terms"]["means3d"])
    assert_grad_gate("colors_precomp", to_np(tin["colors_precomp"].grad), rg["colors_precomp"], rg["mag_terms"]["colors_precomp"])
    assert_grad_gate("opacities", to_np(tin["opacities"].grad), rg["opacities"], rg["mag_terms"]["opacities"])
    assert float(tin["cov3d_precomp"].grad.abs().sum()) == 0.0
