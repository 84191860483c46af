"""BASELINE.json configs[0], [1], [3] and [4] at their stated sizes, against the
oracle on the same seeded inputs (configs[2], cfg3, is test_gpu_fullsize.py).

* cfg1 (plumbing): 16,384 Gaussians at 256x256, SH 0, one forward render and
  the backward of an L1 loss against a seeded U(0,1) target.
* cfg2: 200,000 Gaussians at 1280x720, SH 3, forward-only, two of its eight
  seeded poses.
* cfg4 (heavy-overlap stress): 3,000,000 Gaussians at 1920x1080, SH 3, 2 % of
  them large (about 1.9e8 tile duplicates, the largest touching all 8,160
  tiles), forward and backward.
* cfg5 (densification loop): 100,000 Gaussians from the reference's initial
  model at 1280x720, trained for 100 iterations against targets rendered
  from a hidden 300k scene, then the scores and one densify-and-prune event
  against the densification oracle on the same random draws.

Gates: integer outputs (radii, tile counts, offsets, sorted keys and
values, ranges, bucket arrays, contributor counts) bit-exact; the image
within 1e-4; the gradients through the three gates of
tests.helpers.check_backward_stages; the densification bit-exact.
"""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

from tests.helpers import IMAGE_ATOL, capture_2d_gradients, check_backward_stages, to_np, to_torch

pytestmark = pytest.mark.gpu

REQ = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")


def _say(*a):
    print("[gpu-test]", *a, flush=True)


def _check_forward(out, ref, name):
    """Every integer output bit-exact, the image within 1e-4."""
    K = out["rendered"]
    assert K == ref["rendered"], (name, K, ref["rendered"])
    assert out["num_buckets"] == ref["num_buckets"], (name, out["num_buckets"], ref["num_buckets"])
    for k in ("radii", "geom_tiles_touched", "point_offsets", "bucket_count", "bucket_offsets"):
        np.testing.assert_array_equal(to_np(out[k]).astype(np.int64),
                                      np.asarray(ref[k]).astype(np.int64), err_msg=f"{name} {k}")
    np.testing.assert_array_equal(to_np(out["geom_clamped"]).astype(np.uint8),
                                  np.asarray(ref["geom_clamped"]).astype(np.uint8))
    np.testing.assert_array_equal(to_np(out["point_list_keys"]).view(np.uint64),
                                  ref["point_list_keys"], err_msg=f"{name} point_list_keys")
    np.testing.assert_array_equal(to_np(out["point_list"]).view(np.uint32), ref["point_list"],
                                  err_msg=f"{name} point_list")
    np.testing.assert_array_equal(to_np(out["ranges"]).view(np.uint32), ref["ranges"],
                                  err_msg=f"{name} ranges")
    for k in ("img_n_contrib", "img_max_contrib"):
        np.testing.assert_array_equal(to_np(out[k]).view(np.uint32), ref[k], err_msg=f"{name} {k}")
    err = float(np.abs(to_np(out["out_color"]) - ref["out_color"]).max())
    _say(name, f"K={K} B={out['num_buckets']} image max err {err:.2e}")
    assert err <= IMAGE_ATOL, (name, err)


def test_cfg1_plumbing_l1_step(oracle):
    """16,384 Gaussians, 256x256, SH 0, camera at (0,0,-4) looking +z,
    black background; forward plus the backward of mean |out - target| against a
    seeded U(0,1) target.  The loss gradient the rasterizer receives is
    captured and given to the oracle, so both sides differentiate the same
    cotangent."""
    import torch

    import fastgs_core
    import fastgs_core_amd

    P, W, H = 16384, 256, 256
    sc = syn.scene_config1(0, P)
    cam = syn.config1_camera(W, H)
    _say("cfg1", P, W, H)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, W, H, cam.tan_fovx, cam.tan_fovy, 0)
    tin = to_torch(inp, requires_grad=REQ)
    out = fastgs_core.rasterize_gaussians(tin, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, 0)
    _check_forward(out, ref, "cfg1")
    target = torch.from_numpy(np.random.default_rng(1).uniform(0, 1, (3, W * H))
                              .astype(np.float32)).cuda()
    seen = []
    out["out_color"].register_hook(lambda g: seen.append(g.detach().clone()))
    seen2d = capture_2d_gradients(out)
    loss = fastgs_core_amd.l1_loss(out["out_color"], target)
    loss.backward()
    dL = to_np(seen[0]).reshape(3, -1)
    img = to_np(out["out_color"]).astype(np.float64)
    want = np.sign(img - to_np(target)) / img.size
    np.testing.assert_allclose(dL, want, rtol=1e-6, atol=0)
    ref_loss = float(np.abs(img - to_np(target)).mean())
    assert abs(float(loss.detach()) - ref_loss) <= 1e-6 * ref_loss
    rg = oracle.render_backward(inp, ref, dL, W, H, cam.tan_fovx, cam.tan_fovy, 0, magnitude=True)
    check_backward_stages(oracle, inp, ref, rg, tin, seen2d, W, H, cam, 0,
                          ("means3d", "scales", "rotations", "opacities", "dc",
                           "viewspace_points"))


@pytest.mark.parametrize("pose", [0, 5])
def test_cfg2_forward_poses(oracle, pose):
    """200,000 Gaussians, 1280x720, SH 3, forward only; poses 0 and 5
    of the bench's eight seeded sphere cameras."""
    import fastgs_core

    P, W, H = 200_000, 1280, 720
    sc = syn.scene_config2(0, P, 3)
    cam = syn.sphere_cameras(8, 1, W, H)[pose]
    _say("cfg2 pose", pose)
    inp = syn.make_inputs(sc, cam)
    ref = oracle.render(inp, W, H, cam.tan_fovx, cam.tan_fovy, 3)
    tin = to_torch(inp)
    out = fastgs_core.rasterize_gaussians(tin, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
    _check_forward(out, ref, f"cfg2 pose {pose}")
    for k in ("geom_means2d", "geom_depths", "geom_conic_opacity", "geom_rgb", "geom_cov3d"):
        np.testing.assert_allclose(to_np(out[k]), ref[k], rtol=1e-6, atol=1e-6, err_msg=k)


@pytest.mark.timeout(900)
def test_cfg4_heavy_overlap_forward_and_backward(oracle):
    """3,000,000 Gaussians at 1920x1080 (log-scales N(-4,1.2), 2 % from
    N(-1.5,0.3), opacity logits N(1,1)), SH 3, the first of the bench's poses.
    About 1.9e8 duplicates: keys, values and ranges bit-exact, then the
    gradients through the three gates of check_backward_stages."""
    import torch

    import fastgs_core

    P, W, H = 3_000_000, 1920, 1080
    sc = syn.scene_config4(0, P, 3)
    cam = syn.sphere_cameras(4, 1, W, H)[0]
    inp = syn.make_inputs(sc, cam)
    _say("cfg4 oracle forward")
    ref = oracle.render(inp, W, H, cam.tan_fovx, cam.tan_fovy, 3)
    assert ref["rendered"] > 30_000_000
    _say("cfg4 GPU forward, K =", ref["rendered"], "B =", ref["num_buckets"])
    tin = to_torch(inp, requires_grad=REQ)
    out = fastgs_core.rasterize_gaussians(tin, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
    torch.cuda.synchronize()
    _say("cfg4 forward comparison")
    _check_forward(out, ref, "cfg4")
    tiles = to_np(out["geom_tiles_touched"]).astype(np.int64)
    assert int(tiles.sum()) == out["rendered"] and tiles.max() == (W // 16) * ((H + 15) // 16)
    dL = np.random.default_rng(11).standard_normal((3, W * H)).astype(np.float32)
    _say("cfg4 GPU backward")
    seen = capture_2d_gradients(out)
    (out["out_color"] * torch.from_numpy(dL).cuda()).sum().backward()
    torch.cuda.synchronize()
    _say("cfg4 oracle backward")
    rg = oracle.render_backward(inp, ref, dL, W, H, cam.tan_fovx, cam.tan_fovy, 3, magnitude=True)
    _say("cfg4 gradient comparison")
    check_backward_stages(oracle, inp, ref, rg, tin, seen, W, H, cam, 3)


def _cfg5_state(torch, dev, P_start, seed=0):
    from fastgs_core_amd import scanner
    from fastgs_core_amd.densify import GaussianTrainState

    rng = np.random.default_rng(seed)
    pts = np.clip(rng.standard_normal((P_start, 3)), -2.0, 2.0).astype(np.float32)
    colors = rng.uniform(0.0, 1.0, (P_start, 3)).astype(np.float32)
    return GaussianTrainState({k: torch.from_numpy(v).to(dev)
                               for k, v in scanner.init_model(pts, colors, 3).items()})


@pytest.mark.timeout(600)
def test_cfg5_densify_event_at_size():
    """the reference's initial model of 100,000 points at 1280x720,
    100 training iterations (one sphere camera each, MSE against targets of a
    hidden 300k scene, statistics from the viewspace gradients, the Adam
    cadence), then the event of iteration 100: metric-map scores over 10
    sampled cameras checked against the oracle's score functions on the same
    renders, and densify_and_prune_fastgs against the densification oracle on
    the same draws -- every parameter row, Adam moment and statistic bit-exact."""
    import torch

    import fastgs_core
    import fastgs_core_amd
    from fastgs_core_amd.densify import (PARAM_NAMES, STAT_NAMES, DensifyConfig,
                                         GaussianTrainState, compute_scene_extent)
    from oracle.densify import DensifyOracle

    dev = torch.device("cuda")
    W, H, HW = 1280, 720, 1280 * 720
    cams = syn.sphere_cameras(50, 11, W, H)
    cam_in = [{"viewmatrix": torch.from_numpy(c.viewmatrix.reshape(-1).copy()).to(dev),
               "projmatrix": torch.from_numpy(c.projmatrix.reshape(-1).copy()).to(dev),
               "campos": torch.from_numpy(c.campos.copy()).to(dev),
               "background": torch.zeros(3, device=dev)} for c in cams]
    zeros_mm = torch.zeros(HW, dtype=torch.int32, device=dev)

    def render(ts, idx, degree, metric_map=None, vsp=None):
        d = ts.render_inputs(cam_in[idx])
        d["metric_map"] = metric_map if metric_map is not None else zeros_mm
        if vsp is not None:
            d["viewspace_points"] = vsp
        c = cams[idx]
        return fastgs_core.rasterize_gaussians(d, W, H, 16, 16, c.tan_fovx, c.tan_fovy, degree,
                                               get_flag=metric_map is not None)

    _say("cfg5 targets")
    hsc = syn.scene_config2(101, 300_000, 3)
    opac = np.clip(hsc["opacities"].astype(np.float64), 1e-6, 1 - 1e-6)
    hidden = GaussianTrainState({
        "means3d": torch.from_numpy(hsc["means3d"]).to(dev),
        "features_dc": torch.from_numpy(hsc["dc"]).to(dev),
        "features_rest": torch.from_numpy(hsc["sh"]).to(dev),
        "opacity_logits": torch.from_numpy(np.log(opac / (1 - opac)).astype(np.float32)
                                           .reshape(-1, 1)).to(dev),
        "log_scales": torch.from_numpy(np.log(hsc["scales"]).astype(np.float32)).to(dev),
        "rotations": torch.from_numpy(hsc["rotations"]).to(dev)})
    with torch.no_grad():
        targets = [render(hidden, i, 3)["out_color"].detach().reshape(3, HW).clone()
                   for i in range(len(cams))]
    del hidden
    ts = _cfg5_state(torch, dev, 100_000)
    extent = compute_scene_extent(ts.param("means3d").detach())
    rng = np.random.default_rng(42)
    stack = []
    _say("cfg5 100 iterations")
    for it in range(1, 101):
        ts.update_learning_rate(it)
        if not stack:
            stack = list(range(len(cams)))
        idx = stack.pop(int(rng.integers(0, len(stack))))
        vsp = torch.zeros((ts.P, 4), device=dev, requires_grad=True)
        out = render(ts, idx, 0, vsp=vsp)
        loss = fastgs_core_amd.mse_loss(out["out_color"].reshape(3, HW), targets[idx])
        ts.zero_grad()
        loss.backward()
        ts.update_densification_stats(out["radii"], vsp.grad)
        ts.step(it)
    assert np.isfinite(float(loss.detach()))
    dor = DensifyOracle()
    dcfg = DensifyConfig()
    ids = [int(i) for i in rng.choice(len(cams), size=dcfg.densify_camera_sample, replace=False)]
    renders = []

    def scoring_render(i, mm):
        o = render(ts, i, 0, metric_map=mm)
        renders.append(o)
        return o

    _say("cfg5 scores over", len(ids), "cameras")
    with torch.no_grad():
        imp, prn = ts.compute_gaussian_scores_fastgs(scoring_render, targets, ids,
                                                     dcfg.loss_thresh, True)
    counts = np.zeros(ts.P, np.float32)
    score = np.zeros(ts.P, np.float32)
    for c, i in enumerate(ids):
        pred = to_np(renders[2 * c]["out_color"]).reshape(3, HW)
        _, ploss = dor.metric_map(pred, to_np(targets[i]), dcfg.loss_thresh)
        counts, score = dor.score_accumulate(counts, score, to_np(renders[2 * c + 1]["metric_count"]),
                                             ploss)
    want_imp, want_prn = dor.score_finalize(counts, score, len(ids))
    imp_np, prn_np = to_np(imp), to_np(prn)
    np.testing.assert_array_equal(imp_np, want_imp)
    np.testing.assert_allclose(prn_np, want_prn, rtol=1e-5, atol=1e-6)

    model = {n: to_np(ts.param(n)).copy() for n in PARAM_NAMES}
    adam = {n: tuple(to_np(x).reshape(model[n].shape).copy() for x in ts.moments(n))
            for n in PARAM_NAMES}
    st = {n: to_np(ts.stat(n)).copy() for n in STAT_NAMES}
    st["tmp_radii"] = to_np(ts.tmp_radii()).copy()
    cf, sf = dor.classify(dcfg, extent, st, model["log_scales"], imp_np)
    nc, ns = int(cf.sum()), int(sf.sum())
    draws = np.random.default_rng(7)
    normals = draws.normal(0, 1, (ns * dcfg.split_factor, 3)).astype(np.float32)
    P2 = ts.P - ns + nc + ns * dcfg.split_factor
    uniforms = draws.random(P2).astype(np.float32)
    _say(f"cfg5 densify event: P={ts.P} clones={nc} splits={ns}")
    nm, na, nst, info = dor.densify_and_prune(dcfg, extent, model, adam, st, imp_np, prn_np,
                                              normals, uniforms)
    got = ts.densify_and_prune_fastgs(dcfg, extent, imp, torch.from_numpy(prn_np).cuda(),
                                      normals=torch.from_numpy(normals).cuda(),
                                      uniforms=torch.from_numpy(uniforms).cuda())
    for k in ("cloned", "split_sources", "split_children", "total_prune_candidates",
              "prune_budget", "actual_removed", "points"):
        assert got[k] == info[k], (k, got[k], info[k])
    assert info["cloned"] + info["split_sources"] > 0
    for n in PARAM_NAMES:
        g = to_np(ts.param(n))
        np.testing.assert_array_equal(g.view(np.uint32),
                                      np.asarray(nm[n], np.float32).reshape(g.shape).view(np.uint32),
                                      err_msg=n)
        m, v = ts.moments(n)
        np.testing.assert_array_equal(to_np(m).reshape(g.shape), na[n][0].reshape(g.shape))
        np.testing.assert_array_equal(to_np(v).reshape(g.shape), na[n][1].reshape(g.shape))
    for n in STAT_NAMES:
        np.testing.assert_array_equal(to_np(ts.stat(n)), nst[n], err_msg=n)
    np.testing.assert_array_equal(to_np(ts.tmp_radii()), nst["tmp_radii"])
