"""BASELINE.json configs[0], [1], [3] and [4] at their stated sizes, against the
oracle on the same seeded inputs (configs[2], cfg3, is test_gpu_fullsize.py).

* cfg1 (plumbing): 16,384 Gaussians at 256x256, SH 0, one forward render and
  the backward of an L1 loss against a seeded U(0,1) target.
* cfg2: 200,000 Gaussians at 1280x720, SH 3, forward-only, all eight seeded
  poses.
* cfg4 (heavy-overlap stress): 3,000,000 Gaussians at 1920x1080, SH 3, 2 % of
  them large (about 1.9e8 tile duplicates, the largest touching all 8,160
  tiles), forward and backward.
* cfg5 (densification loop): 100,000 Gaussians from the reference's initial
  model at 1280x720, trained for its 500 iterations against targets rendered
  from a hidden 300k scene; the scores and each of the five densify-and-prune
  events against the densification oracle on the same random draws, then a
  sixth event with thresholds that split and prune.

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


@pytest.mark.parametrize("pose", list(range(8)))
def test_cfg2_forward_poses(oracle, pose):
    """200,000 Gaussians, 1280x720, SH 3, forward only; each of the
    bench's eight seeded sphere cameras."""
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


def _snapshot(ts):
    from fastgs_core_amd.densify import PARAM_NAMES, STAT_NAMES

    model = {n: to_np(ts.param(n)).copy() for n in PARAM_NAMES}
    adam = {n: tuple(to_np(x).reshape(model[n].shape).copy() for x in ts.moments(n))
            for n in PARAM_NAMES}
    st = {n: to_np(ts.stat(n)).copy() for n in STAT_NAMES}
    st["tmp_radii"] = to_np(ts.tmp_radii()).copy()
    return model, adam, st


def _check_event(ts, loop, dor, dcfg, it, targets, HW, draws):
    """One densification event of the loop against the oracles: the scores
    over the sampled cameras from the GPU renders, then densify_and_prune_fastgs
    on the same draws -- every row, Adam moment and statistic bit-exact."""
    import torch

    from fastgs_core_amd.densify import PARAM_NAMES, STAT_NAMES

    renders = []
    ids = loop.sample_cameras()
    imp, prn = loop.scores(it, ids, True, on_render=renders.append)
    counts = np.zeros(ts.P, np.float32)
    score = np.zeros(ts.P, np.float32)
    for c, i in enumerate(ids):
        pred = to_np(renders[2 * c]["out_color"]).reshape(3, HW)
        _, ploss = dor.metric_map(pred, to_np(targets[i]), dcfg.loss_thresh)
        counts, score = dor.score_accumulate(counts, score,
                                             to_np(renders[2 * c + 1]["metric_count"]), ploss)
    want_imp, want_prn = dor.score_finalize(counts, score, len(ids))
    imp_np, prn_np = to_np(imp), to_np(prn)
    np.testing.assert_array_equal(imp_np, want_imp)
    np.testing.assert_allclose(prn_np, want_prn, rtol=1e-5, atol=1e-6)
    model, adam, st = _snapshot(ts)
    cf, sf = dor.classify(dcfg, loop.extent, st, model["log_scales"], imp_np)
    nc, ns = int(cf.sum()), int(sf.sum())
    normals = draws.normal(0, 1, (ns * dcfg.split_factor, 3)).astype(np.float32)
    uniforms = draws.random(ts.P - ns + nc + ns * dcfg.split_factor).astype(np.float32)
    nm, na, nst, info = dor.densify_and_prune(dcfg, loop.extent, model, adam, st, imp_np, prn_np,
                                              normals, uniforms)
    got = ts.densify_and_prune_fastgs(dcfg, loop.extent, imp, torch.from_numpy(prn_np).cuda(),
                                      normals=torch.from_numpy(normals).cuda(),
                                      uniforms=torch.from_numpy(uniforms).cuda())
    _say(f"cfg5 event it={it}:", {k: got[k] for k in ("cloned", "split_sources",
                                                      "total_prune_candidates", "actual_removed",
                                                      "points")})
    for k in ("cloned", "split_sources", "split_children", "total_prune_candidates",
              "prune_budget", "actual_removed", "points"):
        assert got[k] == info[k], (it, k, got[k], info[k])
    for n in PARAM_NAMES:
        g = to_np(ts.param(n))
        np.testing.assert_array_equal(g.view(np.uint32),
                                      np.asarray(nm[n], np.float32).reshape(g.shape).view(np.uint32),
                                      err_msg=f"it {it} {n}")
        m, v = ts.moments(n)
        np.testing.assert_array_equal(to_np(m).reshape(g.shape), na[n][0].reshape(g.shape))
        np.testing.assert_array_equal(to_np(v).reshape(g.shape), na[n][1].reshape(g.shape))
    for n in STAT_NAMES:
        np.testing.assert_array_equal(to_np(ts.stat(n)), nst[n], err_msg=f"it {it} {n}")
    np.testing.assert_array_equal(to_np(ts.tmp_radii()), nst["tmp_radii"])
    return got


@pytest.mark.timeout(900)
def test_cfg5_full_schedule_at_size(oracle):
    """configs[4] through its whole schedule: the reference's initial model of
    100,000 points at 1280x720, 500 iterations of the FastGS loop
    (train_scanner_fastgs.py:968-1060: one sphere camera per iteration, MSE
    against targets of a hidden 300k scene, the Adam cadence, the statistics
    from the viewspace gradients and the post-step statistics render of
    :1014-1019), a densification event every 100 iterations -- all five
    checked against the densification oracle on the same draws, scores
    included -- then, after 50 more iterations, one more event at the same
    size with thresholds that split and prune (densify_and_split_fastgs :567-587 and the budgeted prune
    draw :700-723 at size).  On three iterations the statistics render is
    checked against the oracle: its radii are the oracle's preprocess radii
    of the post-step parameters, and the statistics update is the oracle's."""
    import dataclasses

    import torch

    import fastgs_core
    from fastgs_core_amd.densify import (DensifyConfig, FastGSTrainLoop, GaussianTrainState,
                                         LoopConfig, STAT_NAMES, compute_scene_extent)
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
    dcfg = DensifyConfig()
    lcfg = LoopConfig(interval=100, densify_from=0, stats_render="post_step")
    def radii(ts, idx):
        c = cams[idx]
        return ts.preprocess_radii(cam_in[idx], W, H, c.tan_fovx, c.tan_fovy)

    loop = FastGSTrainLoop(ts, render, targets, len(cams), 3, dcfg, lcfg,
                           compute_scene_extent(ts.param("means3d").detach()), seed=42,
                           radii=radii)
    dor = DensifyOracle()
    draws = np.random.default_rng(7)
    events = []
    radii_moved = 0
    for it in range(1, 501):
        check = it in (1, 137, 333)
        if check:
            _, _, st0 = _snapshot(ts)
        loss, idx = loop.train_iteration(it)
        if check:
            radii, dvsp = loop.last_stats
            d = ts.render_inputs(cam_in[idx])
            c = cams[idx]
            kw = dict(dc=to_np(d["dc"]), sh=to_np(d["sh"]), scales=to_np(d["scales"]),
                      rotations=to_np(d["rotations"]))
            pre = oracle.preprocess_fwd(to_np(d["means3d"]), to_np(d["opacities"]),
                                        c.viewmatrix.reshape(-1), c.projmatrix.reshape(-1),
                                        c.campos, np.zeros((ts.P, 4), np.float32), W, H,
                                        c.tan_fovx, c.tan_fovy, 0, **kw)
            np.testing.assert_array_equal(to_np(radii), pre["radii"], err_msg=f"it {it} radii")
            # the preprocess-only radii are those of a full render of the camera
            with torch.no_grad():
                full = render(ts, idx, loop.active_degree(it))["radii"]
            np.testing.assert_array_equal(to_np(radii), to_np(full), err_msg=f"it {it} full")
            want = dor.update_stats(dict(st0), to_np(radii), to_np(dvsp))
            for n in STAT_NAMES:
                np.testing.assert_array_equal(to_np(ts.stat(n)), want[n], err_msg=f"it {it} {n}")
            _say(f"cfg5 it={it}: statistics render checked, loss {float(loss):.5f}")
        if loop.is_densify_event(it):
            events.append(_check_event(ts, loop, dor, dcfg, it, targets, HW, draws))
        loop.after_iteration(it)
    assert np.isfinite(float(loss))
    assert len(events) == 5
    assert sum(e["cloned"] + e["split_sources"] for e in events) > 0
    # 50 more iterations refill the statistics (the event of iteration 500
    # reset them), then one more event at this size with thresholds that
    # split and prune: rows above 0.05 % of the extent split when their mean
    # |viewspace gradient| passes 2e-4; the prune thresholds come from the
    # state itself (training moves every opacity above the initial 0.1): the
    # 5 % quantile of the opacities and 1.5x the median largest world scale
    for it in range(501, 551):
        loop.train_iteration(it)
    model, _, _ = _snapshot(ts)
    opac = 1.0 / (1.0 + np.exp(-model["opacity_logits"].astype(np.float64).reshape(-1)))
    big = np.exp(model["log_scales"].astype(np.float64)).max(1)
    forced = dataclasses.replace(dcfg, dense=0.0005, grad_abs_thresh=2.0e-4,
                                 min_opacity=float(np.quantile(opac, 0.05)),
                                 max_world_scale_factor=float(1.5 * np.median(big) / loop.extent))
    got = _check_event(ts, loop, dor, forced, 550, targets, HW, draws)
    assert got["split_sources"] > 0 and got["total_prune_candidates"] > 0
    assert got["actual_removed"] > 0
