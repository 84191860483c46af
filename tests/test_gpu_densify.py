"""GPU densification and pruning (csrc/fgs_densify.hip through
fastgs_core_amd.densify) against the oracle restatement of
scripts/train_scanner_fastgs.py (oracle/densify.py): every parameter, Adam
moment and statistics row bit for bit, given the same random draws."""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn
from fastgs_core_amd.densify import PARAM_NAMES, STAT_NAMES, DensifyConfig

from helpers import scene_small

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dor():
    from oracle.densify import DensifyOracle

    return DensifyOracle()


def _say(*a):
    print("[gpu-test] densify", *a, flush=True)


def _model(rng, P, M=3):
    return {
        "means3d": rng.normal(0, 1, (P, 3)).astype(np.float32),
        "features_dc": rng.uniform(0, 1, (P, 3)).astype(np.float32),
        "features_rest": rng.normal(0, 0.05, (P, M, 3)).astype(np.float32),
        "opacity_logits": rng.normal(-1, 2.5, (P, 1)).astype(np.float32),
        "log_scales": rng.normal(-3.5, 1.0, (P, 3)).astype(np.float32),
        "rotations": rng.normal(0, 1, (P, 4)).astype(np.float32),
    }


def _state_for(rng, model, with_stats=True):
    import torch

    from fastgs_core_amd.densify import GaussianTrainState

    dev = torch.device("cuda")
    ts = GaussianTrainState({k: torch.from_numpy(v).to(dev) for k, v in model.items()})
    P = len(model["means3d"])
    adam = {}
    for n in PARAM_NAMES:
        m, v = ts.moments(n)
        mm = rng.normal(0, 1, m.numel()).astype(np.float32)
        vv = rng.uniform(0, 1, v.numel()).astype(np.float32)
        m.copy_(torch.from_numpy(mm))
        v.copy_(torch.from_numpy(vv))
        adam[n] = (mm.reshape(model[n].shape), vv.reshape(model[n].shape))
    st = {"max_radii2d": rng.uniform(0, 40, P).astype(np.float32),
          "grad_accum": rng.uniform(0, 4e-3, P).astype(np.float32),
          "grad_accum_abs": rng.uniform(0, 2e-2, P).astype(np.float32),
          "denom": rng.integers(0, 8, P).astype(np.float32),
          "tmp_radii": rng.integers(0, 30, P).astype(np.int32)}
    for n in STAT_NAMES:
        ts.stat(n).copy_(torch.from_numpy(st[n]))
    ts.tmp_radii().copy_(torch.from_numpy(st["tmp_radii"]))
    return ts, adam, st


def _np(t):
    return t.detach().cpu().numpy()


def _assert_state_equal(ts, nm, na, ns):
    for n in PARAM_NAMES:
        got = _np(ts.param(n))
        np.testing.assert_array_equal(got.view(np.uint32), np.asarray(nm[n], np.float32)
                                      .reshape(got.shape).view(np.uint32), err_msg=n)
        m, v = ts.moments(n)
        np.testing.assert_array_equal(_np(m).reshape(got.shape), na[n][0].reshape(got.shape),
                                      err_msg="m " + n)
        np.testing.assert_array_equal(_np(v).reshape(got.shape), na[n][1].reshape(got.shape),
                                      err_msg="v " + n)
    for n in STAT_NAMES:
        np.testing.assert_array_equal(_np(ts.stat(n)), ns[n], err_msg=n)
    np.testing.assert_array_equal(_np(ts.tmp_radii()), ns["tmp_radii"])


def test_stats_update_matches_oracle(dor):
    import torch

    _say("stats")
    rng = np.random.default_rng(0)
    P = 5001
    ts, adam, st = _state_for(rng, _model(rng, P))
    radii = rng.integers(-2, 40, P).astype(np.int32)
    g = rng.normal(0, 1e-3, (P, 4)).astype(np.float32)
    ts.update_densification_stats(torch.from_numpy(radii).cuda(), torch.from_numpy(g).cuda())
    want = dor.update_stats(dict(st), radii, g)
    for n in STAT_NAMES:
        np.testing.assert_array_equal(_np(ts.stat(n)), want[n], err_msg=n)
    np.testing.assert_array_equal(_np(ts.tmp_radii()), radii)


@pytest.mark.parametrize("case", ["clone_split_prune", "no_append", "no_scores"])
def test_densify_and_prune_matches_oracle(dor, case):
    import torch

    _say(case)
    rng = np.random.default_rng({"clone_split_prune": 1, "no_append": 2, "no_scores": 3}[case])
    P = 4000
    model = _model(rng, P)
    ts, adam, st = _state_for(rng, model)
    cfg = DensifyConfig()
    ext = 3.0
    imp = rng.integers(0, 12, P).astype(np.float32)
    if case == "no_append":
        imp[:] = 0.0  # no metric hits: nothing cloned or split, screen pruning active
    prn = rng.uniform(0, 1, P).astype(np.float32) if case != "no_scores" else None
    cf, sf = dor.classify(cfg, ext, st, model["log_scales"], imp)
    nc, ns = int(cf.sum()), int(sf.sum())
    normals = rng.normal(0, 1, (ns * cfg.split_factor, 3)).astype(np.float32)
    P2 = P - ns + nc + ns * cfg.split_factor
    uniforms = rng.random(P2).astype(np.float32)
    nm, na, nst, info = dor.densify_and_prune(cfg, ext, model, adam, st, imp, prn, normals,
                                              uniforms)
    got = ts.densify_and_prune_fastgs(
        cfg, ext, torch.from_numpy(imp).cuda(),
        torch.from_numpy(prn).cuda() if prn is not None else None,
        normals=torch.from_numpy(normals).cuda(), uniforms=torch.from_numpy(uniforms).cuda())
    for k in ("cloned", "split_sources", "split_children", "total_prune_candidates",
              "prune_budget", "actual_removed", "points"):
        assert got[k] == info[k], (k, got[k], info[k])
    if case == "clone_split_prune":
        assert nc > 0 and ns > 0 and info["actual_removed"] > 0
    if case == "no_append":
        assert nc == 0 and ns == 0 and info["actual_removed"] > 0
    assert ts.P == info["points"]
    _assert_state_equal(ts, nm, na, nst)


@pytest.mark.parametrize("branch", ["min_keep", "mask"])
def test_final_prune_matches_oracle(dor, branch):
    import torch

    _say("final prune", branch)
    rng = np.random.default_rng(11)
    P = 3000
    model = _model(rng, P)
    ts, adam, st = _state_for(rng, model)
    prn = rng.uniform(0, 1, P).astype(np.float32)
    args = (0.99, prn, 0.0, 500) if branch == "min_keep" else (0.05, prn, 0.8, 64)
    nm, na, nst, info = dor.final_prune(model, adam, st, *args)
    got = ts.final_prune_fastgs(args[0], torch.from_numpy(prn).cuda(), args[2], args[3])
    assert got["kept"] == info["kept"] == ts.P
    if branch == "min_keep":
        assert info["kept"] == 500
    _assert_state_equal(ts, nm, na, nst)


def test_opacity_cap_matches_oracle(dor):
    _say("opacity cap")
    rng = np.random.default_rng(12)
    P = 2000
    model = _model(rng, P)
    ts, adam, st = _state_for(rng, model)
    ts.cap_opacity_logits(0.82)
    want = dor.opacity_cap(model["opacity_logits"], 0.82)
    np.testing.assert_array_equal(_np(ts.param("opacity_logits")).reshape(-1), want)
    m, v = ts.moments("opacity_logits")
    assert not _np(m).any() and not _np(v).any()


def _scene_state(seed, P, W, H):
    import torch

    from fastgs_core_amd.densify import GaussianTrainState

    sc, cam = scene_small(seed, P, 3, W, H)
    dev = torch.device("cuda")
    rng = np.random.default_rng(seed)
    q = sc["rotations"]
    params = {
        "means3d": torch.from_numpy(sc["means3d"]).to(dev),
        "features_dc": torch.from_numpy(sc["dc"]).to(dev),
        "features_rest": torch.from_numpy(sc["sh"]).to(dev),
        "opacity_logits": torch.from_numpy(np.log(sc["opacities"] / (1 - sc["opacities"]))
                                           .astype(np.float32).reshape(-1, 1)).to(dev),
        "log_scales": torch.from_numpy(np.log(sc["scales"]).astype(np.float32)).to(dev),
        "rotations": torch.from_numpy(q).to(dev),
    }
    return GaussianTrainState(params), sc, cam, rng


def test_scores_match_oracle(dor):
    import torch

    import fastgs_core

    _say("scores")
    ts, sc, cam, rng = _scene_state(21, 2500, 128, 96)
    inp = syn.make_inputs(sc, cam)
    cam_in = {k: torch.from_numpy(np.ascontiguousarray(inp[k])).cuda()
              for k in ("viewmatrix", "projmatrix", "campos", "background")}
    HW = cam.width * cam.height
    target = torch.from_numpy(rng.uniform(0, 1, (3, HW)).astype(np.float32)).cuda()
    renders = []

    def render(idx, metric_map):
        d = ts.render_inputs(cam_in)
        d["metric_map"] = metric_map if metric_map is not None else \
            torch.zeros(HW, dtype=torch.int32, device="cuda")
        out = fastgs_core.rasterize_gaussians(d, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                              cam.tan_fovy, 3, get_flag=metric_map is not None)
        renders.append(out)
        return out

    imp, prn = ts.compute_gaussian_scores_fastgs(render, [target, target], [0, 1], 0.06, True)
    counts = np.zeros(ts.P, np.float32)
    score = np.zeros(ts.P, np.float32)
    for c in range(2):
        pred = _np(renders[2 * c]["out_color"])
        mm, loss = dor.metric_map(pred, _np(target), 0.06)
        mc = _np(renders[2 * c + 1]["metric_count"])
        counts, score = dor.score_accumulate(counts, score, mc, loss)
    want_imp, want_prn = dor.score_finalize(counts, score, 2)
    np.testing.assert_array_equal(_np(imp), want_imp)
    np.testing.assert_allclose(_np(prn), want_prn, rtol=1e-5, atol=1e-6)


def test_growth_reallocates_and_training_continues():
    """Repeated densification grows the set past its capacity; parameters,
    moments and a training step stay consistent after each rebuild."""
    import torch

    import fastgs_core

    _say("growth")
    ts, sc, cam, rng = _scene_state(22, 1500, 96, 80)
    inp = syn.make_inputs(sc, cam)
    cam_in = {k: torch.from_numpy(np.ascontiguousarray(inp[k])).cuda()
              for k in ("viewmatrix", "projmatrix", "campos", "background")}
    HW = cam.width * cam.height
    target = torch.rand(3, HW, device="cuda")
    cfg = DensifyConfig(min_opacity=0.0, max_screen_size=0.0, max_world_scale_factor=0.0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    sizes = [ts.P]
    for it in range(1, 7):
        d = ts.render_inputs(cam_in)
        d["metric_map"] = torch.zeros(HW, dtype=torch.int32, device="cuda")
        vsp = torch.zeros((ts.P, 4), device="cuda", requires_grad=True)
        d["viewspace_points"] = vsp
        out = fastgs_core.rasterize_gaussians(d, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                              cam.tan_fovy, 3)
        loss = (out["out_color"] - target).abs().mean()
        ts.zero_grad()
        loss.backward()
        ts.update_densification_stats(out["radii"], vsp.grad)
        ts.update_learning_rate(it)
        ts.step(it)
        # clone every row with any gradient: importance above the threshold
        imp = torch.full((ts.P,), 10.0, device="cuda")
        cfg.grad_thresh = 0.0
        cfg.grad_abs_thresh = 0.0
        before = ts.P
        info = ts.densify_and_prune_fastgs(cfg, 1.0, imp, None, generator=gen)
        assert ts.P == before + info["cloned"] + info["split_children"] - info["split_sources"]
        sizes.append(ts.P)
        for n in PARAM_NAMES:
            assert ts.param(n).shape[0] == ts.P and torch.isfinite(ts.param(n)).all(), n
    assert sizes[-1] > 4 * sizes[0] and ts.reallocations >= 2
