"""The preprocess in two halves (fgs_preprocess_geometry_fwd, then
fgs_preprocess_colour_fwd on a side stream; no reference counterpart) against
the fused kernel of fgs_preprocess_fwd: the two halves run the same device
code, so every output is bit-identical, for each SH degree, for precomputed
colours and for the raw parameters of a training step; and a whole frame of
rasterize_gaussians renders the same bits either way."""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

from tests.helpers import to_torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-test]", *a, flush=True)


def _preprocess(torch, rasterizer, d, cam, degree, split):
    old = rasterizer.SPLIT_COLOUR
    rasterizer.SPLIT_COLOUR = split
    try:
        outs, cfg, dev = rasterizer._run_preprocess(
            d, "rasterize_gaussians_forward", rasterizer._RG_NAMES, cam.width, cam.height, 16, 16,
            cam.tan_fovx, cam.tan_fovy, degree, 1.0, 1.0, default_vsp=True, st_records=True)
        assert bool(cfg["split_colour"]) == split
        rasterizer._join_colour(cfg, dev)
        torch.cuda.synchronize()
        return [t.detach().cpu().numpy() for t in outs]
    finally:
        rasterizer.SPLIT_COLOUR = old


@pytest.mark.parametrize("mode", ["sh0", "sh1", "sh2", "sh3", "precomp", "raw"])
def test_split_preprocess_is_bit_exact(mode):
    import torch

    from fastgs_core_amd import rasterizer

    degree = {"sh0": 0, "sh1": 1, "sh2": 2, "sh3": 3}.get(mode, 3)
    P = 40000
    sc = syn.scene_config2(11, P, degree)
    cam = syn.sphere_cameras(4, 3, 320, 240)[2]
    inp = syn.make_inputs(sc, cam)
    rng = np.random.default_rng(5)
    if mode == "precomp":
        inp = {k: v for k, v in inp.items() if k not in ("dc", "sh")}
        inp["colors_precomp"] = rng.uniform(0, 1, (P, 3)).astype(np.float32)
    d = to_torch(inp)
    if mode == "raw":
        opac = np.clip(inp["opacities"].astype(np.float64), 1e-6, 1 - 1e-6).reshape(-1)
        for k in ("scales", "rotations", "opacities"):
            d.pop(k)
        d["log_scales"] = torch.from_numpy(np.log(inp["scales"]).astype(np.float32)).cuda()
        d["raw_rotations"] = torch.from_numpy(
            (inp["rotations"] * rng.uniform(0.5, 2.0, (P, 1))).astype(np.float32)).cuda()
        d["opacity_logits"] = torch.from_numpy(np.log(opac / (1 - opac)).astype(np.float32)).cuda()
    _say("split preprocess", mode)
    fused = _preprocess(torch, rasterizer, d, cam, degree, False)
    split = _preprocess(torch, rasterizer, d, cam, degree, True)
    assert int((fused[0] > 0).sum()) > 1000 and int((fused[0] == 0).sum()) > 0
    for i, (a, b) in enumerate(zip(fused, split)):
        np.testing.assert_array_equal(a, b, err_msg=f"preprocess output {i} ({mode})")


def test_split_preprocess_whole_frame():
    import torch

    import fastgs_core
    from fastgs_core_amd import rasterizer

    degree = 3
    sc = syn.scene_config2(12, 60000, degree)
    cam = syn.sphere_cameras(4, 2, 480, 272)[1]
    inp = syn.make_inputs(sc, cam)
    _say("split preprocess, whole frame")
    res = []
    old = rasterizer.SPLIT_COLOUR
    try:
        for split in (False, True):
            rasterizer.SPLIT_COLOUR = split
            out = fastgs_core.rasterize_gaussians(to_torch(inp), cam.width, cam.height, 16, 16,
                                                  cam.tan_fovx, cam.tan_fovy, degree)
            torch.cuda.synchronize()
            res.append(out)
    finally:
        rasterizer.SPLIT_COLOUR = old
    a, b = res
    assert a["rendered"] == b["rendered"] > 0
    for k, v in a.items():
        if torch.is_tensor(v):
            np.testing.assert_array_equal(v.cpu().numpy(), b[k].cpu().numpy(), err_msg=k)
