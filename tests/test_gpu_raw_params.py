"""rasterize_gaussians with the raw parameters of a training step (log_scales,
raw_rotations, opacity_logits; no reference counterpart) against the
reference-keyed call on the activated parameters (fastgs_core_amd.activate).

* The preprocess with the same upstream gradients: every forward output and
  every gradient of the raw tensors bit-identical, so the activation backward
  fused into the preprocess backward computes exactly what
  fgs_activations_bwd does (the preprocess has no atomics: same inputs, same
  bits).
* The whole frame: forward outputs bit-identical; the raw gradients agree up
  to the order of the rasterize backward's float atomics (which differs from
  run to run), within 1e-4 of each tensor's largest entry.
"""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[gpu-test]", *a, flush=True)


def _scene(degree, P=30000, W=320, H=240):
    sc = syn.scene_config2(5, P, degree)
    cam = syn.sphere_cameras(3, 2, W, H)[1]
    inp = syn.make_inputs(sc, cam)
    rng = np.random.default_rng(3)
    opac = np.clip(inp["opacities"].astype(np.float64), 1e-6, 1 - 1e-6)
    raw = {"log_scales": np.log(inp["scales"]).astype(np.float32),
           "quats": (inp["rotations"] * rng.uniform(0.5, 2.0, (P, 1))).astype(np.float32),
           "logits": np.log(opac / (1 - opac)).astype(np.float32).reshape(-1)}
    return inp, raw, cam, rng


def _inputs(torch, inp, raw, fused, dev):
    import fastgs_core_amd

    base = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
            for k, v in inp.items() if k not in ("scales", "rotations", "opacities")}
    leaves = {k: torch.from_numpy(v.copy()).to(dev).requires_grad_(True) for k, v in raw.items()}
    means = base["means3d"].clone().requires_grad_(True)
    vsp = torch.zeros((means.shape[0], 4), device=dev, requires_grad=True)
    d = dict(base, means3d=means, viewspace_points=vsp)
    if fused:
        d.update(log_scales=leaves["log_scales"], raw_rotations=leaves["quats"],
                 opacity_logits=leaves["logits"])
    else:
        s, r, o = fastgs_core_amd.activate(leaves["log_scales"], leaves["quats"], leaves["logits"])
        d.update(scales=s, rotations=r, opacities=o)
    return d, leaves, means, vsp


@pytest.mark.parametrize("degree", [0, 3])
def test_fused_activation_backward_is_bit_exact(degree):
    import torch

    from fastgs_core_amd import rasterizer

    inp, raw, cam, rng = _scene(degree)
    dev = torch.device("cuda")
    W, H = cam.width, cam.height
    P = inp["means3d"].shape[0]
    g = {"xys": rng.standard_normal((P, 2)), "rgb": rng.standard_normal((P, 3)),
         "conic": rng.standard_normal((P, 4)), "vsp": rng.standard_normal((P, 4))}
    g = {k: torch.from_numpy(v.astype(np.float32)).to(dev) for k, v in g.items()}
    _say("fused activation backward, degree", degree)
    res = []
    for fused in (False, True):
        d, leaves, means, vsp = _inputs(torch, inp, raw, fused, dev)
        outs, cfg, _ = rasterizer._run_preprocess(
            d, "rasterize_gaussians_forward", rasterizer._RG_NAMES, W, H, 16, 16, cam.tan_fovx,
            cam.tan_fovy, degree, 1.0, 1.0, default_vsp=True)
        assert bool(cfg["raw"]) == fused
        radii, xys, depths, cov3d, rgb, conic, tiles, clamped, vsp_out = outs
        torch.autograd.backward([xys, rgb, conic, vsp_out], [g["xys"], g["rgb"], g["conic"], g["vsp"]])
        torch.cuda.synchronize()
        grads = {k: v.grad.cpu().numpy() for k, v in leaves.items()}
        grads["means3d"] = means.grad.cpu().numpy()
        grads["viewspace"] = vsp.grad.cpu().numpy()
        res.append(([t.detach().cpu().numpy() for t in outs], grads))
    (o_a, g_a), (o_b, g_b) = res
    for i, (a, b) in enumerate(zip(o_a, o_b)):
        np.testing.assert_array_equal(a, b, err_msg=f"preprocess output {i}")
    assert int((o_a[0] > 0).sum()) > 1000
    for k in g_a:
        np.testing.assert_array_equal(g_a[k], g_b[k], err_msg=k)
        assert np.isfinite(g_a[k]).all() and np.abs(g_a[k]).max() > 0, k


def test_raw_parameters_whole_frame():
    import torch

    import fastgs_core

    degree = 3
    inp, raw, cam, rng = _scene(degree)
    dev = torch.device("cuda")
    W, H = cam.width, cam.height
    dL = torch.from_numpy(rng.standard_normal((3, H * W)).astype(np.float32)).to(dev)
    _say("raw parameters, whole frame")
    res = []
    for fused in (False, True):
        d, leaves, means, vsp = _inputs(torch, inp, raw, fused, dev)
        out = fastgs_core.rasterize_gaussians(d, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, degree)
        (out["out_color"] * dL).sum().backward()
        torch.cuda.synchronize()
        grads = {k: v.grad.cpu().numpy() for k, v in leaves.items()}
        grads["means3d"] = means.grad.cpu().numpy()
        res.append((out, grads))
    (out_a, g_a), (out_b, g_b) = res
    assert out_a["rendered"] == out_b["rendered"] > 0
    for k, v in out_a.items():
        if torch.is_tensor(v):
            np.testing.assert_array_equal(v.detach().cpu().numpy(),
                                          out_b[k].detach().cpu().numpy(), err_msg=k)
    for k in g_a:
        scale = np.abs(g_a[k]).max()
        assert scale > 0, k
        np.testing.assert_allclose(g_b[k], g_a[k], rtol=0, atol=1e-4 * scale, err_msg=k)
