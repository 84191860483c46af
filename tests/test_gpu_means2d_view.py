"""The rasterize backward hands dL/dmeans2d on as a view of dL/dviewspace
(its first two components; fgs_raster_bwd_io.dL_dmeans2d = NULL) and the
preprocess backward reads it with its row stride
(fgs_preprocess_bwd_io.dL_dxys_stride = 4); no reference counterpart.
- The preprocess backward given one cotangent of the projected means as that
  strided view and as a contiguous copy returns bit-identical gradients (it
  has no atomics, so the two runs are comparable bit for bit).
- A training step with the view and with the copy agrees up to the order of
  the rasterize backward's float atomic adds, also when the projected means
  (geom_means2d) receive a gradient of their own, which autograd sums into a
  new contiguous tensor (stride 2)."""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

from tests.helpers import to_torch

pytestmark = pytest.mark.gpu

REQ = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")


def _say(*a):
    print("[gpu-test]", *a, flush=True)


def _scene(torch):
    import fastgs_core

    sc = syn.scene_config2(21, 30000, 3)
    cam = syn.sphere_cameras(4, 1, 256, 192)[0]
    tin = to_torch(syn.make_inputs(sc, cam), requires_grad=REQ)
    out = fastgs_core.rasterize_gaussians(tin, cam.width, cam.height, 16, 16, cam.tan_fovx,
                                          cam.tan_fovy, 3)
    return cam, tin, out


def test_preprocess_backward_reads_the_strided_xy_cotangent():
    import torch

    _say("preprocess backward: strided vs contiguous xy cotangent")
    _, tin, out = _scene(torch)
    xys = out["geom_means2d"]
    P = xys.shape[0]
    rng = np.random.default_rng(4)
    gv = torch.from_numpy(rng.standard_normal((P, 4)).astype(np.float32)).cuda()
    view = gv[:, :2]
    assert view.stride() == (4, 1)
    params = [tin[k] for k in REQ[:-1]]
    g_view = torch.autograd.grad(xys, params, grad_outputs=view, retain_graph=True,
                                 allow_unused=True)
    g_copy = torch.autograd.grad(xys, params, grad_outputs=view.contiguous(), retain_graph=True,
                                 allow_unused=True)
    torch.cuda.synchronize()
    assert g_view[0] is not None and float(g_view[0].abs().max()) > 0
    for k, a, b in zip(REQ, g_view, g_copy):
        if a is None or b is None:
            assert a is None and b is None, k
            continue
        np.testing.assert_array_equal(a.cpu().numpy(), b.cpu().numpy(), err_msg=k)


def _step(torch, view, extra):
    from fastgs_core_amd import rasterizer

    old = rasterizer.MEANS2D_GRAD_VIEW
    rasterizer.MEANS2D_GRAD_VIEW = view
    try:
        cam, tin, out = _scene(torch)
        rng = np.random.default_rng(3)
        dL = torch.from_numpy(
            rng.standard_normal((3, cam.width * cam.height)).astype(np.float32)).cuda()
        loss = (out["out_color"] * dL).sum()
        if extra:
            loss = loss + 1e-3 * out["geom_means2d"].square().sum()
        loss.backward()
        torch.cuda.synchronize()
        return {k: tin[k].grad.detach().cpu().numpy().astype(np.float64) for k in REQ}
    finally:
        rasterizer.MEANS2D_GRAD_VIEW = old


@pytest.mark.parametrize("extra", [False, True])
def test_training_step_with_the_view_matches_the_copy(extra):
    import torch

    _say("training step, means2d gradient view vs copy, extra xy gradient:", extra)
    copy = _step(torch, False, extra)
    view = _step(torch, True, extra)
    for k in REQ:
        scale = np.abs(copy[k]).max()
        assert scale > 0, k
        # the two steps differ only in the order of float atomic adds
        np.testing.assert_allclose(view[k], copy[k], rtol=1e-4, atol=1e-5 * scale, err_msg=k)
