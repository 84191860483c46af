"""Launch events (fgs_set_launch_events): the library records the caller's
events directly around the main kernel of each stage, so the kernel's time is
positive, inside the time of its whole entry point, and the events stop being
recorded once cleared."""
import numpy as np
import pytest

from fastgs_core_amd import _lib
from fastgs_core_amd import synthetic as syn

from tests.helpers import to_torch

pytestmark = pytest.mark.gpu

NAMES = ("preprocess_fwd", "rasterize_fwd", "rasterize_bwd", "preprocess_bwd", "loss_fwd",
         "loss_bwd", "preprocess_colour")


def test_launch_events_bracket_the_main_kernels():
    import torch

    import fastgs_core
    import fastgs_core_amd
    from fastgs_core_amd import rasterizer

    assert rasterizer.SPLIT_COLOUR  # the colour kernel runs (on the side stream)

    lib = _lib.load()
    W, H = 256, 192
    sc = syn.scene_config2(3, 20000, 3)
    cam = syn.sphere_cameras(4, 1, W, H)[0]
    inp = syn.make_inputs(sc, cam)
    req = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")
    tgt = torch.rand(3, H, W, device="cuda")

    def run():
        tin = to_torch(inp, requires_grad=req)
        out = fastgs_core.rasterize_gaussians(tin, W, H, 16, 16, cam.tan_fovx, cam.tan_fovy, 3)
        loss = fastgs_core_amd.l1_ssim_loss(out["out_color"].view(3, H, W), tgt)
        loss.backward()
        return out

    run()  # warm-up
    torch.cuda.synchronize()
    ev = {}
    for n in NAMES:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        b.record()
        assert lib.fgs_set_launch_events(n.encode(), a.cuda_event, b.cuda_event) == 0
        ev[n] = (a, b)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    try:
        t0.record()
        out = run()
        t1.record()
    finally:
        for n in NAMES:
            lib.fgs_set_launch_events(n.encode(), None, None)
    torch.cuda.synchronize()
    assert out["rendered"] > 0
    total = t0.elapsed_time(t1)
    ms = {n: a.elapsed_time(b) for n, (a, b) in ev.items()}
    print("[gpu-test] launch events ms", ms, "total", total, flush=True)
    for n, v in ms.items():
        assert 0.0 < v < total, (n, v, total)
    # the rasterize forward's kernel runs after the preprocess kernel ends
    assert ev["preprocess_fwd"][1].elapsed_time(ev["rasterize_fwd"][0]) >= 0.0
    # the colour half starts after the geometry half and ends before the
    # rasterize forward reads its colours
    assert ev["preprocess_fwd"][1].elapsed_time(ev["preprocess_colour"][0]) >= 0.0
    assert ev["preprocess_colour"][1].elapsed_time(ev["rasterize_fwd"][0]) >= 0.0
    # cleared: a further frame leaves the events where they were
    before = ev["rasterize_bwd"][0].elapsed_time(ev["rasterize_bwd"][1])
    run()
    torch.cuda.synchronize()
    assert ev["rasterize_bwd"][0].elapsed_time(ev["rasterize_bwd"][1]) == before
    assert np.isfinite(before)
