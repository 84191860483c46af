"""CPU-side checks of the product boundary: the C-ABI library loads and
exports exactly the entry points include/fastgs_hip.h declares; the Python
API validates inputs with the reference's exception classes and messages
(binding.cpp:46-94, 409-453; fastgs_rasterize.cpp:33-43) before touching a
GPU, and fails loudly (no CPU fallback) when no GPU is present."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import fastgs_core
from fastgs_core_amd import _lib
from fastgs_core_amd import synthetic as syn

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "fastgs_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b(fgs_[a-z0-9_]+)\s*\(", src))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _header_functions()
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.fgs_abi_version() == _lib.ABI_VERSION


def test_workspace_queries_and_error_path():
    lib = _lib.load()
    assert lib.fgs_scan_workspace_bytes(1 << 20) >= 4 * ((1 << 20) // 4096)
    assert lib.fgs_binning_workspace_bytes(1000, 5000, 64) > 5000 * 8
    assert lib.fgs_sort_workspace_bytes(1000) >= 1000 * 12
    # argument validation returns before any HIP call
    rc = lib.fgs_preprocess_fwd(None, None, None)
    assert rc == _lib.FGS_ERR_INVALID_ARGUMENT
    assert b"null" in lib.fgs_last_error()
    rc = lib.fgs_inclusive_scan_u32(None, None, -1, None, None, None)
    assert rc == _lib.FGS_ERR_INVALID_ARGUMENT
    with pytest.raises(ValueError):
        _lib.check(rc)


def test_preprocess_rejects_grids_beyond_16_bit_tiles():
    """The packed tile walks keep tile coordinates in 16 bits: a grid with
    more than 65535 tiles on a side is rejected before any launch (the
    pointers are placeholders the check never dereferences)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(256)
    io = _lib.PreprocessFwdIO(*([fake] * len(_lib.PreprocessFwdIO._fields_)))
    io.st_rec = None
    io.st_masks = None
    for gx, gy in ((65536, 4), (4, 70000)):
        prm = _lib.PreprocessParams(10, 0, 0, gx * 16, gy * 16, gx, gy, 0, 0, 1.0, 1.0, 1.0, 1.0)
        rc = lib.fgs_preprocess_geometry_fwd(ctypes.byref(prm), ctypes.byref(io), None)
        assert rc == _lib.FGS_ERR_INVALID_ARGUMENT
        assert b"65535" in lib.fgs_last_error()


def test_wait_spin_limit_setting():
    """fgs_set_wait_spin_limit swaps the process-wide poll bound (default 2^24)
    and returns the previous value; it touches no GPU."""
    lib = _lib.load()
    prev = lib.fgs_set_wait_spin_limit(7)
    try:
        assert prev == 1 << 24
        assert lib.fgs_set_wait_spin_limit(0) == 7
    finally:
        assert lib.fgs_set_wait_spin_limit(prev) == 0


def test_launch_events_argument_checks():
    """fgs_set_launch_events validates its arguments without touching a GPU:
    unknown names and a single event are rejected; clearing (both NULL) is
    accepted for every named kernel."""
    lib = _lib.load()
    assert lib.fgs_set_launch_events(b"no_such_kernel", None, None) == \
        _lib.FGS_ERR_INVALID_ARGUMENT
    assert b"unknown" in lib.fgs_last_error()
    assert lib.fgs_set_launch_events(None, None, None) == _lib.FGS_ERR_INVALID_ARGUMENT
    assert lib.fgs_set_launch_events(b"rasterize_bwd", ctypes.c_void_p(16), None) == \
        _lib.FGS_ERR_INVALID_ARGUMENT
    assert b"both" in lib.fgs_last_error()
    for name in (b"preprocess_fwd", b"rasterize_fwd", b"rasterize_bwd", b"preprocess_bwd",
                 b"loss_fwd", b"loss_bwd", b"preprocess_colour"):
        assert lib.fgs_set_launch_events(name, None, None) == _lib.FGS_OK


def test_loss_rejects_oversized_planes():
    """The SSIM kernels address a plane through a buffer resource whose byte
    offsets must stay below 2^31: planes of 2^29 pixels or more are rejected
    before any pointer is read or any kernel launched."""
    lib = _lib.load()
    for fn, args in (("fgs_l1_ssim_fwd", (None, None, 3, 1 << 15, 1 << 14, 1.0, 0.2, None, None,
                                         None, None)),
                     ("fgs_l1_ssim_bwd", (None, None, None, None, 3, 1 << 14, 1 << 15, 1.0, 0.2,
                                         None, None))):
        assert getattr(lib, fn)(*args) == _lib.FGS_ERR_INVALID_ARGUMENT, fn
        assert b"2^29" in lib.fgs_last_error(), fn


def test_api_raw_parameters_exclusive():
    """The raw training parameters replace the activated ones; both at once is
    an error raised before any GPU work."""
    inp = _inputs()
    P = inp["means3d"].shape[0]
    inp.update(log_scales=np.zeros((P, 3), np.float32), raw_rotations=np.ones((P, 4), np.float32),
               opacity_logits=np.zeros(P, np.float32))
    with pytest.raises(RuntimeError, match="not both"):
        fastgs_core.rasterize_gaussians(inp, 32, 32, 16, 16, 1.0, 1.0, 0)


def _inputs():
    sc = syn.scene_config1(0, 64)
    cam = syn.config1_camera(32, 32)
    return syn.make_inputs(sc, cam)


def test_api_missing_key_errors():
    inp = _inputs()
    del inp["campos"]
    with pytest.raises(RuntimeError, match="missing required input tensor: campos"):
        fastgs_core.rasterize_gaussians(inp, 32, 32)


def test_api_colour_and_geometry_path_errors():
    inp = _inputs()
    inp["colors_precomp"] = np.ones((64, 3), np.float32)  # and dc+sh present
    with pytest.raises(RuntimeError, match="exactly one color path"):
        fastgs_core.rasterize_gaussians(inp, 32, 32)
    inp = _inputs()
    inp["cov3d_precomp"] = np.ones((64, 6), np.float32)  # and scales+rotations present
    with pytest.raises(RuntimeError, match="exactly one geometry path"):
        fastgs_core.rasterize_gaussians(inp, 32, 32)
    inp = _inputs()
    pf = {"means3d": inp["means3d"], "opacities": inp["opacities"], "viewmat": np.eye(4),
          "projmat": np.eye(4), "cam_pos": np.zeros(3), "viewspace_points": np.zeros((64, 4)),
          "scales": inp["scales"], "quats": inp["rotations"]}
    with pytest.raises(RuntimeError, match="exactly one color path"):
        fastgs_core.preprocess_forward(pf, 32, 32)
    del pf["viewspace_points"]
    with pytest.raises(RuntimeError, match="missing required input tensor: viewspace_points"):
        fastgs_core.preprocess_forward(pf, 32, 32)


def test_api_rasterize_forward_shape_errors():
    z = np.zeros
    with pytest.raises(ValueError, match=r"means2d with shape \(N, 2\)"):
        fastgs_core.rasterize_forward(z((1, 2)), z(1), z(1), z((1, 3)), z((1, 3)), z((1, 4)),
                                      z(3), z(1), z(256), z(1), z((1, 4)), 16, 16, 16, 16, 3, 1, 1)
    with pytest.raises(ValueError, match=r"viewspace_points with shape \(N, 4\)"):
        fastgs_core.rasterize_forward(z((1, 2)), z(1), z(1), z((1, 2)), z((1, 3)), z((1, 4)),
                                      z(3), z(1), z(256), z(1), z((1, 3)), 16, 16, 16, 16, 3, 1, 1)
    with pytest.raises(ValueError, match="share the same N"):
        fastgs_core.rasterize_forward(z((1, 2)), z(1), z(1), z((2, 2)), z((1, 3)), z((1, 4)),
                                      z(3), z(1), z(256), z(1), z((1, 4)), 16, 16, 16, 16, 3, 1, 1)


def test_api_rejects_other_tile_sizes_and_short_sh():
    inp = _inputs()
    with pytest.raises(ValueError, match="16x16"):
        fastgs_core.rasterize_gaussians(inp, 32, 32, 8, 8)
    inp = _inputs()
    with pytest.raises(ValueError, match="degree 2 needs 8"):
        fastgs_core.rasterize_gaussians(inp, 32, 32, 16, 16, 1.0, 1.0, 2)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_cpu_fallback():
    with pytest.raises(RuntimeError, match="requires a ROCm GPU"):
        fastgs_core.rasterize_gaussians(_inputs(), 32, 32)


def test_dummy_api():
    assert fastgs_core.dummy_add(20, 22) == 42  # fastgs_core/test/test.cpp:5-12
    assert fastgs_core.dummy_array_size(np.zeros((3, 4))) == 12


def test_camera_convention():
    """viewmatrix is world_to_view^T (scripts/train_square.py:59-86): the eye maps to the
    view origin and the target onto +z; projmatrix = viewmatrix @ projection^T."""
    cam = syn.look_at_camera((1.0, 2.0, -3.0), (0.2, 0.1, 0.3), 64, 48)
    m = cam.viewmatrix.reshape(-1)

    def xf(p):
        return np.array([m[0] * p[0] + m[4] * p[1] + m[8] * p[2] + m[12],
                         m[1] * p[0] + m[5] * p[1] + m[9] * p[2] + m[13],
                         m[2] * p[0] + m[6] * p[1] + m[10] * p[2] + m[14]])

    np.testing.assert_allclose(xf(cam.campos), 0, atol=1e-5)
    t = xf(np.array([0.2, 0.1, 0.3]))
    np.testing.assert_allclose(t[:2], 0, atol=1e-5)
    assert t[2] > 0
    assert abs(cam.tan_fovy / cam.tan_fovx - 48 / 64) < 1e-6
