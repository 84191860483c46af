"""Shared helpers of the test-suite: seeded scenes, GPU <-> numpy glue and the
tolerance checks of the parity gates.

Gates: radii, tiles_touched, sorted keys/values and
tile ranges bit-exact; rendered image within 1e-4 absolute per pixel;
gradients within 1e-3 relative (plus an absolute floor of 1e-5 x the
array's largest magnitude for entries that cancel to ~0).
"""
from __future__ import annotations

import numpy as np

from fastgs_core_amd import synthetic as syn

IMAGE_ATOL = 1e-4
GRAD_RTOL = 1e-3
GRAD_AFLOOR = 1e-5


def to_np(t):
    import torch

    if torch.is_tensor(t):
        t = t.detach().cpu()
        if t.dtype == torch.bool:
            return t.numpy().astype(np.uint8)
        return t.numpy()
    return np.asarray(t)


def to_torch(inputs: dict, device="cuda", requires_grad=()):
    import torch

    out = {}
    for k, v in inputs.items():
        t = torch.from_numpy(np.ascontiguousarray(v)).to(device)
        if k in requires_grad:
            t.requires_grad_(True)
        out[k] = t
    return out


def scene_small(seed=0, P=2000, degree=3, W=128, H=96, eye=None):
    """A small config-2-like scene (SH degree 3, anisotropic, rotated camera)."""
    sc = syn.scene_config2(seed, P, degree)
    sc["means3d"] = (sc["means3d"] * 0.6).astype(np.float32)
    sc["scales"] = (sc["scales"] * 3.0).astype(np.float32)
    if eye is None:
        cam = syn.sphere_cameras(1, seed + 100, W, H, radius=3.0)[0]
    else:
        cam = syn.look_at_camera(eye, (0, 0, 0), W, H)
    return sc, cam


def assert_grad_close(name, got, ref, rtol=GRAD_RTOL, afloor=GRAD_AFLOOR):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    if ref.size == 0:
        return
    scale = float(np.max(np.abs(ref)))
    tol = rtol * np.abs(ref) + afloor * scale
    bad = np.abs(got - ref) > tol
    if bad.any():
        i = np.argmax(np.abs(got - ref) - tol)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{ref.size} entries outside tolerance; worst flat index {i}: "
            f"got {got.flat[i]!r} ref {ref.flat[i]!r} (scale {scale:.3e})")
