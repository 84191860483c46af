"""Seeded synthetic scenes and cameras for the BASELINE configurations.

Camera convention follows the reference training scripts
(scripts/train_square.py:38-86): ``forward = normalize(target - eye)``,
``right = forward x up``, ``up' = right x forward``; ``viewmatrix`` is the
transposed world-to-view matrix flattened, i.e. the column-major 4x4 that
``transform_point_4x3`` reads (fastgs_preprocess.metal:81-86), and
``projmatrix = viewmatrix @ projection^T``.  znear 0.01, zfar 100.

"60 degree FoV" is applied as fovx = 60 deg with fovy = 2*atan(tan(30 deg) * H/W)
(square pixels).  Parameters are returned *activated* (opacity = sigmoid(logit),
scale = exp(log_scale), unit quaternions), which is what the rasterizer API
receives from its callers (train_scanner_fixed.py:523-536).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


def _normalize(v):
    return v / (np.linalg.norm(v) + 1.0e-8)


def projection_matrix(znear: float, zfar: float, fovx: float, fovy: float) -> np.ndarray:
    """Perspective matrix of scripts/train_square.py:38-56 (row-major, z_sign=+1)."""
    tan_half_fovy = math.tan(fovy / 2.0)
    tan_half_fovx = math.tan(fovx / 2.0)
    top = tan_half_fovy * znear
    bottom = -top
    right = tan_half_fovx * znear
    left = -right
    p = np.zeros((4, 4), dtype=np.float32)
    p[0, 0] = 2.0 * znear / (right - left)
    p[1, 1] = 2.0 * znear / (top - bottom)
    p[0, 2] = (right + left) / (right - left)
    p[1, 2] = (top + bottom) / (top - bottom)
    p[3, 2] = 1.0
    p[2, 2] = zfar / (zfar - znear)
    p[2, 3] = -(zfar * znear) / (zfar - znear)
    return p


@dataclass
class Camera:
    viewmatrix: np.ndarray  # (4,4) float32, column-major view (world_to_view^T)
    projmatrix: np.ndarray  # (4,4) float32, viewmatrix @ projection^T
    campos: np.ndarray      # (3,) float32
    width: int
    height: int
    tan_fovx: float
    tan_fovy: float


def look_at_camera(eye, target, width: int, height: int, fovx_deg: float = 60.0,
                   up=(0.0, 1.0, 0.0), znear: float = 0.01, zfar: float = 100.0) -> Camera:
    eye = np.asarray(eye, dtype=np.float32)
    target = np.asarray(target, dtype=np.float32)
    up = np.asarray(up, dtype=np.float32)
    fovx = math.radians(fovx_deg)
    tan_fovx = math.tan(fovx / 2.0)
    tan_fovy = tan_fovx * height / width
    fovy = 2.0 * math.atan(tan_fovy)
    forward = _normalize(target - eye)
    right = _normalize(np.cross(forward, up))
    true_up = _normalize(np.cross(right, forward))
    w2v = np.eye(4, dtype=np.float32)
    w2v[0, :3] = right
    w2v[1, :3] = true_up
    w2v[2, :3] = forward
    w2v[:3, 3] = -w2v[:3, :3] @ eye
    view = w2v.T.astype(np.float32)
    proj = (view @ projection_matrix(znear, zfar, fovx, fovy).T).astype(np.float32)
    return Camera(view, proj, eye.astype(np.float32), width, height, tan_fovx, tan_fovy)


def sphere_cameras(n: int, seed: int, width: int, height: int, radius: float = 4.0,
                   fovx_deg: float = 60.0):
    """n seeded cameras on a sphere of ``radius`` looking at the origin."""
    rng = np.random.default_rng(seed)
    cams = []
    while len(cams) < n:
        v = rng.standard_normal(3)
        eye = radius * v / np.linalg.norm(v)
        if abs(eye[1]) > 0.99 * radius:
            continue
        cams.append(look_at_camera(eye, (0.0, 0.0, 0.0), width, height, fovx_deg))
    return cams


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


def _quats(rng, P):
    q = rng.standard_normal((P, 4)).astype(np.float32)
    return (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float32)


def scene_config1(seed: int = 0, P: int = 16384):
    """Plumbing config: means U[-1,1]^3, log-scale N(-4,0.5), logits N(0,1), SH0 dc U(0,1)."""
    rng = np.random.default_rng(seed)
    return {
        "means3d": rng.uniform(-1, 1, (P, 3)).astype(np.float32),
        "scales": np.exp(rng.normal(-4.0, 0.5, (P, 3))).astype(np.float32),
        "rotations": _quats(rng, P),
        "opacities": _sigmoid(rng.normal(0.0, 1.0, P)).astype(np.float32),
        "dc": rng.uniform(0, 1, (P, 3)).astype(np.float32),
        "sh": np.zeros((P, 0, 3), np.float32),
        "degree": 0,
    }


def scene_config2(seed: int = 0, P: int = 200_000, degree: int = 3):
    """Config 2/3 distributions: means N(0,1)^3 clipped to [-2,2]; log-scale N(-4.5,0.7);
    logits N(0,1.5); dc U(0,1); higher-order SH N(0,0.05)."""
    rng = np.random.default_rng(seed)
    n_rest = (degree + 1) ** 2 - 1
    return {
        "means3d": np.clip(rng.standard_normal((P, 3)), -2, 2).astype(np.float32),
        "scales": np.exp(rng.normal(-4.5, 0.7, (P, 3))).astype(np.float32),
        "rotations": _quats(rng, P),
        "opacities": _sigmoid(rng.normal(0.0, 1.5, P)).astype(np.float32),
        "dc": rng.uniform(0, 1, (P, 3)).astype(np.float32),
        "sh": rng.normal(0.0, 0.05, (P, n_rest, 3)).astype(np.float32),
        "degree": degree,
    }


def scene_config4(seed: int = 0, P: int = 3_000_000, degree: int = 3):
    """Heavy-overlap stress: log-scale N(-4,1.2) with 2% drawn from N(-1.5,0.3);
    logits N(1,1)."""
    rng = np.random.default_rng(seed)
    n_rest = (degree + 1) ** 2 - 1
    ls = rng.normal(-4.0, 1.2, (P, 3))
    big = rng.random(P) < 0.02
    ls[big] = rng.normal(-1.5, 0.3, (int(big.sum()), 3))
    return {
        "means3d": np.clip(rng.standard_normal((P, 3)), -2, 2).astype(np.float32),
        "scales": np.exp(ls).astype(np.float32),
        "rotations": _quats(rng, P),
        "opacities": _sigmoid(rng.normal(1.0, 1.0, P)).astype(np.float32),
        "dc": rng.uniform(0, 1, (P, 3)).astype(np.float32),
        "sh": rng.normal(0.0, 0.05, (P, n_rest, 3)).astype(np.float32),
        "degree": degree,
    }


def config1_camera(width: int = 256, height: int = 256) -> Camera:
    """Pinhole at (0,0,-4) looking +z, 60 degree FoV."""
    return look_at_camera((0.0, 0.0, -4.0), (0.0, 0.0, 0.0), width, height, 60.0)


def make_inputs(scene: dict, cam: Camera, background=(0.0, 0.0, 0.0)):
    """Reference ``rasterize_gaussians`` input dict (numpy) for a scene and camera."""
    P = scene["means3d"].shape[0]
    return {
        "means3d": scene["means3d"],
        "scales": scene["scales"],
        "rotations": scene["rotations"],
        "opacities": scene["opacities"],
        "dc": scene["dc"],
        "sh": scene["sh"],
        "background": np.asarray(background, np.float32),
        "metric_map": np.zeros(cam.width * cam.height, np.int32),
        "viewmatrix": cam.viewmatrix.reshape(-1).copy(),
        "projmatrix": cam.projmatrix.reshape(-1).copy(),
        "campos": cam.campos.copy(),
        "viewspace_points": np.zeros((P, 4), np.float32),
    }
