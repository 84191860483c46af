"""The scanner dataset around the training loop: point cloud, camera JSON,
target images, the initial model and the .spz export, as the reference's
training scripts define them (scripts/train_scanner_fixed.py).

Everything here is host-side numpy (file formats, 4x4 camera algebra); the
arrays it returns are what ``rasterize_gaussians`` and
``GaussianTrainState`` take.  Function names, arguments and results follow
the reference so its training script ports line by line:

* ``load_ply_positions_colors`` (:237-257) through ``ply.read_ply``;
* ``make_axis_transform`` / ``compute_normalization`` (:312-331);
* ``build_camera_from_scanner_json`` (:334-395) -> ``synthetic.Camera``
  (``viewmatrix`` / ``projmatrix`` are the transposed matrices the
  rasterizer reads, as the reference passes ``raw_viewmat.T``);
* ``collect_scanner_frames``, ``load_target_image``, ``prepare_dataset``
  (:265-307, :398-500);
* ``init_model`` (:601-631) -> the parameter dict of ``GaussianTrainState``;
* ``save_as_spz`` (:634-681) through ``spz.save_spz``.
"""
from __future__ import annotations

import json
import math
import re
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import ply as _ply
from . import spz as _spz
from .synthetic import Camera

SH_C0 = 0.28209479177387814


# --------------------------------------------------------------- rotations
def quaternions_wxyz_to_rotation_matrices(quats: np.ndarray) -> np.ndarray:
    """Rotation matrices of (w, x, y, z) quaternions, normalised first
    (train_scanner_fixed.py:160-192)."""
    q = np.asarray(quats, dtype=np.float32)
    q = q / np.clip(np.linalg.norm(q, axis=1, keepdims=True), 1.0e-8, None)
    w, x, y, z = q[:, 0], q[:, 1], q[:, 2], q[:, 3]
    r = np.empty((q.shape[0], 3, 3), dtype=np.float32)
    r[:, 0, 0] = 1.0 - 2.0 * (y * y + z * z)
    r[:, 0, 1] = 2.0 * (x * y - w * z)
    r[:, 0, 2] = 2.0 * (x * z + w * y)
    r[:, 1, 0] = 2.0 * (x * y + w * z)
    r[:, 1, 1] = 1.0 - 2.0 * (x * x + z * z)
    r[:, 1, 2] = 2.0 * (y * z - w * x)
    r[:, 2, 0] = 2.0 * (x * z - w * y)
    r[:, 2, 1] = 2.0 * (y * z + w * x)
    r[:, 2, 2] = 1.0 - 2.0 * (x * x + y * y)
    return r


def rotation_matrices_to_quaternions_wxyz(rot: np.ndarray) -> np.ndarray:
    """(w, x, y, z) quaternions of rotation matrices by the four-branch
    (trace, then largest diagonal) method, normalised
    (train_scanner_fixed.py:195-234)."""
    r = np.asarray(rot, dtype=np.float32)
    q = np.empty((r.shape[0], 4), dtype=np.float32)
    tr = r[:, 0, 0] + r[:, 1, 1] + r[:, 2, 2]
    b0 = tr > 0.0
    bx = ~b0 & (r[:, 0, 0] > r[:, 1, 1]) & (r[:, 0, 0] > r[:, 2, 2])
    by = ~b0 & ~bx & (r[:, 1, 1] > r[:, 2, 2])
    bz = ~b0 & ~bx & ~by
    if b0.any():
        s = np.sqrt(tr[b0] + 1.0) * 2.0
        m = r[b0]
        q[b0] = np.stack([0.25 * s, (m[:, 2, 1] - m[:, 1, 2]) / s, (m[:, 0, 2] - m[:, 2, 0]) / s,
                          (m[:, 1, 0] - m[:, 0, 1]) / s], axis=1)
    if bx.any():
        m = r[bx]
        s = np.sqrt(1.0 + m[:, 0, 0] - m[:, 1, 1] - m[:, 2, 2]) * 2.0
        q[bx] = np.stack([(m[:, 2, 1] - m[:, 1, 2]) / s, 0.25 * s, (m[:, 0, 1] + m[:, 1, 0]) / s,
                          (m[:, 0, 2] + m[:, 2, 0]) / s], axis=1)
    if by.any():
        m = r[by]
        s = np.sqrt(1.0 + m[:, 1, 1] - m[:, 0, 0] - m[:, 2, 2]) * 2.0
        q[by] = np.stack([(m[:, 0, 2] - m[:, 2, 0]) / s, (m[:, 0, 1] + m[:, 1, 0]) / s, 0.25 * s,
                          (m[:, 1, 2] + m[:, 2, 1]) / s], axis=1)
    if bz.any():
        m = r[bz]
        s = np.sqrt(1.0 + m[:, 2, 2] - m[:, 0, 0] - m[:, 1, 1]) * 2.0
        q[bz] = np.stack([(m[:, 1, 0] - m[:, 0, 1]) / s, (m[:, 0, 2] + m[:, 2, 0]) / s,
                          (m[:, 1, 2] + m[:, 2, 1]) / s, 0.25 * s], axis=1)
    return q / np.clip(np.linalg.norm(q, axis=1, keepdims=True), 1.0e-8, None)


# ------------------------------------------------------------- point cloud
def load_ply_positions_colors(path) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """Vertex positions [N,3] and, when the file has red/green/blue, colours
    [N,3] in [0,1] (divided by 255 when any exceeds 1, then clipped)."""
    v = _ply.read_ply(path, elements=("vertex",))["vertex"]
    pts = np.stack([v["x"], v["y"], v["z"]], axis=1).astype(np.float32)
    colors = None
    if {"red", "green", "blue"}.issubset(v):
        colors = np.stack([v["red"], v["green"], v["blue"]], axis=1).astype(np.float32)
        if colors.size and colors.max() > 1.0:
            colors = colors / 255.0
        colors = np.clip(colors, 0.0, 1.0)
    return pts, colors


# ----------------------------------------------------------------- cameras
def make_axis_transform() -> Tuple[np.ndarray, np.ndarray]:
    """The scanner-to-training axis change (x, y, z) -> (x, z, -y), 3x3 and 4x4."""
    a = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0], [0.0, -1.0, 0.0]], dtype=np.float32)
    a4 = np.eye(4, dtype=np.float32)
    a4[:3, :3] = a
    return a, a4


def compute_normalization(camera_positions: Sequence[np.ndarray]) -> Tuple[np.ndarray, float]:
    """Translation = mean camera centre; scale = 1 / max |centre - mean|
    over every coordinate (1 when the centres coincide)."""
    c = np.stack(camera_positions, axis=0).astype(np.float32)
    t = c.mean(axis=0)
    denom = np.max(np.abs(c - t[None, :]))
    return t, (1.0 / float(denom) if denom > 0.0 else 1.0)


def build_camera_from_scanner_json(frame: Dict, image_width: int, image_height: int,
                                   znear: float = 0.001, zfar: float = 1000.0) -> Camera:
    """A training camera from one normalised frame record (``w``, ``h``,
    ``fl_x``, ``fl_y``, ``cx``, ``cy``, ``transform_matrix`` = camera-to-world
    with the camera looking down -z).  The focal lengths are rescaled to the
    image size; the frustum is symmetric (``cx`` / ``cy`` do not enter), as
    in the reference."""
    width, height = float(image_width), float(image_height)
    sx = width / float(frame.get("w", image_width))
    sy = height / float(frame.get("h", image_height))
    fx = float(frame["fl_x"]) * sx
    fy = float(frame["fl_y"]) * sy
    c2w = np.array(frame["transform_matrix"], dtype=np.float32)
    r = c2w[:3, :3].astype(np.float32) @ np.diag([1.0, -1.0, -1.0]).astype(np.float32)
    t = c2w[:3, 3:4].astype(np.float32)
    rinv = r.T
    view = np.eye(4, dtype=np.float32)
    view[:3, :3] = rinv
    view[:3, 3:4] = (-rinv @ t).astype(np.float32)
    fovx = 2.0 * math.atan(width / (2.0 * fx))
    fovy = 2.0 * math.atan(height / (2.0 * fy))
    top = znear * math.tan(0.5 * fovy)
    right = znear * math.tan(0.5 * fovx)
    bottom, left = -top, -right
    proj = np.array([
        [2.0 * znear / (right - left), 0.0, (right + left) / (right - left), 0.0],
        [0.0, 2.0 * znear / (top - bottom), (top + bottom) / (top - bottom), 0.0],
        [0.0, 0.0, (zfar + znear) / (zfar - znear), -(zfar * znear) / (zfar - znear)],
        [0.0, 0.0, 1.0, 0.0]], dtype=np.float32)
    full = proj @ view
    return Camera(viewmatrix=view.T.astype(np.float32), projmatrix=full.T.astype(np.float32),
                  campos=t[:, 0].astype(np.float32), width=int(image_width),
                  height=int(image_height), tan_fovx=float(math.tan(0.5 * fovx)),
                  tan_fovy=float(math.tan(0.5 * fovy)))


def scanner_frame_record(raw: Dict, raw_width: int, raw_height: int, image_name: str = ""
                         ) -> Dict:
    """One scanner JSON (``intrinsics`` row-major 3x3, ``cameraPoseARFrame``
    row-major 4x4 camera-to-world) as the frame record of
    ``build_camera_from_scanner_json``, axes changed by ``make_axis_transform``
    (train_scanner_fixed.py:425-446)."""
    intr = raw.get("intrinsics")
    if intr is None or len(intr) != 9:
        raise RuntimeError("Invalid intrinsics in scanner frame JSON")
    pose = raw.get("cameraPoseARFrame")
    if pose is None or len(pose) != 16:
        raise RuntimeError("Invalid cameraPoseARFrame in scanner frame JSON")
    _, a4 = make_axis_transform()
    c2w = (a4 @ np.array(pose, dtype=np.float32).reshape(4, 4)).astype(np.float32)
    return {"w": int(raw_width), "h": int(raw_height), "file_path": image_name,
            "fl_x": float(intr[0]), "fl_y": float(intr[4]), "cx": float(intr[2]),
            "cy": float(intr[5]), "transform_matrix": c2w.tolist()}


# ---------------------------------------------------------------- dataset
@dataclass
class ScannerFrame:
    index: int
    image_path: Path
    json_path: Path
    frame: Optional[Dict] = None


def extract_frame_index(path: Path) -> Optional[int]:
    m = re.search(r"frame_(\d+)", Path(path).stem)
    return None if m is None else int(m.group(1))


def collect_scanner_frames(dataset_dir, max_frames: int, frame_step: int, start_index: int
                           ) -> List[ScannerFrame]:
    """Frames with both ``frame_*.jpg`` and ``frame_*.json``, from
    ``start_index``, every ``frame_step``-th, at most ``max_frames`` (> 0)."""
    d = Path(dataset_dir)
    images = {extract_frame_index(p): p for p in sorted(d.glob("frame_*.jpg"))}
    jsons = {extract_frame_index(p): p for p in sorted(d.glob("frame_*.json"))}
    images.pop(None, None)
    jsons.pop(None, None)
    common = [i for i in sorted(set(images) & set(jsons)) if i >= start_index]
    if frame_step > 1:
        common = common[::frame_step]
    if max_frames > 0:
        common = common[:max_frames]
    if not common:
        raise RuntimeError(f"No scanner frame pairs found in {d}")
    return [ScannerFrame(i, images[i], jsons[i]) for i in common]


def load_target_image(path, width: int, height: int) -> np.ndarray:
    """[H, W, 3] float32 in [0, 1]: RGBA, bilinear-resized when the size
    differs, composited over white."""
    from PIL import Image

    with Image.open(path) as image:
        rgba = np.array(image.convert("RGBA"), dtype=np.float32) / 255.0
    if rgba.shape[1] != width or rgba.shape[0] != height:
        img = Image.fromarray((rgba * 255.0).astype(np.uint8), mode="RGBA")
        rgba = np.array(img.resize((width, height), Image.Resampling.BILINEAR),
                        dtype=np.float32) / 255.0
    bg = np.array([1.0, 1.0, 1.0], dtype=np.float32)
    return rgba[:, :, :3] * rgba[:, :, 3:4] + bg * (1.0 - rgba[:, :, 3:4])


def prepare_dataset(dataset_dir, width: int, height: int, max_frames: int = 120,
                    frame_step: int = 1, start_index: int = 0, max_points: int = 30_000_000,
                    seed: int = 42, extra_points_ratio: float = 0.0,
                    extra_points_mode: str = "surface-jitter",
                    extra_points_jitter_scale: float = 0.01):
    """(cameras, targets [3,H,W] float32, points, colours, base point count):
    the point cloud and camera centres moved to the training axes and
    normalised by the camera centres, points subsampled to ``max_points``,
    optional extra points (surface jitter or bounding box)."""
    from PIL import Image

    d = Path(dataset_dir)
    a, _ = make_axis_transform()
    frames = collect_scanner_frames(d, max_frames, frame_step, start_index)
    points, colors = load_ply_positions_colors(d / "points.ply")
    points = (a @ points.T).T
    centres = []
    for fr in frames:
        with open(fr.json_path, "r", encoding="utf-8") as f:
            raw = json.load(f)
        with Image.open(fr.image_path) as img:
            rw, rh = img.size
        fr.frame = scanner_frame_record(raw, rw, rh, fr.image_path.name)
        centres.append(np.array(fr.frame["transform_matrix"], dtype=np.float32)[:3, 3])
    translation, norm_scale = compute_normalization(centres)
    points = (points - translation[None, :]) * norm_scale
    rng = np.random.default_rng(seed)
    if max_points > 0 and points.shape[0] > max_points:
        keep = rng.choice(points.shape[0], size=max_points, replace=False)
        points = points[keep]
        if colors is not None:
            colors = colors[keep]
    colors_np = colors.astype(np.float32) if colors is not None else \
        np.full_like(points, 0.5, dtype=np.float32)
    base = int(points.shape[0])
    extra = int(round(points.shape[0] * extra_points_ratio))
    if extra > 0:
        lo, hi = points.min(axis=0), points.max(axis=0)
        if extra_points_mode == "surface-jitter":
            src = rng.integers(0, points.shape[0], size=extra)
            std = extra_points_jitter_scale * float(np.linalg.norm(hi - lo))
            jitter = rng.normal(loc=0.0, scale=std, size=(extra, 3)).astype(np.float32)
            exyz, ergb = points[src] + jitter, colors_np[src]
        elif extra_points_mode == "bbox":
            exyz = rng.uniform(low=lo, high=hi, size=(extra, 3)).astype(np.float32)
            ergb = colors_np[rng.integers(0, colors_np.shape[0], size=extra)]
        else:
            raise ValueError(f"Unsupported --extra-points-mode: {extra_points_mode}")
        points = np.concatenate([points, exyz], axis=0).astype(np.float32)
        colors_np = np.concatenate([colors_np, ergb.astype(np.float32)], axis=0)
    cameras, targets = [], []
    for fr in frames:
        c2w = np.array(fr.frame["transform_matrix"], dtype=np.float32)
        c2w[:3, 3] = (c2w[:3, 3] - translation) * norm_scale
        rec = dict(fr.frame)
        rec["transform_matrix"] = c2w.tolist()
        cameras.append(build_camera_from_scanner_json(rec, width, height))
        targets.append(np.ascontiguousarray(
            np.transpose(load_target_image(fr.image_path, width, height), (2, 0, 1))))
    return cameras, targets, points.astype(np.float32), colors_np, base


# ------------------------------------------------------------------ model
def init_model(points: np.ndarray, colors: np.ndarray, sh_degree: int) -> Dict[str, np.ndarray]:
    """Initial parameters: isotropic scale 0.02 (log-space), identity
    rotations, opacity 0.82 (logit), DC = (colour - 0.5) / C0, higher SH 0.
    Keys and shapes are ``GaussianTrainState``'s."""
    n = int(points.shape[0])
    rot = np.zeros((n, 4), dtype=np.float32)
    rot[:, 0] = 1.0
    p = np.float32(0.82)
    return {
        "means3d": np.asarray(points, dtype=np.float32),
        "features_dc": ((np.asarray(colors, dtype=np.float32) - 0.5) / SH_C0).astype(np.float32),
        "features_rest": np.zeros((n, max(0, (sh_degree + 1) ** 2 - 1), 3), dtype=np.float32),
        "opacity_logits": np.full((n, 1), np.log(p / (np.float32(1.0) - p)), dtype=np.float32),
        "log_scales": np.full((n, 3), math.log(0.02), dtype=np.float32),
        "rotations": rot,
    }


# ----------------------------------------------------------------- export
def save_as_spz(filename, params: Dict, sh_degree: int, version: int = 2) -> bool:
    """Export parameters (``GaussianTrainState`` names; tensors or arrays) as
    .spz the way the reference does: means (x, -z, y), rotations conjugated
    by the same axis change, log scales, opacity logits, DC and higher SH,
    antialiased, no further coordinate conversion.  As in the reference, the
    (w, x, y, z) quaternions fill the cloud's rotation slots unchanged."""
    def arr(k):
        v = params[k]
        v = v.detach().cpu().numpy() if hasattr(v, "detach") else np.asarray(v)
        return np.asarray(v, dtype=np.float32)

    means = arr("means3d")
    means_spz = np.empty_like(means)
    means_spz[:, 0] = means[:, 0]
    means_spz[:, 1] = -means[:, 2]
    means_spz[:, 2] = means[:, 1]
    rots = arr("rotations")
    quats = rots / (np.linalg.norm(rots, axis=1, keepdims=True) + np.float32(1.0e-8))
    axis3, _ = make_axis_transform()
    rm = axis3 @ quaternions_wxyz_to_rotation_matrices(quats) @ axis3.T
    quats_spz = rotation_matrices_to_quaternions_wxyz(rm)
    cloud = _spz.GaussianCloud(
        positions=means_spz.reshape(-1), scales=arr("log_scales").reshape(-1),
        rotations=quats_spz.reshape(-1), alphas=arr("opacity_logits").reshape(-1),
        colors=arr("features_dc").reshape(-1), sh=arr("features_rest").reshape(-1),
        sh_degree=int(sh_degree), antialiased=True)
    return _spz.save_spz(cloud, _spz.PackOptions(version=version), filename)
