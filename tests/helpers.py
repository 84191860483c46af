"""Shared helpers of the test-suite: seeded scenes, GPU <-> numpy glue and the
tolerance checks of the parity gates.

Gates: radii, tiles_touched, sorted keys/values and
tile ranges bit-exact; rendered image within 1e-4 absolute per pixel;
gradients within 1e-3 relative.  A gradient entry is a sum of per-(pixel,
splat) terms that the GPU adds with float atomics in no fixed order, so
"relative" is taken to the sum of the magnitudes of those terms, which the
oracle computes alongside the gradients (Oracle.render_backward(...,
magnitude=True)): |got - ref| <= 1e-3 * sum |terms| for every entry.  On
the well-conditioned entries, whose |ref| is at least a tenth of sum |terms|,
the plain relative bound |got - ref| <= 1e-3 * |ref| must hold as well, so a
wrong sign or a dropped term there cannot hide in a large magnitude sum.
"""
from __future__ import annotations

import numpy as np

from fastgs_core_amd import synthetic as syn

IMAGE_ATOL = 1e-4
GRAD_RTOL = 1e-3


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


WELL_CONDITIONED = 0.1


def assert_grad_gate(name, got, ref, mag, rtol=GRAD_RTOL):
    """Every entry: |got - ref| <= rtol * mag, mag = the sum of the magnitudes
    of the entry's terms (the oracle's ``mag_terms``).  Entries with no terms
    must match exactly.  Entries with |ref| >= WELL_CONDITIONED * mag must
    also satisfy |got - ref| <= rtol * |ref|.  Prints the worst entry relative
    to its gate."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    mag = np.asarray(mag, np.float64)
    assert got.shape == ref.shape == mag.shape, (name, got.shape, ref.shape, mag.shape)
    if ref.size == 0:
        return
    err = np.abs(got - ref)
    tol = rtol * mag
    bad = ~(err <= tol)
    well = np.abs(ref) >= WELL_CONDITIONED * mag
    bad_rel = well & ~(err <= rtol * np.abs(ref))
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(mag > 0, err / mag, np.where(err > 0, np.inf, 0.0))
        rr = np.where(well & (ref != 0), err / np.abs(ref), 0.0)
    i = int(np.argmax(r))
    j = int(np.argmax(rr))
    info = (f"{name}: {int(bad.sum())}/{ref.size} entries outside 1e-3 * sum|terms|; worst flat "
            f"index {i}: got {got.flat[i]!r} ref {ref.flat[i]!r} sum|terms| {mag.flat[i]!r} "
            f"(err / sum|terms| = {r.flat[i]:.2e}); {int(bad_rel.sum())}/{int(well.sum())} "
            f"well-conditioned entries outside 1e-3 * |ref| (worst {rr.flat[j]:.2e} at {j})")
    print("[gate]", info, flush=True)
    if bad.any() or bad_rel.any():
        raise AssertionError(info)


KEYS_3D = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")
KEYS_2D = (("geom_means2d", "means2d"), ("geom_rgb", "colors"),
           ("geom_conic_opacity", "conic_opacity"), ("viewspace_points", "viewspace_points"))


def capture_2d_gradients(out):
    """Hooks on the preprocess outputs that feed the rasterizer (means2d, rgb,
    conic/opacity, the viewspace pass-through): after backward, the returned
    dict holds the gradients the rasterize backward produced for them."""
    seen = {}
    for key, name in KEYS_2D:
        out[key].register_hook(lambda g, name=name: seen.__setitem__(name, g.detach().clone()))
    return seen


def check_backward_stages(oracle, inp, ref, rg, tin, seen, W, H, cam, degree, keys=KEYS_3D):
    """The three gradient gates of a forward + backward against the oracle
    (rg = oracle.render_backward(..., magnitude=True)):

    1. the rasterize backward's outputs (seen: captured by capture_2d_gradients)
       within 1e-3 of the sum of their per-(pixel, splat) terms' magnitudes
       (float atomics add them in no fixed order);
    2. the preprocess backward on identical inputs: the oracle's, given the
       GPU's own rasterize-backward gradients, bit-exact against the GPU's 3D
       gradients (one thread per Gaussian, the same expressions in the same
       order on both sides);
    3. end to end, every 3D gradient within 1e-3 of the sum of its terms'
       magnitudes over the whole chain rule (the preprocess backward can
       amplify the rounding of gate 1 by far more than its gradients' size:
       sums of terms that cancel, for needle-shaped Gaussians by 10^4).
    Gate failures of all three are collected and reported together."""
    failures = []

    def gate(name, got, want, mag, rtol=GRAD_RTOL):
        try:
            assert_grad_gate(name, got, want, mag, rtol)
        except AssertionError as e:
            failures.append(str(e))

    r2 = rg["raster"]
    for _, name in KEYS_2D:
        gate(f"2D {name}", to_np(seen[name]), r2[name], r2["mag_terms"][name])
    pre = ref["pre"]
    g2 = {name: to_np(seen[name]).astype(np.float32) for _, name in KEYS_2D}
    kw = dict(sh=inp.get("sh"), scales=inp.get("scales"), rotations=inp.get("rotations"))
    args = (inp["means3d"], inp["viewmatrix"], inp["projmatrix"], inp["campos"], pre["radii"],
            pre["cov3d"], pre["clamped"])
    same = oracle.preprocess_bwd(*args, g2["means2d"], g2["colors"], g2["conic_opacity"],
                                 g2["viewspace_points"], W, H, cam.tan_fovx, cam.tan_fovy, degree,
                                 **kw)
    for k in keys:
        got = to_np(tin[k].grad)
        neq = int(np.sum(got != same[k]))
        print(f"[gate] preprocess-bwd {k}: {neq}/{got.size} entries differ from the oracle on "
              "the same inputs", flush=True)
        if neq:
            failures.append(f"preprocess-bwd {k}: {neq} entries not bit-exact")
    for k in keys:
        gate(k, to_np(tin[k].grad), rg[k], rg["mag_terms"][k])
    assert not failures, failures
