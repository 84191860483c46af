"""Pins the gradient gate's scale, the oracle's sum of term magnitudes
(orc_rasterize_bwd_mag, Oracle.render_backward(..., magnitude=True)).

A gradient entry of the blend is a sum over pixels of one term per (pixel,
splat): each tile list holds a Gaussian at most once.  So the backward of the
loss restricted to one pixel (the loss gradient zero elsewhere) is exactly
that pixel's term vector, and the sum over pixels of its magnitudes must
equal ``mag_terms`` -- computed here through the finite-difference-pinned
backward (orc_rasterize_bwd, test_oracle_fd.py) and not through the
magnitude code.  Through the preprocess backward the propagated magnitude
must bound the per-pixel sum of |gradient| (triangle inequality), and both
magnitudes must bound |gradient| and scale linearly with the loss gradient.
"""
import numpy as np

from fastgs_core_amd import synthetic as syn

from tests.helpers import scene_small

KEYS3 = ("means3d", "scales", "rotations", "opacities", "dc", "sh", "viewspace_points")
KEYS2 = ("means2d", "colors", "conic_opacity", "viewspace_points")


def _setup(oracle64, seed=4, P=300, deg=3, W=40, H=24):
    sc, cam = scene_small(seed, P, deg, W, H, eye=(0.4, 0.3, -2.6))
    inp = syn.make_inputs(sc, cam, background=(0.2, 0.5, 0.9))
    inp = {k: (np.asarray(v, np.float64) if np.asarray(v).dtype.kind == "f" else v)
           for k, v in inp.items()}
    fwd = oracle64.render(inp, W, H, cam.tan_fovx, cam.tan_fovy, deg)
    assert fwd["rendered"] > 0
    return inp, cam, fwd, deg


def test_term_magnitudes_equal_per_pixel_sums(oracle64):
    inp, cam, fwd, deg = _setup(oracle64)
    W, H = cam.width, cam.height
    dL = np.random.default_rng(3).standard_normal((3, W * H))
    g = oracle64.render_backward(inp, fwd, dL, W, H, cam.tan_fovx, cam.tan_fovy, deg,
                                 magnitude=True)
    s2 = {k: np.zeros_like(g["raster"][k]) for k in KEYS2}
    s3 = {k: np.zeros_like(g[k], dtype=np.float64) for k in KEYS3}
    for p in range(W * H):
        one = np.zeros_like(dL)
        one[:, p] = dL[:, p]
        gp = oracle64.render_backward(inp, fwd, one, W, H, cam.tan_fovx, cam.tan_fovy, deg)
        for k in KEYS2:
            s2[k] += np.abs(gp["raster"][k])
        for k in KEYS3:
            s3[k] += np.abs(gp[k])
    for k in KEYS2:
        m = g["raster"]["mag_terms"][k]
        np.testing.assert_allclose(m, s2[k], rtol=1e-9, atol=1e-300, err_msg=k)
        assert np.all(g["raster"]["mag"][k] >= m * (1 - 1e-12)), k
        assert m.max() > 0, k
    for k in KEYS3:
        m = g["mag_terms"][k]
        assert np.all(m >= s3[k] * (1 - 1e-9)), k
        assert np.all(m >= np.abs(g[k]) * (1 - 1e-9)), k
        assert np.all(g["mag"][k] >= m * (1 - 1e-12)), k
        assert m.max() > 0, k


def test_magnitudes_scale_with_the_loss_gradient(oracle64):
    inp, cam, fwd, deg = _setup(oracle64, seed=9)
    W, H = cam.width, cam.height
    dL = np.random.default_rng(5).standard_normal((3, W * H))
    a = oracle64.render_backward(inp, fwd, dL, W, H, cam.tan_fovx, cam.tan_fovy, deg,
                                 magnitude=True)
    b = oracle64.render_backward(inp, fwd, -2.0 * dL, W, H, cam.tan_fovx, cam.tan_fovy, deg,
                                 magnitude=True)
    for key in ("mag", "mag_terms"):
        for k in KEYS3:
            np.testing.assert_allclose(b[key][k], 2.0 * a[key][k], rtol=1e-12, err_msg=k)


def test_preprocess_magnitudes_bound_the_linear_map(oracle64):
    """The preprocess backward is linear in its cotangents, g = J c; its
    coefficient columns J e_k are its outputs for one-hot cotangents (through
    the finite-difference-pinned orc_preprocess_bwd).  The expanded sum of
    term magnitudes (orc_preprocess_bwd_mag) must bound sum_k |J_k| |c_k|,
    hence |g|, be linear in the cotangent magnitudes, and on needle-shaped
    Gaussians (one scale 100x the others) exceed |g| by orders of magnitude:
    there a plain relative gate on the 3D gradients measures cancellation,
    not parity."""
    rng = np.random.default_rng(2)
    P, W, H = 400, 160, 120
    sc = syn.scene_config2(3, P, 3)
    sc["means3d"] = (sc["means3d"] * 0.5).astype(np.float32)
    ls = rng.normal(-3.5, 0.5, (P, 3))
    ls[: P // 2, 0] = rng.normal(-0.8, 0.3, P // 2)  # needles
    sc["scales"] = np.exp(ls).astype(np.float32)
    cam = syn.look_at_camera((0.3, 0.4, -3.0), (0, 0, 0), W, H)
    inp = {k: (np.asarray(v, np.float64) if np.asarray(v).dtype.kind == "f" else v)
           for k, v in syn.make_inputs(sc, cam).items()}
    pre = oracle64.preprocess_fwd(inp["means3d"], inp["opacities"], inp["viewmatrix"],
                                  inp["projmatrix"], inp["campos"], inp["viewspace_points"], W, H,
                                  cam.tan_fovx, cam.tan_fovy, 3, dc=inp["dc"], sh=inp["sh"],
                                  scales=inp["scales"], rotations=inp["rotations"])
    assert (pre["radii"] > 0).sum() > 100
    widths = (("xys", 2), ("rgb", 3), ("conic", 4), ("vsp", 4))
    cot = {k: rng.normal(0, 1, (P, w)) for k, w in widths}
    args = (inp["means3d"], inp["viewmatrix"], inp["projmatrix"], inp["campos"], pre["radii"],
            pre["cov3d"], pre["clamped"])
    kw = dict(sh=inp["sh"], scales=inp["scales"], rotations=inp["rotations"])

    def bwd(c):
        return oracle64.preprocess_bwd(*args, c["xys"], c["rgb"], c["conic"], c["vsp"], W, H,
                                       cam.tan_fovx, cam.tan_fovy, 3, **kw)

    def mag(c):
        return oracle64.preprocess_bwd_mag(*args, c["xys"], c["rgb"], c["conic"], c["vsp"], W, H,
                                           cam.tan_fovx, cam.tan_fovy, 3, **kw)

    g = bwd(cot)
    m = mag({k: np.abs(v) for k, v in cot.items()})
    lin = {k: np.zeros_like(m[k]) for k in KEYS3}
    for name, w in widths:
        for q in range(w):
            one = {k: np.zeros((P, ww)) for k, ww in widths}
            one[name][:, q] = 1.0
            col = bwd(one)
            for k in KEYS3:
                a = np.abs(col[k])
                lin[k] += a * np.abs(cot[name][:, q]).reshape((P,) + (1,) * (a.ndim - 1))
    m2 = mag({k: 2.0 * np.abs(v) for k, v in cot.items()})
    ratios = []
    for k in KEYS3:
        assert np.all(m[k] >= lin[k] * (1 - 1e-9)), k
        assert np.all(lin[k] >= np.abs(g[k]) * (1 - 1e-9)), k
        np.testing.assert_allclose(m2[k], 2.0 * m[k], rtol=1e-12, err_msg=k)
        nz = np.abs(g[k]) > 0
        ratios.append(float(np.max(m[k][nz] / np.abs(g[k][nz]))))
    assert max(ratios) > 1e3, ratios
