"""Central finite differences of the float64 oracle pin its analytic backward
(orc_rasterize_bwd: semantics of fastgs_rasterize_backward.metal:24-278;
orc_preprocess_bwd: fastgs_preprocess_backward.metal:60-430).

Documented reference conventions checked here:
* d means2d = (W/2, H/2) * dL/d(pixel xy)   (fastgs_rasterize_backward.metal:101-102)
* d conic[1] = 1/2 * dL/d b                   (ibid. :245)
* d_viewspace[:, :2] = d means2d, d_viewspace[:, 2:] >= |d means2d|
* end-to-end gradients w.r.t. means3d, scales, rotations (unnormalised
  quaternion), opacities, dc, sh (degree 3) and colors_precomp are true
  derivatives of the rendered image.
A coordinate whose +-eps evaluations change any integer output (tile lists,
n_contrib) sits on a discontinuity and is skipped.
"""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn

RTOL = 2e-5


def _scene(seed=0, P=40, degree=3, W=48, H=40):
    rng = np.random.default_rng(seed)
    sc = syn.scene_config2(seed, P, degree)
    sc["means3d"] = rng.uniform(-0.5, 0.5, (P, 3))
    sc["scales"] = np.exp(rng.normal(-2.3, 0.4, (P, 3)))
    sc["opacities"] = rng.uniform(0.2, 0.95, P)
    sc["sh"] = rng.normal(0.0, 0.2, sc["sh"].shape)
    for k in list(sc):
        if isinstance(sc[k], np.ndarray):
            sc[k] = sc[k].astype(np.float64)
    cam = syn.look_at_camera((0.9, 0.6, -3.0), (0.05, -0.05, 0.1), W, H)
    inp = syn.make_inputs(sc, cam, background=(0.1, 0.2, 0.3))
    return sc, cam, {k: np.asarray(v, np.float64) if v.dtype != np.int32 else v
                     for k, v in inp.items()}


def _loss_and_sig(orc, inp, cam, deg, w):
    f = orc.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, deg)
    if "out_color" not in f:
        return 0.0, (0,)
    sig = (f["point_list"].tobytes(), f["img_n_contrib"].tobytes())
    return float((w * f["out_color"]).sum()), sig


def _check_param(orc, inp, cam, deg, w, g, key, idxs, eps_rel=1e-6):
    base = inp[key]
    checked = 0
    for idx in idxs:
        eps = eps_rel * max(1.0, abs(base[idx]))
        vals = []
        sigs = []
        for s in (+1, -1):
            x = base.copy()
            x[idx] += s * eps
            inp2 = dict(inp)
            inp2[key] = x
            L, sig = _loss_and_sig(orc, inp2, cam, deg, w)
            vals.append(L)
            sigs.append(sig)
        if sigs[0] != sigs[1]:
            continue
        fd = (vals[0] - vals[1]) / (2 * eps)
        an = g[key][idx]
        scale = np.abs(g[key]).max()
        assert abs(an - fd) <= RTOL * abs(fd) + 1e-7 * scale, (key, idx, an, fd)
        checked += 1
    return checked


@pytest.mark.parametrize("key", ["means3d", "scales", "rotations", "opacities", "dc", "sh"])
def test_end_to_end_gradients_fd(oracle64, key):
    sc, cam, inp = _scene()
    rng = np.random.default_rng(1)
    w = rng.standard_normal((3, cam.width * cam.height))
    f = oracle64.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 3)
    assert f["rendered"] > 0
    g = oracle64.render_backward(inp, f, w, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 3)
    vis = np.nonzero(f["radii"] > 0)[0]
    arr = inp[key]
    idxs = []
    for gi in vis[:12]:
        for j in range(int(np.prod(arr.shape[1:])) if arr.ndim > 1 else 1):
            idxs.append(np.unravel_index(gi * (arr.size // arr.shape[0]) + j, arr.shape))
    idxs = idxs[:60]
    n = _check_param(oracle64, inp, cam, 3, w, g, key, idxs)
    assert n >= min(20, len(idxs) // 2), f"only {n} coordinates checked"


def test_colors_precomp_and_cov3d_precomp_fd(oracle64):
    sc, cam, inp = _scene(2, P=30, degree=0)
    P = sc["means3d"].shape[0]
    rng = np.random.default_rng(3)
    pre = oracle64.preprocess_fwd(inp["means3d"], inp["opacities"], inp["viewmatrix"],
                                  inp["projmatrix"], inp["campos"], inp["viewspace_points"],
                                  cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0,
                                  scales=inp["scales"], rotations=inp["rotations"],
                                  colors_precomp=np.zeros((P, 3)))
    for k in ("scales", "rotations", "dc", "sh"):
        del inp[k]
    inp["cov3d_precomp"] = pre["cov3d"]
    inp["colors_precomp"] = rng.uniform(0, 1, (P, 3))
    w = rng.standard_normal((3, cam.width * cam.height))
    f = oracle64.render(inp, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    g = oracle64.render_backward(inp, f, w, cam.width, cam.height, cam.tan_fovx, cam.tan_fovy, 0)
    vis = np.nonzero(f["radii"] > 0)[0][:10]
    idxs = [(i, c) for i in vis for c in range(3)]
    assert _check_param(oracle64, inp, cam, 0, w, g, "colors_precomp", idxs) >= 20
    assert _check_param(oracle64, inp, cam, 0, w, g, "means3d", idxs) >= 20
    # the reference never writes d_cov3d_precomp (fastgs_preprocess_backward.metal:364-423)
    assert "cov3d_precomp" not in g or not np.asarray(g.get("cov3d_precomp", 0)).any()


def test_rasterize_conventions_fd(oracle64):
    """Standalone rasterize: means2d gradient is (W/2,H/2)-scaled, the conic off-diagonal
    gradient is halved, colour/opacity gradients are plain derivatives; viewspace carries
    (x, y, |x|, |y|)."""
    rng = np.random.default_rng(4)
    n, W, H = 12, 32, 32
    xy = rng.uniform(4, 28, (n, 2))
    ev = np.exp(rng.uniform(np.log(2), np.log(30), (n, 2)))
    th = rng.uniform(0, np.pi, n)
    co = np.zeros((n, 4))
    for i in range(n):
        Rm = np.array([[np.cos(th[i]), -np.sin(th[i])], [np.sin(th[i]), np.cos(th[i])]])
        c = np.linalg.inv(Rm @ np.diag(ev[i]) @ Rm.T)
        co[i] = [c[0, 0], c[0, 1], c[1, 1], rng.uniform(0.3, 0.9)]
    col = rng.uniform(0, 1, (n, 3))
    bg = np.array([0.3, 0.1, 0.2])
    ranges = np.array([[0, n], [0, n], [0, n], [0, n]])
    offs = np.array([1, 2, 3, 4])
    plist = np.arange(n)
    w = rng.standard_normal((3, W * H))

    def render(xy_, col_, co_):
        r = oracle64.rasterize_fwd(ranges, plist, offs, xy_, col_, co_, bg, None, W, H)
        return float((w * r["out_color"]).sum()), r

    _, r = render(xy, col, co)
    g = oracle64.rasterize_bwd(ranges, plist, xy, col, co, bg, r["final_t"], r["n_contrib"], w,
                               W, H)
    eps = 1e-6
    checked = 0
    for i in range(n):
        for which, arr, scale in (("means2d", xy, (W / 2, H / 2)), ("colors", col, (1, 1, 1)),
                                  ("conic_opacity", co, (1, 0.5, 1, 1))):
            for j in range(arr.shape[1]):
                a = arr.copy()
                a[i, j] += eps
                b = arr.copy()
                b[i, j] -= eps
                args_p = {"means2d": (a, col, co), "colors": (xy, a, co),
                          "conic_opacity": (xy, col, a)}[which]
                args_m = {"means2d": (b, col, co), "colors": (xy, b, co),
                          "conic_opacity": (xy, col, b)}[which]
                Lp, rp = render(*args_p)
                Lm, rm = render(*args_m)
                if not np.array_equal(rp["n_contrib"], rm["n_contrib"]):
                    continue
                fd = (Lp - Lm) / (2 * eps) * scale[j]
                an = g[which][i, j]
                assert abs(an - fd) <= 1e-5 * abs(fd) + 1e-8 * np.abs(g[which]).max(), \
                    (which, i, j, an, fd)
                checked += 1
    assert checked > 80
    # same per-pixel terms; OpenMP atomics may sum them in different orders
    np.testing.assert_allclose(g["viewspace_points"][:, :2], g["means2d"], rtol=1e-12,
                               atol=1e-15 * np.abs(g["means2d"]).max())
    assert (g["viewspace_points"][:, 2:] >= np.abs(g["means2d"]) - 1e-12).all()
