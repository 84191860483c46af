"""The rasterize backward skips a 16x4 strip when it lies outside a splat's
row extent (splat_rows in fastgs_core_amd/csrc/fgs_raster.hip).  Skipping a
strip that holds a pixel with alpha >= 1/255 would corrupt that pixel's
transmittance recovery, so the extent must contain every such pixel.

This CPU test restates the kernel's float32 arithmetic with numpy (the
base-2 exponent as splat_power computes it from splat_log2_coeffs, fused
multiply-adds emulated in float64; the exp and the hardware log perturbed by
at least their error) on splats from
isotropic to the most
elongated the extent is used for (det just above 1e-3 a c), and checks that
every pixel that blends lies inside the extent, and that the extent is not
loose by more than its stated margins.
"""
import numpy as np

f32 = np.float32


EXP_ERR = 2.5e-7  # blend_exp2f's relative error against 2^t is below 2e-7
LOG2E = f32(1.44269504088896341)


def _fma32(x, y, z):
    return f32(np.float64(x) * np.float64(y) + np.float64(z))


def _power32(a, b, c, dx, dy):
    """splat_power on splat_log2_coeffs: fma(dy, fma(C, dy, B dx), (A dx) dx),
    A = (-a/2) log2(e), B = -b log2(e), C = (-c/2) log2(e), in float32 (works
    elementwise on arrays): the base-2 exponent t, G = 2^t."""
    A, B, C = f32(f32(-0.5) * a) * LOG2E, f32(-b) * LOG2E, f32(f32(-0.5) * c) * LOG2E
    return _fma32(dy, _fma32(C, dy, f32(B * dx)), f32(f32(A * dx) * dx))


def _rows(y, a, b, c, o, log_err):
    """splat_rows: returns (lo, hi) or None when the splat is not culled."""
    if not (f32(255.0) * o >= f32(0.999)):
        return (np.inf, -np.inf)
    tau = f32(2.0) * f32(np.log(np.float64(f32(255.0) * o)) * (1.0 + log_err))
    det = f32(a * c - b * b)
    if not (a > 0 and c > 0 and det > f32(1e-3) * a * c):
        return None
    tq = f32(max(tau, f32(0.0)) * f32(1.01) + f32(0.05))
    hy = f32(np.sqrt(f32(f32(tq * a) / det))) * f32(1.001) + f32(0.25)
    return f32(y - hy), f32(y + hy)


def _splats(rng, n):
    out = []
    for _ in range(n):
        s1, s2 = np.exp(rng.uniform(np.log(0.3), np.log(60.0), 2))
        th = rng.uniform(0, np.pi)
        R = np.array([[np.cos(th), -np.sin(th)], [np.sin(th), np.cos(th)]])
        cov = R @ np.diag([s1 * s1, s2 * s2]) @ R.T
        con = np.linalg.inv(cov)
        a, b, c = (f32(con[0, 0]), f32(con[0, 1]), f32(con[1, 1]))
        o = f32(np.exp(rng.uniform(np.log(1.0 / 255.0), 0.0)))
        x, y = f32(rng.uniform(-3, 3)), f32(rng.uniform(-3, 3))
        out.append((x, y, a, b, c, o))
    # the most elongated conics the extent is used for: det just above 1e-3 a c
    for _ in range(n // 4):
        a = f32(np.exp(rng.uniform(-6, 1)))
        c = f32(np.exp(rng.uniform(-6, 1)))
        rho = np.sqrt(1.0 - 1.0015e-3) * rng.choice([-1.0, 1.0])
        b = f32(rho * np.sqrt(np.float64(a) * np.float64(c)))
        o = f32(np.exp(rng.uniform(np.log(1.0 / 255.0), 0.0)))
        out.append((f32(rng.uniform(-3, 3)), f32(rng.uniform(-3, 3)), a, b, c, o))
    return out


def _active_rows(x, y, a, b, c, o, rng):
    """Rows of pixels (integer coordinates) whose alpha >= 1/255, with the
    kernel's float32 power and an exp raised by EXP_ERR."""
    det = np.float64(a) * np.float64(c) - np.float64(b) ** 2
    tau = 2.0 * np.log(255.0 * np.float64(o))
    ry = np.sqrt(max(tau, 0.0) * np.float64(a) / det) + 3
    rx = np.sqrt(max(tau, 0.0) * np.float64(c) / det) + 3
    py = np.arange(np.floor(y - ry), np.ceil(y + ry) + 1, dtype=np.float32)
    px = np.arange(np.floor(x - rx), np.ceil(x + rx) + 1, dtype=np.float32)
    if py.size * px.size > 4_000_000:
        px = px[rng.integers(0, px.size, 4_000_000 // max(py.size, 1))]
    X, Y = np.meshgrid(px, py)
    dx = f32(x) - X
    dy = f32(y) - Y
    power = _power32(a, b, c, dx, dy).astype(np.float32)
    G = np.exp2(power.astype(np.float64)) * (1.0 + EXP_ERR)
    alpha = np.minimum(0.99, np.float64(o) * G)
    act = (alpha >= 1.0 / 255.0) & ~(power > 0)
    return Y[act]


def test_row_extent_contains_every_blending_pixel():
    rng = np.random.default_rng(11)
    checked = 0
    for (x, y, a, b, c, o) in _splats(rng, 600):
        rows = _active_rows(x, y, a, b, c, o, rng)
        for log_err in (-3e-6, 3e-6):
            r = _rows(y, a, b, c, o, log_err)
            if r is None or rows.size == 0:
                continue
            lo, hi = r
            assert rows.min() >= lo and rows.max() <= hi, (x, y, a, b, c, o, lo, hi,
                                                           rows.min(), rows.max())
            checked += 1
    assert checked > 500


def test_row_extent_at_the_ellipse_tip():
    """Pixels placed at the top and bottom tips of the alpha = 1/255 ellipse
    (scaled by 1 - eps, so they blend): each must lie inside the extent."""
    rng = np.random.default_rng(13)
    hits = 0
    for (x0, y0, a, b, c, o) in _splats(rng, 400):
        det = np.float64(a) * np.float64(c) - np.float64(b) ** 2
        tau = 2.0 * np.log(255.0 * np.float64(o))
        if tau <= 0:
            continue
        dy = np.sqrt(tau * np.float64(a) / det)
        dx = -np.float64(b) * dy / np.float64(a)
        for eps in (1e-7, 1e-6, 1e-5, 1e-4):
            for sgn in (1.0, -1.0):
                # pixel (0, 0); centre so that the pixel is at the tip
                x = f32(-sgn * dx * (1 - eps))
                y = f32(-sgn * dy * (1 - eps))
                fx, fy = f32(x - f32(0.0)), f32(y - f32(0.0))
                power = _power32(a, b, c, fx, fy)
                alpha = min(0.99, np.float64(o) * np.exp2(np.float64(power)) * (1 + EXP_ERR))
                if not (alpha >= 1.0 / 255.0) or power > 0:
                    continue
                for log_err in (-3e-6, 3e-6):
                    r = _rows(y, a, b, c, o, log_err)
                    if r is None:
                        continue
                    assert r[0] <= 0.0 <= r[1], (a, b, c, o, eps, x, y, r)
                    hits += 1
    assert hits > 1000


def test_row_extent_is_tight():
    """The extent exceeds the exact ellipse by no more than its margins
    (1 % in q, 0.1 % in rows, a quarter pixel)."""
    rng = np.random.default_rng(12)
    for (x, y, a, b, c, o) in _splats(rng, 200):
        r = _rows(y, a, b, c, o, 0.0)
        if r is None or not np.isfinite(r[0]) or r[0] > r[1]:
            continue
        det = np.float64(a) * np.float64(c) - np.float64(b) ** 2
        tau = max(2.0 * np.log(255.0 * np.float64(o)), 0.0)
        exact = np.sqrt(tau * np.float64(a) / det)
        half = (np.float64(r[1]) - np.float64(r[0])) / 2
        bound = np.sqrt((1.01 * tau + 0.05) * np.float64(a) / det) * 1.001 + 0.25
        assert exact <= half + 1e-3 * max(1.0, exact)
        assert half <= bound * (1 + 1e-4) + 1e-3
