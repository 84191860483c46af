"""Pins the oracle's deterministic exp/log and its SH basis against mathematics.

orc_expf / orc_logf / orc_blend_exp2f are the transcendental functions both
the oracle and the HIP kernels implement with the same IEEE operations; here
they are checked against float64 numpy within their stated bounds, and the
base-2 blend exponent splat_power against log2(e) times the float64 quadratic
form.  The SH basis of orc_color_from_sh
(fastgs_preprocess.metal:117-169) is checked function by function against
scipy's spherical harmonics (which carry the Condon-Shortley phase), at the
six axis directions, the eight cube diagonals and random directions: a
flipped sign, a swapped index or a wrong constant of any one of the 16
functions fails it.  Orthonormality on the sphere and the degree truncation
are checked as well.
"""
import numpy as np
from scipy.special import sph_harm_y


def test_expf_error_bound(oracle):
    xs = np.concatenate([np.linspace(-87.0, 0.0, 20001), -np.logspace(-8, 1.9, 2000),
                         np.array([0.0, -1e-30, -0.5, -1.0, -5.54])]).astype(np.float32)
    got = np.array([oracle.expf(float(x)) for x in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    rel = np.abs(got - ref) / ref
    assert rel.max() < 2e-7, rel.max()  # ~1.5 ulp
    assert oracle.expf(0.0) == 1.0
    # monotone non-decreasing on the grid
    order = np.argsort(xs, kind="stable")
    assert np.all(np.diff(got[order]) >= 0)


def test_blend_exp2f_error_bound(oracle):
    """orc_blend_exp2f (2^t for the rasterizer's base-2 blend exponent):
    relative error at most 2e-7 against float64 exp2, point by point over
    [-126, 0] and densely over [-8, 0], where alpha >= 1/255 can hold; exact
    at 0 and at the integers.  Just below 0, t - floor(t) rounds to 1 and is
    clamped to 0x1.fffffep-1 as v_fract_f32 does; the result stays within the
    bound there."""
    rng = np.random.default_rng(1)
    ts = np.concatenate([np.linspace(-126.0, 0.0, 20001), rng.uniform(-8.0, 0.0, 40000),
                         -np.logspace(-12, 2.1, 3000),
                         np.array([0.0, -1e-30, -2.0 ** -26, -2.0 ** -25, -0.5, -1.0, -8.0,
                                   -125.99])]).astype(np.float32)
    got = np.array([oracle.blend_exp2f(float(t)) for t in ts], np.float64)
    ref = np.exp2(ts.astype(np.float64))
    rel = np.abs(got - ref) / ref
    assert rel.max() < 2.0e-7, rel.max()
    for k in range(-126, 1):
        assert oracle.blend_exp2f(float(k)) == 2.0 ** k
    # below the clamp the value is that of -126
    assert oracle.blend_exp2f(-1000.0) == 2.0 ** -126
    assert oracle.blend_exp2f(float("-inf")) == 2.0 ** -126


def test_splat_power_error_bound(oracle):
    """splat_power (oracle and kernels): fma(dy, fma(C, dy, B dx), (A dx) dx)
    with A = (-a/2) log2(e), B = -b log2(e), C = (-c/2) log2(e) equals
    log2(e) (-1/2 (a dx^2 + c dy^2) - b dx dy) within
    (4 * 2^-24 + 1.4e-8) log2(e) (a dx^2 / 2 + |b dx dy| + c dy^2 / 2): three
    roundings of the evaluation, one of each coefficient, and log2(e) rounded
    to float (1.34e-8 relative); a sign slip or a dropped term is far outside
    it."""
    rng = np.random.default_rng(2)
    n = 20000
    a = np.exp(rng.uniform(-8, 2, n)).astype(np.float32)
    c = np.exp(rng.uniform(-8, 2, n)).astype(np.float32)
    rho = rng.uniform(-0.999, 0.999, n)
    b = (rho * np.sqrt(a.astype(np.float64) * c)).astype(np.float32)
    dx = rng.uniform(-40, 40, n).astype(np.float32)
    dy = rng.uniform(-40, 40, n).astype(np.float32)
    A, B, C, X, Y = (v.astype(np.float64) for v in (a, b, c, dx, dy))
    L = np.log2(np.e)
    exact = L * (-0.5 * (A * X * X + C * Y * Y) - B * X * Y)
    scale = L * (0.5 * A * X * X + np.abs(B * X * Y) + 0.5 * C * Y * Y)
    got = np.array([oracle.splat_power(*v) for v in zip(a, b, c, dx, dy)])
    err = np.abs(got - exact)
    assert np.all(err <= (4 * 2.0 ** -24 + 1.4e-8) * scale + 1e-30), (err / scale).max()
    # known answers: each term alone, with the sign of the reference's power
    Lf = float(np.float32(L))
    assert oracle.splat_power(2.0, 0.0, 0.0, 1.0, 0.0) == -Lf
    assert oracle.splat_power(0.0, 0.0, 2.0, 0.0, 1.0) == -Lf
    assert oracle.splat_power(0.0, 1.0, 0.0, 1.0, 1.0) == -Lf
    assert oracle.splat_power(0.0, 1.0, 0.0, 1.0, -1.0) == Lf


def test_logf_error_bound(oracle):
    rng = np.random.default_rng(0)
    xs = np.concatenate([np.exp(rng.uniform(-80, 80, 20000)), rng.uniform(0.5, 2.0, 5000),
                         np.array([1.0, 255.0, 1 / 255.0, 2.0, 0.70710677, 1.4142135])])
    xs = xs.astype(np.float32)
    got = np.array([oracle.logf(float(x)) for x in xs], np.float64)
    ref = np.log(xs.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(got - ref) / np.maximum(ulp, 1e-45)
    assert err.max() <= 0.5000001, err.max()  # correctly rounded
    assert oracle.logf(1.0) == 0.0
    assert np.isneginf(oracle.logf(0.0))
    assert np.isnan(oracle.logf(-1.0))


def _fibonacci_sphere(n):
    i = np.arange(n) + 0.5
    phi = np.arccos(1 - 2 * i / n)
    theta = np.pi * (1 + 5 ** 0.5) * i
    return np.stack([np.cos(theta) * np.sin(phi), np.sin(theta) * np.sin(phi), np.cos(phi)], 1)


def _sh_basis_scipy(dirs):
    """The 16 real SH functions of degree <= 3 in the coefficient order of
    fastgs_preprocess.metal:117-169 (k = l*l + l + m, m = -l..l), from scipy's
    complex Y_l^m (Condon-Shortley phase included):
    sqrt(2) Im Y_l^|m| for m < 0, Y_l^0 for m = 0, sqrt(2) Re Y_l^m for m > 0."""
    d = dirs / np.linalg.norm(dirs, axis=1, keepdims=True)
    theta = np.arccos(np.clip(d[:, 2], -1.0, 1.0))  # polar angle from +z
    phi = np.arctan2(d[:, 1], d[:, 0])  # azimuth from +x towards +y
    out = np.zeros((16, d.shape[0]))
    for l in range(4):
        for m in range(-l, l + 1):
            y = sph_harm_y(l, abs(m), theta, phi)
            if m < 0:
                v = np.sqrt(2.0) * y.imag
            elif m == 0:
                v = y.real
            else:
                v = np.sqrt(2.0) * y.real
            out[l * l + l + m] = v
    return out


def _sh_basis_oracle(oracle64, dirs):
    """Y_k(dir) read back through orc_color_from_sh: coefficient k = 0.1, the
    others 0, colour = 0.5 + 0.1 Y_k (no clamp at |Y_k| <= 1.1)."""
    Y = np.zeros((16, dirs.shape[0]))
    for k in range(16):
        dc = np.zeros(3)
        sh = np.zeros((15, 3))
        if k == 0:
            dc[0] = 0.1
        else:
            sh[k - 1, 0] = 0.1
        for j in range(dirs.shape[0]):
            col, clamped = oracle64.color_from_sh(3, dirs[j], np.zeros(3), dc, sh)
            assert not clamped.any()
            Y[k, j] = (col[0] - 0.5) / 0.1
    return Y


def test_sh_basis_against_scipy(oracle64):
    """Each of the 16 basis functions, sign included, equals scipy's at the axis
    directions, the cube diagonals and random directions."""
    axes = np.concatenate([np.eye(3), -np.eye(3)])
    diag = np.array([[sx, sy, sz] for sx in (1, -1) for sy in (1, -1) for sz in (1, -1)], float)
    rng = np.random.default_rng(7)
    rand = rng.standard_normal((40, 3))
    dirs = np.concatenate([axes, diag, rand])
    got = _sh_basis_oracle(oracle64, dirs)
    ref = _sh_basis_scipy(dirs)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-6)
    # the check separates every pair of functions and both signs of each
    for k in range(16):
        assert np.abs(ref[k]).max() > 0.1
        for j in range(16):
            if j != k:
                assert np.abs(ref[k] - ref[j]).max() > 0.1 and np.abs(ref[k] + ref[j]).max() > 0.1


def test_sh_basis_known_values(oracle64):
    """Hand-evaluated values of the degree-1 functions at the axes and of a
    few higher ones at (1,1,1)/sqrt3, from the closed forms
    Y_1 = -c1 y, c1 z, -c1 x with c1 = sqrt(3/(4 pi))."""
    c1 = np.sqrt(3.0 / (4.0 * np.pi))
    got = _sh_basis_oracle(oracle64, np.concatenate([np.eye(3), np.ones((1, 3))]))
    np.testing.assert_allclose(got[1:4, 0], [0.0, 0.0, -c1], atol=1e-7)  # +x
    np.testing.assert_allclose(got[1:4, 1], [-c1, 0.0, 0.0], atol=1e-7)  # +y
    np.testing.assert_allclose(got[1:4, 2], [0.0, c1, 0.0], atol=1e-7)  # +z
    # at (1,1,1)/sqrt3: xy = yz = xz = 1/3, 2zz - xx - yy = 0, xx - yy = 0
    c2 = 0.5 * np.sqrt(15.0 / np.pi)
    np.testing.assert_allclose(got[4:9, 3], [c2 / 3, -c2 / 3, 0.0, -c2 / 3, 0.0], atol=1e-7)
    # degree 3 at (1,1,1)/sqrt3: xyz = 3^-1.5, the other six vanish or cancel
    # except y(4zz-xx-yy) = x(4zz-xx-yy) = 2/3^1.5, y(3xx-yy) = 2/3^1.5,
    # z(2zz-3xx-3yy) = -4/3^1.5, x(xx-3yy) = -2/3^1.5
    s3 = 3.0 ** -1.5
    k31 = 0.25 * np.sqrt(35.0 / (2 * np.pi))  # |m| = 3
    k32 = 0.5 * np.sqrt(105.0 / np.pi)        # |m| = 2
    k33 = 0.25 * np.sqrt(21.0 / (2 * np.pi))  # |m| = 1
    k30 = 0.25 * np.sqrt(7.0 / np.pi)         # m = 0
    want3 = [-k31 * 2 * s3, k32 * s3, -k33 * 2 * s3, k30 * -4 * s3, -k33 * 2 * s3, 0.0,
             -k31 * -2 * s3]
    np.testing.assert_allclose(got[9:16, 3], want3, atol=1e-7)


def test_sh_basis_orthonormal(oracle64):
    """Y_k(dir) read back through orc_color_from_sh (coefficient k = 0.1, others 0):
    the 16 real SH functions of degree <= 3 are orthonormal on the unit sphere."""
    dirs = _fibonacci_sphere(4000)
    n = dirs.shape[0]
    Y = np.zeros((16, n))
    for k in range(16):
        dc = np.zeros(3)
        sh = np.zeros((15, 3))
        if k == 0:
            dc[0] = 0.1
        else:
            sh[k - 1, 0] = 0.1
        for j in range(n):
            col, clamped = oracle64.color_from_sh(3, dirs[j], np.zeros(3), dc, sh)
            assert not clamped.any()
            Y[k, j] = (col[0] - 0.5) / 0.1
    gram = Y @ Y.T * (4 * np.pi / n)
    np.testing.assert_allclose(gram, np.eye(16), atol=2e-3)


def test_sh_degree_truncation(oracle64):
    """Degree d uses exactly the first (d+1)^2 - 1 rest coefficients."""
    rng = np.random.default_rng(1)
    dirv = rng.standard_normal(3)
    dc = rng.uniform(0, 1, 3)
    sh = rng.normal(0, 0.05, (15, 3))
    for d, used in ((0, 0), (1, 3), (2, 8), (3, 15)):
        a, _ = oracle64.color_from_sh(d, dirv, np.zeros(3), dc, sh)
        sh2 = sh.copy()
        sh2[used:] += 1.0  # perturb the unused coefficients only
        b, _ = oracle64.color_from_sh(d, dirv, np.zeros(3), dc, sh2)
        np.testing.assert_array_equal(a, b)
        if used < 15:
            c, _ = oracle64.color_from_sh(d + 1, dirv, np.zeros(3), dc, sh2)
            assert np.abs(c - a).max() > 1e-6
