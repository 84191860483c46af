"""Pins the oracle's deterministic exp/log and its SH basis against mathematics.

orc_expf / orc_logf are the transcendental functions both the oracle and the
HIP kernels implement with the same IEEE operations; here they are checked
against float64 numpy within a few ulp.  The SH basis of orc_color_from_sh
(fastgs_preprocess.metal:117-169) is checked for orthonormality on the
sphere, which a dropped term, a wrong constant or a wrong coefficient index
breaks.
"""
import numpy as np


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
