"""Pins the oracle's tile footprint, duplication, sort, scan and compositing by
brute force and invariants (tiles_walk restates fastgs_preprocess.metal:247-382
and fastgs_binning.metal:23-180)."""
import numpy as np
import pytest

from fastgs_core_amd import synthetic as syn


def _min_q_over_rect(px, py, a, b, c, x0, x1, y0, y1):
    """min over [x0,x1]x[y0,y1] of q = a dx^2 + 2 b dx dy + c dy^2 (convex)."""
    if x0 <= px <= x1 and y0 <= py <= y1:
        return 0.0
    best = np.inf
    for xe in (x0, x1):
        dx = xe - px
        dy = np.clip(-b * dx / c, y0 - py, y1 - py)
        best = min(best, a * dx * dx + 2 * b * dx * dy + c * dy * dy)
    for ye in (y0, y1):
        dy = ye - py
        dx = np.clip(-b * dy / a, x0 - px, x1 - px)
        best = min(best, a * dx * dx + 2 * b * dx * dy + c * dy * dy)
    return best


def _brute_tiles(px, py, co, gx, gy, mult=1.0):
    a, b, c, o = co
    t = mult * 2 * np.log(255 * o)
    sure, ambiguous = set(), set()
    for ty in range(gy):
        for tx in range(gx):
            m = _min_q_over_rect(px, py, a, b, c, 16 * tx, 16 * tx + 16, 16 * ty, 16 * ty + 16)
            if m < t * (1 - 1e-4) - 1e-9:
                sure.add(ty * gx + tx)
            elif m <= t * (1 + 1e-4) + 1e-9:
                ambiguous.add(ty * gx + tx)
    return sure, ambiguous


@pytest.mark.parametrize("double", [True, False])
def test_tile_footprint_matches_brute_force(oracle, oracle64, double):
    orc = oracle64 if double else oracle
    rng = np.random.default_rng(3 if double else 4)
    gx, gy = 8, 7
    checked = 0
    for _ in range(400):
        ev = np.exp(rng.uniform(np.log(0.5), np.log(600), 2))
        th = rng.uniform(0, np.pi)
        Rm = np.array([[np.cos(th), -np.sin(th)], [np.sin(th), np.cos(th)]])
        cov = Rm @ np.diag(ev) @ Rm.T
        con = np.linalg.inv(cov)
        o = rng.uniform(0.01, 1.0)
        co = np.array([con[0, 0], con[0, 1], con[1, 1], o])
        co = co.astype(np.float32).astype(np.float64)
        px, py = [float(np.float32(v)) for v in rng.uniform(-20, 150, 2)]
        sure, amb = _brute_tiles(px, py, co, gx, gy)
        cnt = orc.tiles_touched_one(px, py, co, gx, gy)
        keys, vals = orc.duplicate_with_keys(np.array([[px, py]]), np.array([5.0]),
                                             np.array([cnt]), np.array([co]), np.array([cnt]),
                                             1.0, gx, gy, cnt)
        got = [int(k >> 32) for k in keys]
        assert len(set(got)) == len(got), "a Gaussian emitted a tile twice"
        got = set(got)
        if o < 1 / 255:
            assert cnt == 0
            continue
        assert sure <= got, (sure - got)
        assert got <= (sure | amb), (got - sure - amb)
        checked += 1
    assert checked > 300


def test_scene_invariants(oracle):
    sc, cam = syn.scene_config2(0, 3000, 3), syn.sphere_cameras(1, 9, 160, 120, 3.0)[0]
    sc["means3d"] *= 0.5
    sc["scales"] *= 4
    inp = syn.make_inputs(sc, cam)
    f = oracle.render(inp, 160, 120, cam.tan_fovx, cam.tan_fovy, 3)
    tt = f["geom_tiles_touched"].astype(np.int64)
    assert int(tt.sum()) == f["rendered"] > 0
    assert ((f["radii"] > 0) == (tt > 0)).all()
    keys = f["point_list_keys_unsorted"]
    vals = f["point_list_unsorted"]
    offs = np.concatenate([[0], f["point_offsets"].astype(np.int64)])
    for g in np.nonzero(tt)[0][:500]:
        seg = keys[offs[g]:offs[g + 1]]
        assert (vals[offs[g]:offs[g + 1]] == g).all()
        tiles = seg >> np.uint64(32)
        assert len(np.unique(tiles)) == len(tiles)
        assert ((seg & np.uint64(0xFFFFFFFF)) == np.float32(f["geom_depths"][g]).view(np.uint32)).all()
    # sorted keys non-decreasing; permutation of the unsorted pairs
    sk = f["point_list_keys"]
    assert (sk[1:] >= sk[:-1]).all()
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(sk, keys[order])
    np.testing.assert_array_equal(f["point_list"], vals[order])
    # ranges partition [0, K) in tile order
    r = f["ranges"].astype(np.int64)
    touched = r[:, 1] > r[:, 0]
    assert (r[touched, 1] - r[touched, 0]).sum() == f["rendered"]
    np.testing.assert_array_equal(f["bucket_count"], (r[:, 1] - r[:, 0] + 31) // 32)
    np.testing.assert_array_equal(f["bucket_offsets"], np.cumsum(f["bucket_count"]))


def test_sort_is_stable_radix(oracle):
    rng = np.random.default_rng(1)
    keys = (rng.integers(0, 50, 20000).astype(np.uint64) << np.uint64(32)) | \
        rng.integers(0, 30, 20000).astype(np.uint64)
    vals = np.arange(20000, dtype=np.uint32)
    k, v = oracle.sort_pairs(keys, vals)
    order = np.argsort(keys, kind="stable")
    np.testing.assert_array_equal(k, keys[order])
    np.testing.assert_array_equal(v, vals[order])


def test_scan_wraps_u32(oracle):
    rng = np.random.default_rng(2)
    x = rng.integers(0, 2 ** 31, 5000).astype(np.uint32)
    np.testing.assert_array_equal(oracle.inclusive_scan(x),
                                  (np.cumsum(x.astype(np.uint64)) % (1 << 32)).astype(np.uint32))


def test_compositing_matches_brute_force(oracle64):
    """Tiled blend == per-pixel depth-ordered compositing over all visible Gaussians."""
    rng = np.random.default_rng(5)
    sc = syn.scene_config1(3, 60)
    sc["scales"] = np.exp(rng.normal(-2.5, 0.4, (60, 3)))
    cam = syn.look_at_camera((0.4, 0.3, -3.5), (0, 0, 0), 40, 36)
    inp = syn.make_inputs(sc, cam, background=(0.1, 0.2, 0.3))
    f = oracle64.render(inp, 40, 36, cam.tan_fovx, cam.tan_fovy, 0)
    pre = f["pre"]
    vis = np.nonzero(pre["radii"] > 0)[0]
    order = vis[np.argsort(pre["depths"][vis].astype(np.float32).view(np.uint32), kind="stable")]
    img = np.zeros((3, 36, 40))
    for y in range(36):
        for x in range(40):
            T, C = 1.0, np.zeros(3)
            for g in order:
                dx, dy = pre["xys"][g] - (x, y)
                a, b, c, o = pre["conic_opacity"][g]
                power = -0.5 * (a * dx * dx + c * dy * dy) - b * dx * dy
                if power > 0:
                    continue
                al = min(0.99, o * np.exp(power))
                if al < 1 / 255:
                    continue
                if T * (1 - al) < 1e-4:
                    break
                C += pre["rgb"][g] * al * T
                T *= 1 - al
            img[:, y, x] = C + T * np.array([0.1, 0.2, 0.3])
    np.testing.assert_allclose(f["out_color"].reshape(3, 36, 40), img, atol=1e-9)
