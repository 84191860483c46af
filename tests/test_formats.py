"""On-disk formats (CPU): PLY point clouds, the .spz container, scanner
camera JSON and dataset preparation (fastgs_core_amd.ply / .spz / .scanner).

Pins, since neither ``plyfile`` nor the ``spz`` binding is installed and the
reference ships no data files:
* PLY: hand-assembled byte files in all three encodings (known answers),
  element skipping with list properties, writer round trips;
* spz: header and per-field bytes against the format's closed forms,
  half-way rounding, decode(encode(x)) within one quantisation step, the
  smallest-three quaternions, and the coordinate conversion against the
  mathematics it must satisfy (R(q') = F R(q) F, SH colour invariant under
  the flipped view direction, through the oracle's SH evaluation);
* cameras: the pinhole projection of points in front of a scanner pose
  lands at the pixel the intrinsics give, with positive view depth.
"""
import gzip
import json
import math
import struct

import numpy as np
import pytest

from fastgs_core_amd import ply, scanner, spz


# ---------------------------------------------------------------- PLY
def _ply_bytes(fmt, body, extra_header=""):
    head = (f"ply\nformat {fmt} 1.0\ncomment made by hand\n{extra_header}"
            "element vertex 2\nproperty float x\nproperty float y\nproperty float z\n"
            "property uchar red\nproperty uchar green\nproperty uchar blue\n"
            "element face 1\nproperty list uchar int vertex_indices\nend_header\n")
    return head.encode() + body


def test_ply_known_answers(tmp_path):
    want_xyz = np.array([[1.5, -2.0, 0.25], [0.0, 3.0, -1.0]], np.float32)
    want_rgb = np.array([[255, 0, 51], [10, 20, 30]], np.uint8)
    face = [0, 1, 1]
    for fmt, order in (("binary_little_endian", "<"), ("binary_big_endian", ">")):
        body = b""
        for p, c in zip(want_xyz, want_rgb):
            body += struct.pack(order + "fff", *p) + bytes(c)
        body += struct.pack(order + "B", 3) + struct.pack(order + "iii", *face)
        path = tmp_path / f"{fmt}.ply"
        path.write_bytes(_ply_bytes(fmt, body))
        got = ply.read_ply(path)
        np.testing.assert_array_equal(np.stack([got["vertex"][k] for k in "xyz"], 1), want_xyz)
        np.testing.assert_array_equal(got["vertex"]["red"], want_rgb[:, 0])
        assert got["vertex"]["red"].dtype == np.uint8
        np.testing.assert_array_equal(got["face"]["vertex_indices"][0], face)
    body = b"1.5 -2 0.25 255 0 51\n0 3 -1 10 20 30\n3 0 1 1\n"
    path = tmp_path / "ascii.ply"
    path.write_bytes(_ply_bytes("ascii", body))
    pts, cols = scanner.load_ply_positions_colors(path)
    np.testing.assert_array_equal(pts, want_xyz)
    np.testing.assert_allclose(cols, want_rgb / 255.0, rtol=1e-7)


def test_ply_vertex_after_list_element_and_float_colours(tmp_path):
    """A list element before the vertices is walked; float colours in [0,1]
    are kept (no /255), colours above 1 are scaled, then clipped."""
    head = ("ply\nformat binary_little_endian 1.0\nelement face 2\n"
            "property list uchar uint vertex_indices\nelement vertex 3\nproperty double x\n"
            "property double y\nproperty double z\nproperty float red\nproperty float green\n"
            "property float blue\nend_header\r\n")
    body = struct.pack("<B3I", 3, 0, 1, 2) + struct.pack("<B4I", 4, 0, 1, 2, 0)
    rows = [(0.1, 0.2, 0.3, 0.5, 1.0, 0.0), (1, 2, 3, 0.25, 0.75, 1.0), (-1, -2, -3, 0, 0, 0.5)]
    for r in rows:
        body += struct.pack("<3d3f", *r)
    path = tmp_path / "f.ply"
    path.write_bytes(head.encode() + body)
    pts, cols = scanner.load_ply_positions_colors(path)
    np.testing.assert_array_equal(pts, np.float32([r[:3] for r in rows]))
    np.testing.assert_array_equal(cols, np.float32([r[3:] for r in rows]))
    # uchar-range floats are divided by 255 and clipped
    ply.write_ply(path, {"vertex": {"x": np.float32([0, 1]), "y": np.float32([0, 0]),
                                    "z": np.float32([0, 0]), "red": np.float32([300, 51]),
                                    "green": np.float32([0, 255]), "blue": np.float32([-5, 0])}})
    _, cols = scanner.load_ply_positions_colors(path)
    np.testing.assert_allclose(cols, [[1.0, 0.0, 0.0], [0.2, 1.0, 0.0]], rtol=1e-6)


@pytest.mark.parametrize("fmt", ["ascii", "binary_little_endian", "binary_big_endian"])
def test_ply_writer_round_trip(tmp_path, fmt):
    rng = np.random.default_rng(0)
    el = {"vertex": {"x": rng.normal(size=50).astype(np.float32),
                     "y": rng.normal(size=50).astype(np.float64),
                     "red": rng.integers(0, 256, 50).astype(np.uint8),
                     "n": rng.integers(-1000, 1000, 50).astype(np.int32)},
          "extra": {"v": np.arange(3, dtype=np.uint16)}}
    path = tmp_path / "rt.ply"
    ply.write_ply(path, el, fmt=fmt, comments=["round trip"])
    got = ply.read_ply(path)
    for e, props in el.items():
        for k, v in props.items():
            assert got[e][k].dtype == v.dtype
            np.testing.assert_array_equal(got[e][k], v)
    assert list(ply.read_ply(path, elements=["vertex"])) == ["vertex"]


def test_ply_rejects_malformed(tmp_path):
    p = tmp_path / "bad.ply"
    p.write_bytes(b"ply\nformat binary_little_endian 1.0\nelement vertex 10\nproperty float x\n"
                  b"end_header\n" + b"\0" * 8)
    with pytest.raises(ply.PlyError):
        ply.read_ply(p)
    p.write_bytes(b"not a ply")
    with pytest.raises(ply.PlyError):
        ply.read_ply(p)


# ---------------------------------------------------------------- spz
def _cloud(n=64, deg=3, seed=0):
    rng = np.random.default_rng(seed)
    dim = spz.SH_DIM[deg]
    return spz.GaussianCloud(
        positions=rng.uniform(-50, 50, 3 * n).astype(np.float32),
        scales=rng.uniform(-9, 5, 3 * n).astype(np.float32),
        rotations=rng.standard_normal(4 * n).astype(np.float32),
        alphas=rng.normal(0, 2, n).astype(np.float32),
        colors=rng.normal(0, 1, 3 * n).astype(np.float32),
        sh=rng.uniform(-0.9, 0.9, n * dim * 3).astype(np.float32), sh_degree=deg,
        antialiased=True)


def test_spz_bytes_closed_form():
    c = spz.GaussianCloud(
        positions=np.float32([1 / 8192, -1 / 8192, 1.0, -2.5, 0.0, 2047.0]),
        scales=np.float32([-10, -4.5, 5.9375, 0, -11, 10]),
        rotations=np.float32([0, 0, 0, 1, 0, 0, 0, -2]),   # identity, then -identity
        alphas=np.float32([0.0, 100.0]),
        colors=np.float32([0.0, 1.0, -4.0, 0.1, 0.0, 0.0]),
        sh=np.zeros(2 * 3 * 3, np.float32), sh_degree=1, antialiased=True)
    c.sh[0], c.sh[1], c.sh[9] = 0.1, -0.0546875, 0.1
    raw = spz.pack_gaussians(c)
    assert raw[:16] == struct.pack("<IIIBBBB", 0x5053474E, 2, 2, 1, 12, 1, 0)
    pos = np.frombuffer(raw[16:34], np.uint8).reshape(6, 3)
    # 0.5 -> 1 (half away from zero), -0.5 -> -1, 4096, -10240, 0, 2047*4096 (24-bit)
    want = [1, -1, 4096, -10240, 0, 2047 * 4096]
    for row, v in zip(pos, want):
        assert int(row[0]) | int(row[1]) << 8 | int(row[2]) << 16 == v & 0xFFFFFF
    off = 34
    alphas = np.frombuffer(raw[off:off + 2], np.uint8)
    np.testing.assert_array_equal(alphas, [128, 255])  # 127.5 rounds up; saturates
    colors = np.frombuffer(raw[off + 2:off + 8], np.uint8)
    np.testing.assert_array_equal(colors, [128, 166, 0, 131, 128, 128])  # 165.75, 131.325
    scales = np.frombuffer(raw[off + 8:off + 14], np.uint8)
    np.testing.assert_array_equal(scales, [0, 88, 255, 160, 0, 255])
    rots = np.frombuffer(raw[off + 14:off + 20], np.uint8)
    np.testing.assert_array_equal(rots, [128, 128, 128, 128, 128, 128])  # w < 0 negated
    sh = np.frombuffer(raw[off + 20:off + 38], np.uint8)
    # degree 1: all 9 values per point in buckets of 8.  0.1 -> round(12.8) + 128 = 141 -> 144;
    # -0.0546875 -> -7 + 128 = 121 -> 120; 0 -> 128 (a bucket centre); index 9 is point 2's first
    assert sh[0] == 144 and sh[1] == 120 and sh[9] == 144 and sh[2] == 128


def test_spz_sh_buckets_degree3():
    c = _cloud(1, 3)
    c.sh[:] = 0.0
    c.sh[8] = 0.1    # last degree-1 value: bucket 8
    c.sh[9] = 0.1    # first degree-2 value: bucket 16
    c.sh[10] = 0.17  # round(21.76) + 128 = 150 -> bucket 16: 144
    raw = spz.pack_gaussians(c)
    sh = np.frombuffer(raw[-45:], np.uint8)
    assert (sh[8], sh[9], sh[10]) == (144, 144, 144)
    c.sh[10] = 0.19  # round(24.32) = 24 -> 152 -> (152 + 8) // 16 * 16 = 160
    assert np.frombuffer(spz.pack_gaussians(c)[-45:], np.uint8)[10] == 160


@pytest.mark.parametrize("version", [2, 3])
def test_spz_round_trip(tmp_path, version):
    c = _cloud(300, 3, seed=version)
    path = tmp_path / "c.spz"
    assert spz.save_spz(c, spz.PackOptions(version=version), str(path))
    blob = path.read_bytes()
    assert blob[:2] == b"\x1f\x8b"  # gzip
    d = spz.load_spz(path)
    assert d.num_points == 300 and d.sh_degree == 3 and d.antialiased
    assert gzip.decompress(blob) == spz.pack_gaussians(c, spz.PackOptions(version=version))
    np.testing.assert_allclose(d.positions, c.positions, atol=0.5 / 4096 + 1e-6)
    np.testing.assert_allclose(d.scales, c.scales, atol=0.5 / 16 + 1e-6)
    np.testing.assert_allclose(1 / (1 + np.exp(-d.alphas)), 1 / (1 + np.exp(-c.alphas)),
                               atol=0.5 / 255 + 1e-6)
    np.testing.assert_allclose(d.colors, np.clip(c.colors, -127.5 / 38.25, 127.5 / 38.25),
                               atol=0.5 / 38.25 + 1e-6)
    q = c.rotations.reshape(-1, 4)
    q = q / np.linalg.norm(q, axis=1, keepdims=True)
    dq = d.rotations.reshape(-1, 4)
    dots = np.abs((q * dq).sum(axis=1))
    assert dots.min() > (0.995 if version == 2 else 0.99995)
    # SH: 5-bit buckets for degree 1, 4-bit for the rest
    sh = c.sh.reshape(-1, 45)
    dsh = d.sh.reshape(-1, 45)
    assert np.abs(dsh[:, :9] - sh[:, :9]).max() <= 4.5 / 128
    assert np.abs(dsh[:, 9:] - sh[:, 9:]).max() <= 8.5 / 128


def test_spz_smallest_three_layout():
    """Largest |component| index in bits 30-31, then (sign, 9-bit magnitude)
    per other component, the first in the highest bits; the largest is made
    positive (q and -q are one rotation)."""
    q = np.float32([[0.1, -0.2, -0.9, 0.3]])  # xyzw, largest = z (index 2), negative
    q = q / np.linalg.norm(q)
    b = spz._smallest_three(q)
    comp = int(b[0, 0]) | int(b[0, 1]) << 8 | int(b[0, 2]) << 16 | int(b[0, 3]) << 24
    assert comp >> 30 == 2
    s = 511 / math.sqrt(0.5)
    fields = [(comp >> 20) & 1023, (comp >> 10) & 1023, comp & 1023]  # x, y, w
    for f, v in zip(fields, (q[0, 0], q[0, 1], q[0, 3])):
        neg = (v < 0) ^ True  # sign relative to the flipped quaternion
        assert (f >> 9) == int(neg)
        mag = np.float32(511) * (np.float32(abs(v)) / np.float32(math.sqrt(0.5))) + np.float32(0.5)
        assert f & 511 == int(mag) and abs(int(mag) - abs(float(v)) * s) <= 0.5 + 1e-4
    back = spz._unpack_smallest_three(b)
    np.testing.assert_allclose(back[0], -q[0], atol=2e-3)


def _rotmat_xyzw(q):
    x, y, z, w = q / np.linalg.norm(q)
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
                     [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
                     [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)]])


def test_spz_coordinate_conversion_invariants(oracle64):
    rng = np.random.default_rng(4)
    n = 8
    pos = rng.normal(size=3 * n).astype(np.float32)
    rot = rng.standard_normal(4 * n).astype(np.float32)
    sh = rng.normal(0, 0.3, n * 45).astype(np.float32)
    for cs in spz.CoordinateSystem:
        if cs == spz.CoordinateSystem.UNSPECIFIED:
            continue
        f = spz._flips(cs, spz.CoordinateSystem.RUB)
        F = np.diag(f)
        p2, r2, s2 = spz._convert(pos, rot, sh, 15, f)
        np.testing.assert_array_equal(p2.reshape(-1, 3), pos.reshape(-1, 3) * np.float32(f))
        for i in range(n):
            R = _rotmat_xyzw(rot[4 * i:4 * i + 4].astype(np.float64))
            R2 = _rotmat_xyzw(r2[4 * i:4 * i + 4].astype(np.float64))
            np.testing.assert_allclose(R2, F @ R @ F, atol=1e-6)
            d = rng.normal(size=3)
            dc = rng.uniform(0, 1, 3)
            a, _ = oracle64.color_from_sh(3, d, np.zeros(3), dc, sh[45 * i:45 * i + 45])
            b, _ = oracle64.color_from_sh(3, F @ d, np.zeros(3), dc, s2[45 * i:45 * i + 45])
            np.testing.assert_allclose(a, b, atol=1e-6)
        # pack from cs, unpack to cs: the cloud comes back (quantisation aside)
        c = _cloud(16, 3, seed=int(cs))
        d2 = spz.unpack_gaussians(spz.pack_gaussians(c, spz.PackOptions(from_coord=cs)),
                                  spz.UnpackOptions(to_coord=cs))
        np.testing.assert_allclose(d2.positions, c.positions, atol=0.5 / 4096 + 1e-6)


def test_spz_rejects_inconsistent_cloud():
    c = _cloud(4, 2)
    c.sh = c.sh[:-1]
    with pytest.raises(spz.SpzError):
        spz.pack_gaussians(c)
    with pytest.raises(spz.SpzError):
        spz.unpack_gaussians(b"\0" * 16)


# -------------------------------------------------------------- cameras
def _pose(rng):
    q = rng.standard_normal(4)
    R = scanner.quaternions_wxyz_to_rotation_matrices(q[None].astype(np.float32))[0]
    c2w = np.eye(4, dtype=np.float32)
    c2w[:3, :3] = R
    c2w[:3, 3] = rng.normal(size=3)
    return c2w


def test_scanner_camera_projects_like_a_pinhole():
    """A point at (X, Y, -Z) in the scanner camera frame (x right, y up,
    looking down -z) lands at pixel (W/2 + fx X / Z - 1/2, H/2 - fy Y / Z - 1/2)
    in the rasterizer's pixel-centre convention, at view depth Z > 0."""
    rng = np.random.default_rng(2)
    W, H = 640, 480
    for _ in range(20):
        c2w = _pose(rng)
        fx, fy = rng.uniform(300, 900), rng.uniform(300, 900)
        frame = {"w": 1280, "h": 960, "fl_x": 2 * fx, "fl_y": 2 * fy, "cx": 0.0, "cy": 0.0,
                 "transform_matrix": c2w.tolist()}
        cam = scanner.build_camera_from_scanner_json(frame, W, H)
        assert abs(cam.tan_fovx - W / (2 * fx)) < 1e-6 and abs(cam.tan_fovy - H / (2 * fy)) < 1e-6
        np.testing.assert_allclose(cam.campos, c2w[:3, 3], atol=1e-6)
        X, Y, Z = rng.uniform(-1, 1), rng.uniform(-1, 1), rng.uniform(1, 10)
        pw = c2w.astype(np.float64) @ np.array([X, Y, -Z, 1.0])
        view = cam.viewmatrix.astype(np.float64).T  # world -> view
        clip = cam.projmatrix.astype(np.float64).T @ pw
        assert abs((view @ pw)[2] - Z) < 1e-4
        ndc = clip[:3] / clip[3]
        px = ((ndc[0] + 1) * W - 1) / 2
        py = ((ndc[1] + 1) * H - 1) / 2
        assert abs(px - (W / 2 + fx * X / Z - 0.5)) < 2e-3
        assert abs(py - (H / 2 - fy * Y / Z - 0.5)) < 2e-3


def test_scanner_frame_record_and_normalisation():
    pose = np.arange(16, dtype=np.float32).reshape(4, 4)
    pose[3] = [0, 0, 0, 1]
    raw = {"intrinsics": [500, 0, 320, 0, 510, 240, 0, 0, 1],
           "cameraPoseARFrame": pose.reshape(-1).tolist()}
    rec = scanner.scanner_frame_record(raw, 640, 480, "frame_00001.jpg")
    a, a4 = scanner.make_axis_transform()
    np.testing.assert_array_equal(np.array(rec["transform_matrix"], np.float32), a4 @ pose)
    assert (rec["fl_x"], rec["fl_y"], rec["cx"], rec["cy"]) == (500, 510, 320, 240)
    # a maps (x, y, z) to (x, z, -y): a right-handed rotation
    np.testing.assert_array_equal(a @ np.float32([1, 2, 3]), [1, 3, -2])
    assert abs(np.linalg.det(a) - 1) < 1e-7
    with pytest.raises(RuntimeError):
        scanner.scanner_frame_record({"intrinsics": [1] * 8, "cameraPoseARFrame": [0] * 16}, 1, 1)
    t, s = scanner.compute_normalization([np.float32([0, 0, 0]), np.float32([2, 4, 0])])
    np.testing.assert_array_equal(t, [1, 2, 0])
    assert s == 0.5
    assert scanner.compute_normalization([np.float32([1, 1, 1])] * 2)[1] == 1.0


def test_prepare_dataset_end_to_end(tmp_path):
    from PIL import Image

    rng = np.random.default_rng(3)
    for i in range(3):
        c2w = _pose(rng)
        Image.new("RGB", (64, 48), (255, 0, 0)).save(tmp_path / f"frame_{i:05d}.jpg", quality=100)
        (tmp_path / f"frame_{i:05d}.json").write_text(json.dumps(
            {"intrinsics": [60, 0, 32, 0, 60, 24, 0, 0, 1],
             "cameraPoseARFrame": c2w.reshape(-1).tolist()}))
    (tmp_path / "frame_00009.json").write_text("{}")  # no image: ignored
    pts = rng.normal(size=(500, 3)).astype(np.float32)
    ply.write_ply(tmp_path / "points.ply",
                  {"vertex": {"x": pts[:, 0], "y": pts[:, 1], "z": pts[:, 2],
                              "red": np.full(500, 255, np.uint8),
                              "green": np.zeros(500, np.uint8), "blue": np.zeros(500, np.uint8)}})
    cams, targets, points, colors, base = scanner.prepare_dataset(
        tmp_path, 32, 24, max_points=400, seed=1, extra_points_ratio=0.5)
    assert len(cams) == 3 and base == 400 and points.shape == (600, 3)
    assert targets[0].shape == (3, 24, 32)
    np.testing.assert_allclose(targets[0][:, 12, 16], [1, 0, 0], atol=0.02)
    np.testing.assert_array_equal(colors[:400], np.tile([1.0, 0.0, 0.0], (400, 1)))
    # camera centres are normalised: max |centre - mean| = 1
    cen = np.stack([c.campos for c in cams])
    assert abs(np.abs(cen - cen.mean(axis=0)).max() - 1.0) < 1e-5


def test_init_model_and_save_as_spz(tmp_path):
    rng = np.random.default_rng(5)
    pts = rng.normal(size=(20, 3)).astype(np.float32)
    cols = rng.uniform(0, 1, (20, 3)).astype(np.float32)
    m = scanner.init_model(pts, cols, 3)
    assert m["features_rest"].shape == (20, 15, 3) and not m["features_rest"].any()
    np.testing.assert_allclose(1 / (1 + np.exp(-m["opacity_logits"])), 0.82, rtol=1e-6)
    np.testing.assert_allclose(np.exp(m["log_scales"]), 0.02, rtol=1e-6)
    np.testing.assert_allclose(m["features_dc"] * scanner.SH_C0 + 0.5, cols, atol=1e-6)
    m["rotations"] = rng.standard_normal((20, 4)).astype(np.float32)
    path = tmp_path / "m.spz"
    assert scanner.save_as_spz(path, m, 3)
    d = spz.load_spz(path)
    p = d.positions.reshape(-1, 3)
    np.testing.assert_allclose(p, np.stack([pts[:, 0], -pts[:, 2], pts[:, 1]], 1),
                               atol=0.5 / 4096 + 1e-6)
    # the rotation slots hold the (w, x, y, z) quaternion of A R A^T (A the axis change)
    a, _ = scanner.make_axis_transform()
    R = scanner.quaternions_wxyz_to_rotation_matrices(m["rotations"])
    got = d.rotations.reshape(-1, 4)  # decoded as (x, y, z, w) slots
    for i in range(20):
        want = scanner.rotation_matrices_to_quaternions_wxyz((a @ R[i] @ a.T)[None])[0]
        assert abs(float(got[i] @ want)) > 0.995, (got[i], want)  # q and -q: one rotation
        Rw = scanner.quaternions_wxyz_to_rotation_matrices(want[None])[0]
        np.testing.assert_allclose(Rw, a @ R[i] @ a.T, atol=1e-5)
