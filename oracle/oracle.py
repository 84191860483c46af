"""CPU parity oracle for the FastGS rasterizer (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or the timed CPU
baseline.  The product package ``fastgs_core_amd`` never imports it.

This is a numpy/ctypes driver around ``fgs_oracle.c`` (a C restatement of the
reference Metal kernels).  ``Oracle.render`` mirrors the stage orchestration
of ``rasterize_gaussians_forward`` (reference binding.cpp:33-282) and
``Oracle.render_backward`` chains the two vjps (fastgs_rasterize.cpp:191-206
then fastgs_preprocess.cpp:191-206).

Parity status of each C function (how it is pinned; see tests/test_oracle_*):
  orc_expf / orc_logf /    : error bounds against numpy float64 exp/log/exp2.
  orc_blend_exp2f
  splat_power              : error bound against log2(e) times the float64
                             quadratic form.
  orc_preprocess_fwd       : closed forms (identity camera cov2D = J J^T + 0.3),
                             reference KAT (preprocess_smoke: all zero), and the
                             double build's finite differences through it.
  tiles_walk (A4/A6)       : brute-force ellipse/tile-rectangle intersection in
                             float64 on random small ellipses; invariants.
  orc_duplicate_with_keys  : reference KAT (binning_smoke: all zero) + emitted
                             tiles equal the brute-force tile set.
  orc_sort_pairs_u64       : numpy stable argsort.
  orc_tile_ranges          : reference KAT (tile_prep_smoke, hand-derived).
  orc_rasterize_fwd        : closed form single splat (rasterize_smoke), brute
                             force per-pixel compositing on tiny scenes, and a
                             float64 array formulation (cumulative products
                             over list positions) of n_contrib as a position,
                             max_contrib, metric_count, final_T, the sampled
                             state (including the slots left zero after a
                             break) on multi-bucket ragged tiles
                             (test_oracle_raster_state).  ref_order=True: the
                             reference's operation order, used to measure how
                             often the mirrored order decides differently.
  orc_rasterize_bwd        : central finite differences of the double build.
  orc_rasterize_bwd_mag    : equal to the per-pixel sums of |gradient| of the
  orc_preprocess_bwd_mag     FD-pinned backward, bound the gradients, bound the
                             f32 vs f64 differences of ill-conditioned rows
                             (test_oracle_mag).
  orc_preprocess_bwd       : central finite differences of the double build and
                             the preprocess_backward_validation KAT (0.01).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int32, c_int64, c_uint32, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
TILE = 16


class OrcParams(ctypes.Structure):
    _fields_ = [
        ("P", c_int32),
        ("degree", c_int32),
        ("max_sh_coeffs", c_int32),
        ("image_width", c_int32),
        ("image_height", c_int32),
        ("grid_x", c_int32),
        ("grid_y", c_int32),
        ("use_cov3d_precomp", c_int32),
        ("use_colors_precomp", c_int32),
        ("scale_modifier", c_float),
        ("mult", c_float),
        ("tan_fovx", c_float),
        ("tan_fovy", c_float),
    ]


class OrcRParams(ctypes.Structure):
    _fields_ = [
        ("image_width", c_int32),
        ("image_height", c_int32),
        ("num_channels", c_int32),
        ("num_tiles", c_int32),
        ("bucket_sum", c_int64),
        ("get_flag", c_int32),
        ("write_sampled", c_int32),
        ("ref_order", c_int32),
    ]


def build_oracle() -> None:
    """Compile the oracle libraries with oracle/Makefile."""
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_void_p)


class Oracle:
    """ctypes wrapper; ``double=True`` loads the float64 build."""

    def __init__(self, double: bool = False):
        name = "liborc_f64.so" if double else "liborc_f32.so"
        path = os.path.join(_HERE, "lib", name)
        if not os.path.exists(path):
            build_oracle()
        self.lib = ctypes.CDLL(path)
        self.double = double
        self.dt = np.float64 if double else np.float32
        L = self.lib
        L.orc_expf.restype = c_float
        L.orc_expf.argtypes = [c_float]
        L.orc_blend_exp2f.restype = c_float
        L.orc_blend_exp2f.argtypes = [c_float]
        L.orc_splat_power.restype = c_double
        L.orc_splat_power.argtypes = [c_double] * 5
        L.orc_logf.restype = c_float
        L.orc_logf.argtypes = [c_float]
        L.orc_sizeof_real.restype = c_int32
        assert L.orc_sizeof_real() == (8 if double else 4)

    # -- helpers --------------------------------------------------------
    def _f(self, a, shape=None):
        if a is None:
            return None
        a = np.ascontiguousarray(np.asarray(a, dtype=self.dt))
        if shape is not None:
            a = a.reshape(shape)
        return a

    def expf(self, x: float) -> float:
        return self.lib.orc_expf(float(x))

    def blend_exp2f(self, t: float) -> float:
        return self.lib.orc_blend_exp2f(float(t))

    def splat_power(self, a, b, c, dx, dy) -> float:
        return self.lib.orc_splat_power(float(a), float(b), float(c), float(dx), float(dy))

    def logf(self, x: float) -> float:
        return self.lib.orc_logf(float(x))

    def tiles_touched_one(self, px, py, conic_opacity, gx, gy, mult=1.0) -> int:
        fn = self.lib.orc_tiles_touched_one
        fn.restype = c_uint32
        rt = ctypes.c_double if self.double else c_float
        fn.argtypes = [rt, rt, c_void_p, c_int32, c_int32, rt]
        co = self._f(conic_opacity, (4,))
        return int(fn(px, py, _ptr(co), gx, gy, mult))

    def color_from_sh(self, degree, mean, campos, dc, sh):
        """orc_color_from_sh for one Gaussian: returns (rgb, clamped)."""
        fn = self.lib.orc_color_from_sh
        fn.restype = None
        fn.argtypes = [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
        col = np.zeros(3, self.dt)
        cl = np.zeros(3, np.uint8)
        shv = self._f(sh, (-1,)) if sh is not None and np.asarray(sh).size else np.zeros(45, self.dt)
        fn(degree, _ptr(self._f(mean, (3,))), _ptr(self._f(campos, (3,))), _ptr(self._f(dc, (3,))),
           _ptr(shv), _ptr(col), _ptr(cl))
        return col, cl.astype(bool)

    # -- stages ----------------------------------------------------------
    def preprocess_fwd(self, means3d, opacities, viewmatrix, projmatrix, campos, vsp_in,
                       image_width, image_height, tan_fovx=1.0, tan_fovy=1.0, degree=0,
                       scale_modifier=1.0, mult=1.0, dc=None, sh=None, colors_precomp=None,
                       scales=None, rotations=None, cov3d_precomp=None):
        means3d = self._f(means3d)
        P = means3d.shape[0]
        use_cov = cov3d_precomp is not None
        use_col = colors_precomp is not None
        sh_arr = self._f(sh) if sh is not None else np.zeros((P, 0, 3), self.dt)
        max_sh = sh_arr.shape[1] if sh_arr.ndim >= 2 else 0
        prm = OrcParams(P, degree, max_sh, image_width, image_height,
                        (image_width + TILE - 1) // TILE, (image_height + TILE - 1) // TILE,
                        int(use_cov), int(use_col), scale_modifier, mult, tan_fovx, tan_fovy)
        dt = self.dt
        out = {
            "radii": np.zeros(P, np.int32),
            "xys": np.zeros((P, 2), dt),
            "depths": np.zeros(P, dt),
            "cov3d": np.zeros((P, 6), dt),
            "rgb": np.zeros((P, 3), dt),
            "conic_opacity": np.zeros((P, 4), dt),
            "tiles_touched": np.zeros(P, np.uint32),
            "clamped": np.zeros((P, 3), np.uint8),
            "viewspace_points": np.zeros((P, 4), dt),
        }
        args = [
            ctypes.byref(prm), _ptr(means3d),
            _ptr(self._f(dc, (P, 3)) if dc is not None else None),
            _ptr(sh_arr if not use_col else None),
            _ptr(self._f(colors_precomp, (P, 3)) if use_col else None),
            _ptr(self._f(opacities, (P,))),
            _ptr(self._f(scales, (P, 3)) if not use_cov else None),
            _ptr(self._f(rotations, (P, 4)) if not use_cov else None),
            _ptr(self._f(cov3d_precomp, (P, 6)) if use_cov else None),
            _ptr(self._f(viewmatrix, (16,))), _ptr(self._f(projmatrix, (16,))),
            _ptr(self._f(campos, (3,))), _ptr(self._f(vsp_in, (P, 4))),
        ] + [_ptr(out[k]) for k in ("radii", "xys", "depths", "cov3d", "rgb", "conic_opacity",
                                     "tiles_touched", "clamped", "viewspace_points")]
        self.lib.orc_preprocess_fwd(*args)
        out["clamped"] = out["clamped"].astype(bool)
        out["max_sh_coeffs"] = max_sh
        return out

    def inclusive_scan(self, x):
        x = np.ascontiguousarray(x, dtype=np.uint32)
        out = np.zeros_like(x)
        self.lib.orc_inclusive_scan_u32(c_int64(x.size), _ptr(x), _ptr(out))
        return out

    def duplicate_with_keys(self, xys, depths, point_offsets, conic_opacity, tiles_touched,
                            mult, gx, gy, num_rendered):
        xys = self._f(xys)
        P = xys.shape[0]
        keys = np.zeros(num_rendered, np.uint64)
        vals = np.zeros(num_rendered, np.uint32)
        self.lib.orc_duplicate_with_keys(
            c_int32(P), _ptr(xys), _ptr(self._f(depths, (P,))),
            _ptr(np.ascontiguousarray(point_offsets, np.uint32)),
            _ptr(self._f(conic_opacity, (P, 4))),
            _ptr(np.ascontiguousarray(tiles_touched, np.uint32)), c_float(mult), c_int32(gx),
            c_int32(gy), c_int64(num_rendered), _ptr(keys), _ptr(vals))
        return keys, vals

    def sort_pairs(self, keys, vals):
        k = np.array(keys, dtype=np.uint64, copy=True)
        v = np.array(vals, dtype=np.uint32, copy=True)
        self.lib.orc_sort_pairs_u64(c_int64(k.size), _ptr(k), _ptr(v))
        return k, v

    def tile_ranges(self, keys, num_tiles):
        keys = np.ascontiguousarray(keys, np.uint64)
        ranges = np.zeros((num_tiles, 2), np.uint32)
        bc = np.zeros(num_tiles, np.uint32)
        self.lib.orc_tile_ranges(c_int64(keys.size), _ptr(keys), c_int32(num_tiles), _ptr(ranges),
                                 _ptr(bc))
        return ranges, bc

    def rasterize_fwd(self, ranges, point_list, bucket_offsets, means2d, colors, conic_opacity,
                      background, metric_map, image_width, image_height, num_channels=3,
                      num_tiles=None, bucket_sum=None, get_flag=False, write_sampled=False,
                      num_points=None, ref_order=False):
        """orc_rasterize_fwd.  ``ref_order``: evaluate the blend in the
        reference's operation order (libm expf of the natural-base power,
        T (1 - alpha) with two roundings) in place of the HIP kernels' order."""
        gx = (image_width + TILE - 1) // TILE
        gy = (image_height + TILE - 1) // TILE
        if num_tiles is None:
            num_tiles = gx * gy
        bucket_offsets = np.ascontiguousarray(bucket_offsets, np.uint32)
        if bucket_sum is None:
            bucket_sum = int(bucket_offsets[-1]) if bucket_offsets.size else 0
        means2d = self._f(means2d)
        P = means2d.shape[0] if num_points is None else num_points
        HW = image_width * image_height
        dt = self.dt
        ss = bucket_sum * 256 if write_sampled else 0
        out = {
            "bucket_to_tile": np.zeros(bucket_sum, np.uint32),
            "sampled_t": np.zeros(ss, dt),
            "sampled_ar": np.zeros(num_channels * ss, dt),
            "final_t": np.zeros(HW, dt),
            "n_contrib": np.zeros(HW, np.uint32),
            "max_contrib": np.zeros(num_tiles, np.uint32),
            "pixel_colors": np.zeros((num_channels, HW), dt),
            "out_color": np.zeros((num_channels, HW), dt),
            "metric_count": np.zeros(P if get_flag else 0, np.int32),
        }
        rp = OrcRParams(image_width, image_height, num_channels, num_tiles, bucket_sum,
                        int(get_flag), int(write_sampled), int(ref_order))
        mm = np.ascontiguousarray(metric_map, np.int32) if metric_map is not None else \
            np.zeros(HW, np.int32)
        self.lib.orc_rasterize_fwd(
            ctypes.byref(rp), _ptr(np.ascontiguousarray(ranges, np.uint32)),
            _ptr(np.ascontiguousarray(point_list, np.uint32)), _ptr(bucket_offsets),
            _ptr(means2d), _ptr(self._f(colors)), _ptr(self._f(conic_opacity)),
            _ptr(self._f(background, (-1,))), _ptr(mm),
            *[_ptr(out[k]) for k in ("bucket_to_tile", "sampled_t", "sampled_ar", "final_t",
                                     "n_contrib", "max_contrib", "pixel_colors", "out_color",
                                     "metric_count")])
        out["sampled_ar"] = out["sampled_ar"].reshape(num_channels, ss) if ss else \
            out["sampled_ar"].reshape(num_channels, 0)
        return out

    def rasterize_bwd(self, ranges, point_list, means2d, colors, conic_opacity, background,
                      final_t, n_contrib, dL_dout, image_width, image_height, num_channels=3,
                      num_tiles=None, magnitude=False):
        """Gradients of the blend.  With ``magnitude`` also, for every gradient
        entry, float64 arrays of the gradients' keys and shapes
        (orc_rasterize_bwd_mag): ``g["mag_terms"]`` = sum over its (pixel,
        splat) terms of |term|, the scale of the gradient gate; ``g["mag"]`` =
        the same sum with every sum inside a term also taken over magnitudes."""
        gx = (image_width + TILE - 1) // TILE
        gy = (image_height + TILE - 1) // TILE
        if num_tiles is None:
            num_tiles = gx * gy
        means2d = self._f(means2d)
        P = means2d.shape[0]
        dt = self.dt
        g = {
            "means2d": np.zeros((P, 2), dt),
            "colors": np.zeros((P, num_channels), dt),
            "conic_opacity": np.zeros((P, 4), dt),
            "viewspace_points": np.zeros((P, 4), dt),
        }
        rp = OrcRParams(image_width, image_height, num_channels, num_tiles, 0, 0, 0, 0)
        aw = 10 + num_channels
        mag = np.zeros((P, 2, aw), np.float64) if magnitude else None
        fn = self.lib.orc_rasterize_bwd_mag
        fn.restype = None
        fn.argtypes = [c_void_p] * 15 + [c_int64]
        fn(ctypes.byref(rp), _ptr(np.ascontiguousarray(ranges, np.uint32)),
           _ptr(np.ascontiguousarray(point_list, np.uint32)), _ptr(means2d),
           _ptr(self._f(colors)), _ptr(self._f(conic_opacity)), _ptr(self._f(background, (-1,))),
           _ptr(self._f(final_t, (-1,))), _ptr(np.ascontiguousarray(n_contrib, np.uint32)),
           _ptr(self._f(dL_dout)), _ptr(g["means2d"]), _ptr(g["colors"]),
           _ptr(g["conic_opacity"]), _ptr(g["viewspace_points"]), _ptr(mag), P)
        if magnitude:
            for key, j in (("mag", 0), ("mag_terms", 1)):
                m = mag[:, j]
                g[key] = {"means2d": m[:, 0:2], "viewspace_points": m[:, 2:6],
                          "conic_opacity": m[:, 6:10], "colors": m[:, 10:10 + num_channels]}
        return g

    def preprocess_bwd(self, means3d, viewmatrix, projmatrix, campos, radii, cov3d_fwd, clamped,
                       dL_dxys, dL_drgb, dL_dconic_opacity, dL_dvsp, image_width, image_height,
                       tan_fovx=1.0, tan_fovy=1.0, degree=0, scale_modifier=1.0, dL_dcov3d=None,
                       sh=None, scales=None, rotations=None, cov3d_precomp=None,
                       use_colors_precomp=False):
        means3d = self._f(means3d)
        P = means3d.shape[0]
        dt = self.dt
        use_cov = cov3d_precomp is not None
        sh_arr = self._f(sh) if sh is not None else np.zeros((P, 0, 3), dt)
        max_sh = sh_arr.shape[1] if sh_arr.ndim >= 2 else 0
        prm = OrcParams(P, degree, max_sh, image_width, image_height, 0, 0, int(use_cov),
                        int(use_colors_precomp), scale_modifier, 1.0, tan_fovx, tan_fovy)
        g = {
            "means3d": np.zeros((P, 3), dt),
            "dc": np.zeros((P, 3), dt),
            "sh": np.zeros(sh_arr.shape, dt),
            "colors_precomp": np.zeros((P, 3), dt),
            "opacities": np.zeros(P, dt),
            "scales": np.zeros((P, 3), dt),
            "rotations": np.zeros((P, 4), dt),
            "viewspace_points": np.zeros((P, 4), dt),
        }
        if dL_dcov3d is None:
            dL_dcov3d = np.zeros((P, 6), dt)
        self.lib.orc_preprocess_bwd(
            ctypes.byref(prm), _ptr(means3d),
            _ptr(self._f(scales, (P, 3)) if not use_cov else None),
            _ptr(self._f(rotations, (P, 4)) if not use_cov else None),
            _ptr(self._f(viewmatrix, (16,))), _ptr(self._f(projmatrix, (16,))),
            _ptr(self._f(campos, (3,))), _ptr(sh_arr),
            _ptr(self._f(cov3d_precomp, (P, 6)) if use_cov else None), _ptr(self._f(cov3d_fwd)),
            _ptr(self._f(dL_dcov3d, (P, 6))), _ptr(self._f(dL_drgb, (P, 3))),
            _ptr(self._f(dL_dxys, (P, 2))), _ptr(self._f(dL_dconic_opacity, (P, 4))),
            _ptr(self._f(dL_dvsp, (P, 4))), _ptr(np.ascontiguousarray(radii, np.int32)),
            _ptr(np.ascontiguousarray(clamped, np.uint8)),
            *[_ptr(g[k]) for k in ("means3d", "dc", "sh", "colors_precomp", "opacities", "scales",
                                   "rotations", "viewspace_points")])
        return g

    def preprocess_bwd_mag(self, means3d, viewmatrix, projmatrix, campos, radii, cov3d_fwd,
                           clamped, m_xys, m_rgb, m_conic_opacity, m_vsp, image_width,
                           image_height, tan_fovx=1.0, tan_fovy=1.0, degree=0,
                           scale_modifier=1.0, m_cov3d=None, sh=None, scales=None,
                           rotations=None, cov3d_precomp=None, use_colors_precomp=False):
        """orc_preprocess_bwd_mag: the sums of term magnitudes of every output of
        preprocess_bwd, given the magnitudes (float64) of its cotangents."""
        means3d = self._f(means3d)
        P = means3d.shape[0]
        use_cov = cov3d_precomp is not None
        sh_arr = self._f(sh) if sh is not None else np.zeros((P, 0, 3), self.dt)
        max_sh = sh_arr.shape[1] if sh_arr.ndim >= 2 else 0
        prm = OrcParams(P, degree, max_sh, image_width, image_height, 0, 0, int(use_cov),
                        int(use_colors_precomp), scale_modifier, 1.0, tan_fovx, tan_fovy)
        d = lambda a, shape: np.ascontiguousarray(np.asarray(a, np.float64).reshape(shape))  # noqa
        out = {
            "means3d": np.zeros((P, 3)), "dc": np.zeros((P, 3)), "sh": np.zeros(sh_arr.shape),
            "colors_precomp": np.zeros((P, 3)), "opacities": np.zeros(P),
            "scales": np.zeros((P, 3)), "rotations": np.zeros((P, 4)),
            "viewspace_points": np.zeros((P, 4)),
        }
        fn = self.lib.orc_preprocess_bwd_mag
        fn.restype = None
        fn.argtypes = [c_void_p] * 25
        fn(ctypes.byref(prm), _ptr(means3d),
           _ptr(self._f(scales, (P, 3)) if not use_cov else None),
           _ptr(self._f(rotations, (P, 4)) if not use_cov else None),
           _ptr(self._f(viewmatrix, (16,))), _ptr(self._f(projmatrix, (16,))),
           _ptr(self._f(campos, (3,))), _ptr(sh_arr),
           _ptr(self._f(cov3d_precomp, (P, 6)) if use_cov else None), _ptr(self._f(cov3d_fwd)),
           _ptr(d(m_cov3d, (P, 6)) if m_cov3d is not None else None), _ptr(d(m_rgb, (P, 3))),
           _ptr(d(m_xys, (P, 2))), _ptr(d(m_conic_opacity, (P, 4))), _ptr(d(m_vsp, (P, 4))),
           _ptr(np.ascontiguousarray(radii, np.int32)),
           _ptr(np.ascontiguousarray(clamped, np.uint8)),
           *[_ptr(out[k]) for k in ("means3d", "dc", "sh", "colors_precomp", "opacities",
                                    "scales", "rotations", "viewspace_points")])
        return out

    # -- full pipeline (binding.cpp:33-282) ------------------------------
    def render(self, inputs: dict, image_width: int, image_height: int, tan_fovx=1.0,
               tan_fovy=1.0, degree=0, scale_modifier=1.0, mult=1.0, get_flag=False,
               write_sampled=False, timings: dict | None = None):
        """Forward of ``rasterize_gaussians`` on numpy inputs (reference key names).
        ``timings``: a dict that receives the wall seconds of each stage
        (preprocess_fwd, scan, duplicate, sort, ranges, rasterize_fwd)."""
        import time

        clock = [time.perf_counter()]

        def lap(name):
            if timings is not None:
                t = time.perf_counter()
                timings[name] = timings.get(name, 0.0) + t - clock[0]
                clock[0] = t
        col = inputs.get("colors_precomp", inputs.get("colors"))
        has_col = col is not None and np.asarray(col).size != 0
        has_sh = "dc" in inputs and "sh" in inputs
        if has_col == has_sh:
            raise RuntimeError("rasterize_gaussians_forward expects exactly one color path: "
                               "either colors_precomp (or colors) OR dc+sh")
        cov = inputs.get("cov3d_precomp")
        has_cov = cov is not None and np.asarray(cov).size != 0
        sc, rot = inputs.get("scales"), inputs.get("rotations")
        has_sr = sc is not None and rot is not None and np.asarray(sc).size and np.asarray(rot).size
        if has_cov == bool(has_sr):
            raise RuntimeError("rasterize_gaussians_forward expects exactly one geometry path: "
                               "either cov3d_precomp OR scales+rotations")
        means3d = np.asarray(inputs["means3d"])
        P = means3d.shape[0]
        vsp = inputs.get("viewspace_points")
        if vsp is None or np.asarray(vsp).size == 0:
            vsp = np.zeros((P, 4), self.dt)
        gx = (image_width + TILE - 1) // TILE
        gy = (image_height + TILE - 1) // TILE
        T = gx * gy
        pre = self.preprocess_fwd(
            means3d, inputs["opacities"], inputs["viewmatrix"], inputs["projmatrix"],
            inputs["campos"], vsp, image_width, image_height, tan_fovx, tan_fovy, degree,
            scale_modifier, mult, dc=inputs.get("dc") if not has_col else None,
            sh=inputs.get("sh") if not has_col else None, colors_precomp=col if has_col else None,
            scales=sc if not has_cov else None, rotations=rot if not has_cov else None,
            cov3d_precomp=cov if has_cov else None)
        lap("preprocess_fwd")
        point_offsets = self.inclusive_scan(pre["tiles_touched"])
        K = int(point_offsets[-1]) if P else 0
        lap("scan")
        out = {"rendered": K, "num_buckets": 0, "radii": pre["radii"],
               "point_offsets": point_offsets, "pre": pre, "num_tiles": T,
               "viewspace_points": pre["viewspace_points"], "geom_means2d": pre["xys"],
               "geom_depths": pre["depths"], "geom_cov3d": pre["cov3d"], "geom_rgb": pre["rgb"],
               "geom_conic_opacity": pre["conic_opacity"],
               "geom_tiles_touched": pre["tiles_touched"], "geom_clamped": pre["clamped"]}
        if K == 0:
            return out
        keys_u, vals_u = self.duplicate_with_keys(pre["xys"], pre["depths"], point_offsets,
                                                  pre["conic_opacity"], pre["tiles_touched"],
                                                  mult, gx, gy, K)
        lap("duplicate")
        keys, vals = self.sort_pairs(keys_u, vals_u)
        lap("sort")
        ranges, bucket_count = self.tile_ranges(keys, T)
        bucket_offsets = self.inclusive_scan(bucket_count)
        B = int(bucket_offsets[-1])
        lap("ranges")
        out.update({"point_list_keys_unsorted": keys_u, "point_list_unsorted": vals_u,
                    "point_list_keys": keys, "point_list": vals, "ranges": ranges,
                    "bucket_count": bucket_count, "bucket_offsets": bucket_offsets,
                    "num_buckets": B})
        if B == 0:
            return out
        metric_map = inputs.get("metric_map")
        r = self.rasterize_fwd(ranges, vals, bucket_offsets, pre["xys"], pre["rgb"],
                               pre["conic_opacity"], inputs["background"], metric_map,
                               image_width, image_height, 3, T, B, get_flag, write_sampled, P)
        lap("rasterize_fwd")
        out["raster"] = r
        out.update({"out_color": r["out_color"], "metric_count": r["metric_count"],
                    "sample_bucket_to_tile": r["bucket_to_tile"], "sample_t": r["sampled_t"],
                    "sample_ar": r["sampled_ar"], "img_final_t": r["final_t"],
                    "img_n_contrib": r["n_contrib"], "img_max_contrib": r["max_contrib"],
                    "img_pixel_colors": r["pixel_colors"]})
        return out

    def render_backward(self, inputs: dict, fwd: dict, dL_dout_color, image_width, image_height,
                        tan_fovx=1.0, tan_fovy=1.0, degree=0, scale_modifier=1.0,
                        dL_dvsp_out=None, dL_dxys_extra=None, magnitude=False,
                        timings: dict | None = None):
        """Gradients of sum(dL_dout_color * out_color) (+ optional direct cotangents of the
        preprocess outputs) w.r.t. the differentiable inputs, chained exactly as
        FastGSRasterize::vjp -> FastGSPreprocess::vjp.

        ``magnitude``: also ``g["mag_terms"]`` and ``g["mag"]`` (float64, the
        gradients' keys and shapes): for every gradient entry the sum of the
        magnitudes of the terms it is made of.  The blend's per-(pixel, splat)
        terms come from rasterize_bwd; orc_preprocess_bwd_mag carries them
        through the preprocess backward's own sums and products (each sum
        taken over magnitudes), so an entry's value is the sum of |term| over
        the fully expanded chain rule.  ``timings``: receives the wall seconds of
        rasterize_bwd and preprocess_bwd."""
        import time

        t0 = time.perf_counter()
        pre = fwd["pre"]
        P = pre["xys"].shape[0]
        dt = self.dt
        if "raster" in fwd:
            r = fwd["raster"]
            g2 = self.rasterize_bwd(fwd["ranges"], fwd["point_list"], pre["xys"], pre["rgb"],
                                    pre["conic_opacity"], inputs["background"], r["final_t"],
                                    r["n_contrib"], np.asarray(dL_dout_color, dt).reshape(3, -1),
                                    image_width, image_height, 3, fwd["num_tiles"],
                                    magnitude=magnitude)
        else:
            g2 = {"means2d": np.zeros((P, 2), dt), "colors": np.zeros((P, 3), dt),
                  "conic_opacity": np.zeros((P, 4), dt), "viewspace_points": np.zeros((P, 4), dt)}
            if magnitude:
                g2["mag"] = {k: np.zeros(v.shape, np.float64) for k, v in g2.items()}
        t1 = time.perf_counter()
        dvsp = g2["viewspace_points"].copy()
        if dL_dvsp_out is not None:
            dvsp += np.asarray(dL_dvsp_out, dt)
        dxys = g2["means2d"].copy()
        if dL_dxys_extra is not None:
            dxys += np.asarray(dL_dxys_extra, dt)
        col = inputs.get("colors_precomp", inputs.get("colors"))
        has_col = col is not None and np.asarray(col).size != 0
        cov = inputs.get("cov3d_precomp")
        has_cov = cov is not None and np.asarray(cov).size != 0
        g = self.preprocess_bwd(
            inputs["means3d"], inputs["viewmatrix"], inputs["projmatrix"], inputs["campos"],
            pre["radii"], pre["cov3d"], pre["clamped"], dxys, g2["colors"], g2["conic_opacity"],
            dvsp, image_width, image_height, tan_fovx, tan_fovy, degree, scale_modifier,
            sh=inputs.get("sh") if not has_col else None,
            scales=inputs.get("scales") if not has_cov else None,
            rotations=inputs.get("rotations") if not has_cov else None,
            cov3d_precomp=cov if has_cov else None, use_colors_precomp=has_col)
        if timings is not None:
            t2 = time.perf_counter()
            timings["rasterize_bwd"] = timings.get("rasterize_bwd", 0.0) + t1 - t0
            timings["preprocess_bwd"] = timings.get("preprocess_bwd", 0.0) + t2 - t1
        g["raster"] = g2
        if magnitude:
            if "mag_terms" not in g2:
                g2["mag_terms"] = g2["mag"]
            for key in ("mag", "mag_terms"):
                m2 = g2[key]
                m_xys = m2["means2d"].copy()
                if dL_dxys_extra is not None:
                    m_xys += np.abs(np.asarray(dL_dxys_extra, np.float64))
                m_vsp = m2["viewspace_points"].copy()
                if dL_dvsp_out is not None:
                    m_vsp += np.abs(np.asarray(dL_dvsp_out, np.float64))
                g[key] = self.preprocess_bwd_mag(
                    inputs["means3d"], inputs["viewmatrix"], inputs["projmatrix"],
                    inputs["campos"], pre["radii"], pre["cov3d"], pre["clamped"], m_xys,
                    m2["colors"], m2["conic_opacity"], m_vsp, image_width, image_height,
                    tan_fovx, tan_fovy, degree, scale_modifier,
                    sh=inputs.get("sh") if not has_col else None,
                    scales=inputs.get("scales") if not has_cov else None,
                    rotations=inputs.get("rotations") if not has_cov else None,
                    cov3d_precomp=cov if has_cov else None, use_colors_precomp=has_col)
        return g
