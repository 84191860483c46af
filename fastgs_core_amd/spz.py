"""The .spz Gaussian-splat container, with the API of the ``spz`` Python
binding the reference exports through (scripts/train_scanner_fixed.py:630-681,
scripts/test_spz_export.py): ``GaussianCloud``, ``PackOptions`` /
``UnpackOptions``, ``CoordinateSystem``, ``save_spz``, ``load_spz``.

The binding is nianticlabs/spz pinned at ef094fd (an un-vendored submodule,
.gitmodules:1-3, Readme.md:45-51); it is absent here, so the format is
restated from spz's published encoder and decoder:

* a 16-byte little-endian header -- magic 0x5053474E ("NGSP"), version,
  point count, SH degree, fractional bits (12), flags (bit 0: antialiased),
  a reserved byte -- then the arrays in the order positions, alphas, colours,
  scales, rotations, SH, the whole stream gzip-compressed;
* positions: 24-bit two's-complement fixed point, round(x * 2^12);
* alphas: round(sigmoid(logit) * 255); colours (SH DC): round(c * 0.15 * 255
  + 127.5); scales (log): round((s + 10) * 16); every byte clamped to
  [0, 255], rounding half away from zero (C's ``round``);
* rotations, version 2: the normalised (x, y, z, w) quaternion negated if
  w < 0, then round(x * 127.5 + 127.5) for x, y, z; version 3: "smallest
  three" -- 2 bits for the index of the largest |component| (made positive),
  then for each other component a sign bit and a 9-bit magnitude
  round(511 * |c| / sqrt(1/2)), first component in the highest bits;
* SH: [point][coefficient][channel], q = round(x * 128) + 128 rounded to
  the centre of a bucket of 8 (the 9 degree-1 values) or 16 (the rest);
* ``PackOptions.from_coord`` converts from the named axis convention to
  spz's RUB (right, up, back): axis flips of the positions, the matching
  sign flips of the quaternion's vector part and of each SH coefficient by
  the parity of its basis function; UNSPECIFIED converts nothing.

Byte-for-byte agreement with the pinned binary is unverifiable here (no
spz build, no .spz fixture in the reference); the encoding is pinned by
its closed forms, round trips and the invariances of the coordinate
conversion (tests/test_formats.py).  Version 2 is written by default:
every spz reader accepts it.
"""
from __future__ import annotations

import enum
import gzip
import math
import os
import struct
import zlib
from dataclasses import dataclass, field
from typing import Optional, Tuple, Union

import numpy as np

__all__ = ["CoordinateSystem", "GaussianCloud", "PackOptions", "UnpackOptions", "pack_gaussians",
           "unpack_gaussians", "save_spz", "load_spz", "SpzError"]

MAGIC = 0x5053474E
HEADER = struct.Struct("<IIIBBBB")
FLAG_ANTIALIASED = 0x1
COLOR_SCALE = 0.15
FRACTIONAL_BITS = 12
SH_DIM = {0: 0, 1: 3, 2: 8, 3: 15}


class SpzError(ValueError):
    """Malformed .spz data or an inconsistent GaussianCloud."""


class CoordinateSystem(enum.IntEnum):
    """Axis conventions: [L|R] x, [D|U] y, [B|F] z."""
    UNSPECIFIED = 0
    LDB = 1
    RDB = 2
    LUB = 3
    RUB = 4
    LDF = 5
    RDF = 6
    LUF = 7
    RUF = 8


@dataclass
class PackOptions:
    from_coord: CoordinateSystem = CoordinateSystem.UNSPECIFIED
    version: int = 2


@dataclass
class UnpackOptions:
    to_coord: CoordinateSystem = CoordinateSystem.UNSPECIFIED


@dataclass
class GaussianCloud:
    """Flat float32 arrays as the binding takes them: ``positions`` [3N],
    ``scales`` [3N] (log), ``rotations`` [4N] (x, y, z, w), ``alphas`` [N]
    (logits), ``colors`` [3N] (SH DC), ``sh`` [N * dim(sh_degree) * 3]
    ([point][coefficient][channel])."""
    positions: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    scales: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    rotations: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    alphas: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    colors: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    sh: np.ndarray = field(default_factory=lambda: np.zeros(0, np.float32))
    sh_degree: int = 0
    antialiased: bool = False

    @property
    def num_points(self) -> int:
        return int(np.asarray(self.positions).size // 3)

    def check(self) -> int:
        n = self.num_points
        if self.sh_degree not in SH_DIM:
            raise SpzError(f"sh_degree must be 0..3, got {self.sh_degree}")
        want = {"positions": 3 * n, "scales": 3 * n, "rotations": 4 * n, "alphas": n,
                "colors": 3 * n, "sh": n * SH_DIM[self.sh_degree] * 3}
        for k, v in want.items():
            if np.asarray(getattr(self, k)).size != v:
                raise SpzError(f"GaussianCloud.{k} has {np.asarray(getattr(self, k)).size} "
                               f"values, {v} expected for {n} points at SH degree "
                               f"{self.sh_degree}")
        return n


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))


def _round_away(x: np.ndarray) -> np.ndarray:
    """C's round(): halves away from zero, exact in float32."""
    t = np.trunc(x)
    return t + np.where(np.abs(x - t) >= np.float32(0.5), np.sign(x), np.float32(0.0))


def _to_u8(x: np.ndarray) -> np.ndarray:
    return np.clip(_round_away(x.astype(np.float32)), 0, 255).astype(np.uint8)


_AXES = {c: (s[0], s[1], s[2]) for c, s in
         ((CoordinateSystem.LDB, "LDB"), (CoordinateSystem.RDB, "RDB"),
          (CoordinateSystem.LUB, "LUB"), (CoordinateSystem.RUB, "RUB"),
          (CoordinateSystem.LDF, "LDF"), (CoordinateSystem.RDF, "RDF"),
          (CoordinateSystem.LUF, "LUF"), (CoordinateSystem.RUF, "RUF"))}


def _flips(a: CoordinateSystem, b: CoordinateSystem) -> Tuple[float, float, float]:
    if a == CoordinateSystem.UNSPECIFIED or b == CoordinateSystem.UNSPECIFIED:
        return 1.0, 1.0, 1.0
    return tuple(1.0 if x == y else -1.0 for x, y in zip(_AXES[a], _AXES[b]))


def _sh_signs(f: Tuple[float, float, float]) -> np.ndarray:
    """Sign of each real SH basis function (degree 1..3, the rasterizer's
    order) under the axis flips f: the product of the flips of the
    coordinates it is odd in."""
    x, y, z = f
    return np.array([y, z, x,                                   # y, z, x
                     x * y, y * z, 1.0, x * z, 1.0,             # xy, yz, 3z^2-1, xz, x^2-y^2
                     y, x * y * z, y, z, x, z, x], np.float32)  # degree 3


def _convert(pos, rot, sh, dim, f):
    if f == (1.0, 1.0, 1.0):
        return pos, rot, sh
    fx, fy, fz = f
    pos = (pos.reshape(-1, 3) * np.float32([fx, fy, fz])).reshape(-1)
    rot = (rot.reshape(-1, 4) * np.float32([fy * fz, fx * fz, fx * fy, 1.0])).reshape(-1)
    if dim:
        sh = (sh.reshape(-1, dim, 3) * _sh_signs(f)[:dim, None]).reshape(-1)
    return pos, rot, sh


def _quantize_sh(x: np.ndarray, bucket: int) -> np.ndarray:
    q = (_round_away(x * np.float32(128.0)) + np.float32(128.0)).astype(np.int64)
    q = ((q + bucket // 2) // bucket) * bucket  # q < 0 clamps to 0 either way
    return np.clip(q, 0, 255).astype(np.uint8)


def pack_gaussians(cloud: GaussianCloud, opts: Optional[PackOptions] = None) -> bytes:
    """The uncompressed .spz stream (header + arrays) of ``cloud``."""
    opts = opts or PackOptions()
    n = cloud.check()
    if opts.version not in (2, 3):
        raise SpzError("spz versions 2 and 3 can be written")
    deg = int(cloud.sh_degree)
    dim = SH_DIM[deg]
    pos, rot, sh = _convert(_f32(cloud.positions), _f32(cloud.rotations), _f32(cloud.sh), dim,
                            _flips(opts.from_coord, CoordinateSystem.RUB))
    fixed = _round_away(pos * np.float32(1 << FRACTIONAL_BITS)).astype(np.int64)
    pos_b = np.stack([fixed & 0xFF, (fixed >> 8) & 0xFF, (fixed >> 16) & 0xFF], axis=1)
    alpha = _f32(cloud.alphas)
    sig = np.float32(1.0) / (np.float32(1.0) + np.exp(-alpha))
    alpha_b = _to_u8(sig * np.float32(255.0))
    color_b = _to_u8(_f32(cloud.colors) * np.float32(COLOR_SCALE * 255.0) + np.float32(127.5))
    scale_b = _to_u8((_f32(cloud.scales) + np.float32(10.0)) * np.float32(16.0))
    q = rot.reshape(n, 4)
    q = q * (np.float32(1.0) / np.sqrt((q * q).sum(axis=1, dtype=np.float32)))[:, None]
    if opts.version == 2:
        q = q * np.where(q[:, 3:4] < 0, np.float32(-127.5), np.float32(127.5))
        rot_b = _to_u8(q[:, :3] + np.float32(127.5))
    else:
        rot_b = _smallest_three(q)
    sh_b = np.zeros(0, np.uint8)
    if dim:
        v = sh.reshape(n, dim * 3)
        sh_b = np.concatenate([_quantize_sh(v[:, :9], 8), _quantize_sh(v[:, 9:], 16)], axis=1)
    flags = FLAG_ANTIALIASED if cloud.antialiased else 0
    head = HEADER.pack(MAGIC, opts.version, n, deg, FRACTIONAL_BITS, flags, 0)
    return b"".join([head, pos_b.astype(np.uint8).tobytes(), alpha_b.tobytes(), color_b.tobytes(),
                     scale_b.tobytes(), rot_b.tobytes(), sh_b.tobytes()])


def _smallest_three(q: np.ndarray) -> np.ndarray:
    n = q.shape[0]
    big = np.argmax(np.abs(q), axis=1)  # the first of equal largest magnitudes
    neg = q[np.arange(n), big] < 0
    comp = big.astype(np.uint64)
    sqrt_half = np.float32(math.sqrt(0.5))
    for i in range(4):
        c = q[:, i]
        bit = ((c < 0) ^ neg).astype(np.uint64)
        # 511 * (|c| / sqrt(1/2)) + 0.5, truncated
        mag = (np.float32(511.0) * (np.abs(c) / sqrt_half) + np.float32(0.5)).astype(np.uint64)
        mag = np.minimum(mag, 511)
        take = big != i
        comp = np.where(take, (comp << np.uint64(10)) | (bit << np.uint64(9)) | mag, comp)
    comp = comp.astype(np.uint32)
    return np.stack([comp & 0xFF, (comp >> 8) & 0xFF, (comp >> 16) & 0xFF, comp >> 24],
                    axis=1).astype(np.uint8)


def _unpack_smallest_three(b: np.ndarray) -> np.ndarray:
    comp = (b[:, 0].astype(np.uint32) | (b[:, 1].astype(np.uint32) << 8)
            | (b[:, 2].astype(np.uint32) << 16) | (b[:, 3].astype(np.uint32) << 24))
    n = len(comp)
    big = (comp >> 30).astype(np.int64)
    q = np.zeros((n, 4), np.float32)
    ss = np.zeros(n, np.float32)
    for i in (3, 2, 1, 0):
        take = big != i
        mag = (comp & 511).astype(np.float32)
        neg = ((comp >> 9) & 1) == 1
        v = np.float32(math.sqrt(0.5)) * mag / np.float32(511.0)
        v = np.where(neg, -v, v)
        q[:, i] = np.where(take, v, q[:, i])
        ss = ss + np.where(take, v * v, np.float32(0.0))
        comp = np.where(take, comp >> 10, comp)
    q[np.arange(n), big] = np.sqrt(np.maximum(np.float32(0.0), np.float32(1.0) - ss))
    return q


def unpack_gaussians(data: bytes, opts: Optional[UnpackOptions] = None) -> GaussianCloud:
    """Decode an uncompressed .spz stream (versions 1-3)."""
    opts = opts or UnpackOptions()
    if len(data) < HEADER.size:
        raise SpzError("spz stream shorter than its header")
    magic, version, n, deg, fbits, flags, _ = HEADER.unpack_from(data, 0)
    if magic != MAGIC:
        raise SpzError("not an spz stream (bad magic)")
    if version not in (1, 2, 3) or deg not in SH_DIM:
        raise SpzError(f"unsupported spz version {version} / SH degree {deg}")
    dim = SH_DIM[deg]
    pos_bytes = n * 3 * (2 if version == 1 else 3)
    rot_bytes = n * (4 if version >= 3 else 3)
    sizes = [pos_bytes, n, 3 * n, 3 * n, rot_bytes, n * dim * 3]
    if len(data) < HEADER.size + sum(sizes):
        raise SpzError("spz stream shorter than its header declares")
    off = HEADER.size
    parts = []
    for s in sizes:
        parts.append(np.frombuffer(data, dtype=np.uint8, count=s, offset=off))
        off += s
    pb, ab, cb, sb, rb, hb = parts
    if version == 1:
        pos = np.frombuffer(pb.tobytes(), dtype="<f2").astype(np.float32)
    else:
        p = pb.reshape(-1, 3).astype(np.int32)
        v = p[:, 0] | (p[:, 1] << 8) | (p[:, 2] << 16)
        v = np.where(v & 0x800000, v - (1 << 24), v)
        pos = v.astype(np.float32) / np.float32(1 << fbits)
    alpha_lin = ab.astype(np.float32) / np.float32(255.0)
    with np.errstate(divide="ignore"):
        alphas = np.log(alpha_lin / (np.float32(1.0) - alpha_lin)).astype(np.float32)
    colors = (cb.astype(np.float32) / np.float32(255.0) - np.float32(0.5)) / np.float32(COLOR_SCALE)
    scales = sb.astype(np.float32) / np.float32(16.0) - np.float32(10.0)
    if version >= 3:
        rot = _unpack_smallest_three(rb.reshape(n, 4))
    else:
        xyz = rb.reshape(n, 3).astype(np.float32) / np.float32(127.5) - np.float32(1.0)
        w = np.sqrt(np.maximum(np.float32(0.0), np.float32(1.0) - (xyz * xyz).sum(axis=1)))
        rot = np.concatenate([xyz, w[:, None]], axis=1)
    sh = (hb.astype(np.float32) - np.float32(128.0)) / np.float32(128.0)
    pos, rot, sh = _convert(pos.reshape(-1), rot.reshape(-1), sh, dim,
                            _flips(CoordinateSystem.RUB, opts.to_coord))
    return GaussianCloud(positions=pos, scales=scales, rotations=rot.astype(np.float32),
                         alphas=alphas, colors=colors, sh=sh.astype(np.float32), sh_degree=deg,
                         antialiased=bool(flags & FLAG_ANTIALIASED))


def save_spz(cloud: GaussianCloud, opts: Optional[PackOptions] = None,
             filename: Union[str, os.PathLike, None] = None) -> bool:
    """``spz.save_spz(cloud, opts, filename)``: pack, gzip (zlib's default
    level) and write.  Returns True; raises on an inconsistent cloud."""
    if filename is None:
        raise SpzError("save_spz needs a file name")
    raw = pack_gaussians(cloud, opts)
    co = zlib.compressobj(zlib.Z_DEFAULT_COMPRESSION, zlib.DEFLATED, 16 + zlib.MAX_WBITS)
    with open(filename, "wb") as f:
        f.write(co.compress(raw) + co.flush())
    return True


def load_spz(filename: Union[str, os.PathLike], opts: Optional[UnpackOptions] = None
             ) -> GaussianCloud:
    with open(filename, "rb") as f:
        blob = f.read()
    try:
        raw = gzip.decompress(blob)
    except (OSError, EOFError, zlib.error) as e:
        raise SpzError(f"{filename}: not a gzip stream ({e})") from None
    return unpack_gaussians(raw, opts)
