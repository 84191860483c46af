// fgs_device.hpp -- device-side building blocks shared by the FastGS HIP
// kernels (gfx950, wave64).
//
// Numerics contract: every integer-deciding quantity (radii, tile counts,
// depth bits, blend skip/stop decisions) is computed with the operation order
// of the reference Metal source, with FP contraction disabled for the whole
// library (-ffp-contract=off), IEEE correctly rounded '/' and sqrt, and the
// deterministic exp/log below.  The CPU parity oracle evaluates the same
// operations, so those integers agree bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace fgs {

constexpr int kTile = 16;
constexpr int kTilePixels = kTile * kTile;
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Deterministic transcendental functions.
// ---------------------------------------------------------------------------

// exp(x): Cody-Waite reduction n = floor(x*log2(e)), r = x - n*ln2 (ln2 as a
// float head and tail, fused multiply-adds); e^r = 1 + r*q(r), q a degree-5
// polynomial fitted at 400 Chebyshev nodes on [-0.02, 0.72], Horner with fused
// multiply-adds; scaled by ldexp.  x clamped at -87 (normal range).  Max
// relative error 9.6e-8 on [-87, 0].
__device__ __forceinline__ float det_expf(float x) {
  x = fmaxf(x, -87.0f);
  const float t = x * 1.44269504088896341f;
  const float n = floorf(t);
  float r = __builtin_fmaf(-n, 0.6931471824645996f, x);
  r = __builtin_fmaf(-n, -1.9046542121259336e-09f, r);
  float q = 0.0018846612656489015f;
  q = __builtin_fmaf(q, r, 0.00792612787336111f);
  q = __builtin_fmaf(q, r, 0.041812896728515625f);
  q = __builtin_fmaf(q, r, 0.16664455831050873f);
  q = __builtin_fmaf(q, r, 0.5000009536743164f);
  q = __builtin_fmaf(q, r, 1.0f);
  const float p = __builtin_fmaf(r, q, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// log2(e) rounded to float.
constexpr float kLog2e = 1.44269504088896341f;

// The rasterizer's blend exponent is kept in base 2: G = exp(power) =
// 2^t with t = log2(e) power.  log2(e) enters the splat's conic coefficients
// once per splat (splat_log2_coeffs), so no pixel multiplies by it.
//
// 2^t for t <= 0 where it is used: t is clamped at -126, n = floor(t) and
// f = min(t - floor(t), 0x1.fffffep-1) in [0, 1), which are what
// v_cvt_flr_i32_f32 and v_fract_f32 return (checked against floorf and the
// IEEE subtraction for every float in [-126, 8]); 2^f = 1 + f*q(f), q of
// degree 4 fitted to the relative error at 400 Chebyshev nodes on [0, 1]
// (iteratively reweighted least squares), Horner with fused multiply-adds;
// scaled by ldexp.  Relative error at most 2e-7 against 2^t.  Nine
// instructions; used by the rasterizer's forward and backward, which decide
// from the same value.
__device__ __forceinline__ float blend_exp2f(float t) {
  t = fmaxf(t, -126.0f);
  const float f = __builtin_amdgcn_fractf(t);
  int n;
  asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(t));
  float q = 0x1.e86492p-10f;
  q = __builtin_fmaf(q, f, 0x1.279248p-7f);
  q = __builtin_fmaf(q, f, 0x1.c925b2p-5f);
  q = __builtin_fmaf(q, f, 0x1.ebd92ep-3f);
  q = __builtin_fmaf(q, f, 0x1.62e4d4p-1f);
  return __builtin_ldexpf(__builtin_fmaf(f, q, 1.0f), n);
}

// Base-2 exponent coefficients of a splat with conic (a, b, c):
// A = (-a/2) log2(e), B = -b log2(e), C = (-c/2) log2(e), one rounding each,
// so that t = A dx^2 + B dx dy + C dy^2 = log2(e) power.
__device__ __forceinline__ float3 splat_log2_coeffs(float a, float b, float c) {
  return make_float3((-0.5f * a) * kLog2e, -b * kLog2e, (-0.5f * c) * kLog2e);
}

// Exponent of a splat at offset (dx, dy) from its centre, from the
// coefficients (A, B, C) of splat_log2_coeffs: t = A dx^2 + B dx dy + C dy^2,
// evaluated as fma(dy, fma(C, dy, B dx), (A dx) dx) so that per splat B dx
// and (A dx) dx can be kept and every pixel row costs two fused
// multiply-adds.  Absolute error at most 3 * 2^-24 (|A| dx^2 + |B dx dy| +
// |C| dy^2), plus the coefficients' roundings (2^-24 relative each).
__device__ __forceinline__ float splat_power_rows(float Bdx, float Adxdx, float C, float dy) {
  return __builtin_fmaf(dy, __builtin_fmaf(C, dy, Bdx), Adxdx);
}
__device__ __forceinline__ float splat_power(float A, float B, float C, float dx, float dy) {
  return splat_power_rows(B * dx, (A * dx) * dx, C, dy);
}

// The training scripts' parameter activations (train_scanner_fixed.py:523-536):
// scale = exp(log_scale), rotation = q / (|q| + 1e-8), opacity =
// sigmoid(logit).  Shared by the activation kernel and the preprocess kernels'
// raw-parameter forms, so they agree bit for bit.
__device__ __forceinline__ float act_scale(float log_scale) { return expf(log_scale); }
__device__ __forceinline__ float4 act_rotation(float4 q) {
  const float n = sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
  const float d = n + 1e-8f;
  return make_float4(q.x / d, q.y / d, q.z / d, q.w / d);
}
__device__ __forceinline__ float act_opacity(float logit) { return 1.0f / (1.0f + expf(-logit)); }

// Gradient through the training scripts' rotation activation
// r = q / (|q| + 1e-8): dq = g/d - q (q.g) / (d^2 |q|), d = |q| + 1e-8 (the
// second term is 0 at q = 0).  Shared by the activation backward and the
// preprocess backward's fused form, so the two agree bit for bit.
__device__ __forceinline__ float4 quat_normalize_grad(float4 q, float4 g) {
  const float n = sqrtf(q.x * q.x + q.y * q.y + q.z * q.z + q.w * q.w);
  const float d = n + 1e-8f;
  const float qg = q.x * g.x + q.y * g.y + q.z * g.z + q.w * g.w;
  const float c = n > 0.0f ? qg / (d * d * n) : 0.0f;
  return make_float4(g.x / d - q.x * c, g.y / d - q.y * c, g.z / d - q.z * c, g.w / d - q.w * c);
}

// XCD-aware workgroup order.  The GPU hands the workgroups of a launch to its
// 8 XCDs round robin in dispatch order (linear id L goes to XCD L % 8), and
// each XCD has its own L2.  xcd_local_order(L, N) maps the N linear ids onto
// logical indices so that every XCD runs one contiguous range of them:
// workgroups that are neighbours in the logical order (and read overlapping
// data) then run on the same XCD, at about the same time, and share its L2.
// A bijection of [0, N).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_local_order(int L, int N) {
  const int x = L % kXcds, k = L / kXcds;
  const int q = N / kXcds, r = N % kXcds;
  return x * q + (x < r ? x : r) + k;
}

// ln(x): x = m*2^e with m in [sqrt(1/2), sqrt(2)); ln(m) = 2*atanh(s),
// s = (m-1)/(m+1), Taylor series to s^19 in double, rounded to float.
__device__ __forceinline__ float det_logf(float x) {
  if (!(x > 0.0f)) return (x == 0.0f) ? -__builtin_huge_valf() : __builtin_nanf("");
  if (__builtin_isinf(x)) return x;
  int e;
  float m = __builtin_frexpf(x, &e);
  if (m < 0.70710678118654752f) {
    m = m * 2.0f;
    e = e - 1;
  }
  const double md = (double)m;
  const double s = (md - 1.0) / (md + 1.0);
  const double s2 = s * s;
  double poly = 0.052631578947368418;
  poly = poly * s2 + 0.058823529411764705;
  poly = poly * s2 + 0.066666666666666666;
  poly = poly * s2 + 0.076923076923076927;
  poly = poly * s2 + 0.090909090909090912;
  poly = poly * s2 + 0.1111111111111111;
  poly = poly * s2 + 0.14285714285714285;
  poly = poly * s2 + 0.2;
  poly = poly * s2 + 0.33333333333333331;
  poly = poly * s2 + 1.0;
  const double r = (double)e * 0.69314718055994529 + 2.0 * s * poly;
  return (float)r;
}

// float -> int: truncation toward zero, NaN -> 0, saturating.
__device__ __forceinline__ int f2i(float v) {
  if (!(v == v)) return 0;
  if (v >= 2147483648.0f) return 2147483647;
  if (v <= -2147483648.0f) return (-2147483647 - 1);
  return (int)v;
}

__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }
__device__ __forceinline__ int imax(int a, int b) { return a > b ? a : b; }

// ---------------------------------------------------------------------------
// Exact tile footprint walk (reference fastgs_preprocess.metal:247-382 and
// fastgs_binning.metal:23-180).  The longer tile axis is swept line by line,
// intersecting the ellipse {d : 1/2 d^T Conic d <= t}, t = mult*2*ln(255 o),
// with the tile-boundary lines.  emit(tile_id) is called for every touched
// tile in sweep order; the number of touched tiles is returned.  A line whose
// tile interval is empty or inverted contributes nothing.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void ellipse_isect(float4 co, float disc, float t, float px, float py,
                                              bool is_y, float coord, float& lo, float& hi) {
  const float p_u = is_y ? py : px;
  const float p_v = is_y ? px : py;
  const float coeff = is_y ? co.x : co.z;
  const float h = coord - p_u;
  const float sq = __builtin_sqrtf(disc * h * h + t * coeff);
  lo = (-co.y * h - sq) / coeff + p_v;
  hi = (-co.y * h + sq) / coeff + p_v;
}

// Walk consumers may define rect(x0, x1, y0, y1): it is called once, before
// any span, with the walk's tile rectangle [x0, x1) x [y0, y1), which holds
// every span the walk emits.
template <typename E, typename = void>
struct HasRect : std::false_type {};
template <typename E>
struct HasRect<E, std::void_t<decltype(std::declval<E&>().rect(0, 0, 0, 0))>> : std::true_type {};

// The walk's set-up: the bounding box of the ellipse, its tile rectangle
// (emit.rect is called with it) and the swept axis.  Axis 0 is the swept one
// after the swap (is_y: the walk runs over tile rows).  empty: a degenerate
// conic or an empty rectangle (the walk touches nothing).
struct WalkSetup {
  float disc, t;
  float am1, aM1;                  // the bounding box's argmin / argmax on the other axis
  float bmin0, bmax0, bmin1, bmax1;
  int rmin0, rmax0, rmin1, rmax1;  // tile rectangle, axis 0 swept
  bool is_y;
  bool empty;
};

template <typename Emit>
__device__ __forceinline__ WalkSetup walk_setup(float px, float py, float4 co, int gx, int gy,
                                                float mult, Emit& emit) {
  WalkSetup w;
  w.empty = true;
  w.disc = co.y * co.y - co.x * co.z;
  if (co.x <= 0.0f || co.z <= 0.0f || w.disc >= 0.0f) return w;
  const float disc = w.disc;
  float t = 2.0f * det_logf(co.w * 255.0f);
  t = mult * t;
  w.t = t;
  float x_term = __builtin_sqrtf(-(co.y * co.y * t) / (disc * co.x));
  x_term = (co.y < 0.0f) ? x_term : -x_term;
  float y_term = __builtin_sqrtf(-(co.y * co.y * t) / (disc * co.z));
  y_term = (co.y < 0.0f) ? y_term : -y_term;
  float am0 = py - y_term, am1 = px - x_term;  // bbox_argmin
  float aM0 = py + y_term, aM1 = px + x_term;  // bbox_argmax
  float lo, hi;
  float bmin0, bmin1, bmax0, bmax1;
  ellipse_isect(co, disc, t, px, py, true, am0, lo, hi);
  bmin0 = lo;
  ellipse_isect(co, disc, t, px, py, false, am1, lo, hi);
  bmin1 = lo;
  ellipse_isect(co, disc, t, px, py, true, aM0, lo, hi);
  bmax0 = hi;
  ellipse_isect(co, disc, t, px, py, false, aM1, lo, hi);
  bmax1 = hi;
  int rmin0 = imax(0, imin(gx, f2i(bmin0 / 16.0f)));
  int rmin1 = imax(0, imin(gy, f2i(bmin1 / 16.0f)));
  int rmax0 = imax(0, imin(gx, f2i(bmax0 / 16.0f + 1.0f)));
  int rmax1 = imax(0, imin(gy, f2i(bmax1 / 16.0f + 1.0f)));
  const int y_span = rmax1 - rmin1;
  const int x_span = rmax0 - rmin0;
  if (y_span * x_span == 0) return w;
  if constexpr (HasRect<std::remove_reference_t<Emit>>::value) emit.rect(rmin0, rmax0, rmin1, rmax1);
  const bool is_y = y_span < x_span;
  if (is_y) {
    int ti;
    float tf;
    ti = rmin0; rmin0 = rmin1; rmin1 = ti;
    ti = rmax0; rmax0 = rmax1; rmax1 = ti;
    tf = bmin0; bmin0 = bmin1; bmin1 = tf;
    tf = bmax0; bmax0 = bmax1; bmax1 = tf;
    tf = am0; am0 = am1; am1 = tf;
    tf = aM0; aM0 = aM1; aM1 = tf;
  }
  w.am1 = am1;
  w.aM1 = aM1;
  w.bmin0 = bmin0;
  w.bmax0 = bmax0;
  w.bmin1 = bmin1;
  w.bmax1 = bmax1;
  w.rmin0 = rmin0;
  w.rmax0 = rmax0;
  w.rmin1 = rmin1;
  w.rmax1 = rmax1;
  w.is_y = is_y;
  w.empty = false;
  return w;
}

// One line's tile interval [vmin, vmax) on the other axis, from the line's
// near-edge intersection il and far-edge intersection iM.
__device__ __forceinline__ void walk_line_span(const WalkSetup& w, float min_line, float max_line,
                                               float il0, float il1, float iM0, float iM1,
                                               int& vmin, int& vmax) {
  float e_min, e_max;
  if (min_line <= w.am1 && w.am1 < max_line)
    e_min = w.bmin1;
  else
    e_min = fminf(il0, iM0);
  if (min_line <= w.aM1 && w.aM1 < max_line)
    e_max = w.bmax1;
  else
    e_max = fmaxf(il1, iM1);
  vmin = imax(w.rmin1, imin(w.rmax1, f2i(e_min / 16.0f)));
  vmax = imin(w.rmax1, imax(w.rmin1, f2i(e_max / 16.0f + 1.0f)));
}

// The line loop of the walk over lines [u0, u1) of the swept axis (u0 >=
// rmin0).  The line state at u0 is the one the full walk reaches there: the
// previous line's far edge u0*16 is always intersected.
template <typename Emit>
__device__ __forceinline__ uint32_t walk_lines(const WalkSetup& w, float px, float py, float4 co,
                                               int u0, int u1, Emit&& emit) {
  uint32_t count = 0;
  float il0, il1;                      // intersect_min_line
  float iM0 = w.bmax1, iM1 = w.bmin1;  // intersect_max_line
  float min_line = (float)u0 * 16.0f;
  if (u0 > w.rmin0) {
    // the full walk's line u0-1 intersected its far edge u0*16 (u0*16 <= bmax0)
    ellipse_isect(co, w.disc, w.t, px, py, w.is_y, min_line, il0, il1);
    iM0 = il0;
    iM1 = il1;
  } else if (w.bmin0 <= min_line) {
    ellipse_isect(co, w.disc, w.t, px, py, w.is_y, (float)w.rmin0 * 16.0f, il0, il1);
  } else {
    il0 = iM0;
    il1 = iM1;
  }
  for (int u = u0; u < u1; ++u) {
    const float max_line = min_line + 16.0f;
    if (max_line <= w.bmax0) ellipse_isect(co, w.disc, w.t, px, py, w.is_y, max_line, iM0, iM1);
    int min_tile_v, max_tile_v;
    walk_line_span(w, min_line, max_line, il0, il1, iM0, iM1, min_tile_v, max_tile_v);
    if (max_tile_v > min_tile_v) {
      count += (uint32_t)(max_tile_v - min_tile_v);
      emit(u, min_tile_v, max_tile_v, w.is_y);
    }
    il0 = iM0;
    il1 = iM1;
    min_line = max_line;
  }
  return count;
}

// The walk restricted to the tile window [wx0, wx1) x [wy0, wy1): lines u
// outside the window's range on the walked axis are not visited, and the
// line state at the first visited line is the one the full walk reaches
// there (the previous line's far edge, u*16, is always intersected), so every
// emitted span is bit-identical to the full walk's.  Spans are not clipped on
// the other axis.
template <typename Emit>
__device__ __forceinline__ uint32_t tiles_walk_window(float px, float py, float4 co, int gx, int gy,
                                                      float mult, int wx0, int wx1, int wy0,
                                                      int wy1, Emit&& emit) {
  const WalkSetup w = walk_setup(px, py, co, gx, gy, mult, emit);
  if (w.empty) return 0u;
  int u0 = w.rmin0, u1 = w.rmax0;
  if (w.is_y) {
    u0 = imax(u0, wy0);
    u1 = imin(u1, wy1);
  } else {
    u0 = imax(u0, wx0);
    u1 = imin(u1, wx1);
  }
  return walk_lines(w, px, py, co, u0, u1, emit);
}

template <typename Emit>
__device__ __forceinline__ uint32_t tiles_walk(float px, float py, float4 co, int gx, int gy,
                                               float mult, Emit&& emit) {
  return tiles_walk_window(px, py, co, gx, gy, mult, 0, gx, 0, gy, emit);
}

// The full walk of one Gaussian by a whole wavefront: every lane passes the
// same (px, py, co); lane l takes lines rmin0 + l, rmin0 + l + 64, ... and
// computes each line's span as walk_lines does.  The state walk_lines carries
// from line to line is rebuilt per line: the far edge (u+1)*16 is intersected
// while it is at most bmax0 (a prefix of the lines), later lines keep the
// last such intersection, and a line's near-edge state is the previous line's
// far-edge state (the lane below, or the previous round's last lane).  Each
// lane's spans go to its own emit; the return value is the wavefront's total
// (the same on every lane).  Called by all 64 lanes with uniform inputs.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, kWave);
  return v;
}

template <typename Emit>
__device__ __forceinline__ uint32_t tiles_walk_wave(float px, float py, float4 co, int gx, int gy,
                                                    float mult, Emit&& emit) {
  const WalkSetup w = walk_setup(px, py, co, gx, gy, mult, emit);
  if (w.empty) return 0u;  // uniform
  const int u0 = w.rmin0, u1 = w.rmax0;
  const int l = (int)(threadIdx.x & (kWave - 1));
  // far-edge state before the first line, and the near-edge state of line u0
  float last0 = w.bmax1, last1 = w.bmin1;
  float prev0 = last0, prev1 = last1;
  if (w.bmin0 <= (float)u0 * 16.0f)
    ellipse_isect(co, w.disc, w.t, px, py, w.is_y, (float)w.rmin0 * 16.0f, prev0, prev1);
  uint32_t count = 0;
  for (int base = u0; base < u1; base += kWave) {
    const int u = base + l;
    const bool in = u < u1;
    const float min_line = (float)u * 16.0f;
    const float max_line = min_line + 16.0f;
    const bool far = in && max_line <= w.bmax0;
    float iM0 = 0.0f, iM1 = 0.0f;
    if (far) ellipse_isect(co, w.disc, w.t, px, py, w.is_y, max_line, iM0, iM1);
    const int nf = __popcll(__ballot(far));  // the far lanes are lanes [0, nf)
    if (nf > 0) {
      last0 = __shfl(iM0, nf - 1, kWave);
      last1 = __shfl(iM1, nf - 1, kWave);
    }
    if (!far) {
      iM0 = last0;
      iM1 = last1;
    }
    float il0 = __shfl_up(iM0, 1, kWave), il1 = __shfl_up(iM1, 1, kWave);
    if (l == 0) {
      il0 = prev0;
      il1 = prev1;
    }
    if (in) {
      int vmin, vmax;
      walk_line_span(w, min_line, max_line, il0, il1, iM0, iM1, vmin, vmax);
      if (vmax > vmin) {
        count += (uint32_t)(vmax - vmin);
        emit(u, vmin, vmax, w.is_y);
      }
    }
    prev0 = __shfl(iM0, kWave - 1, kWave);
    prev1 = __shfl(iM1, kWave - 1, kWave);
  }
  return wave_sum_u32(count);
}

struct NoEmit {
  __device__ __forceinline__ void operator()(int, int, int, bool) const {}
};

// ---------------------------------------------------------------------------
// Super-tile record of a Gaussian, built during the exact walk for the
// two-level tile binning.  Super-tiles are 8x8 tiles, numbered row-major on a
// grid sgx wide.  Two forms share four 64-bit words m0..m3:
//  - fits: the walk rectangle lies in the 2x2 super-tiles from (bx, by), the
//    super-tile of its corner.  m_k holds the tiles in super-tile
//    (bx + (k & 1), by + (k >> 1)), bit (y mod 8) * 8 + (x mod 8) for tile
//    (x, y).  Record word bx | by << 12 | kStRecFits.
//  - set: any other rectangle, on grids of at most 256 super-tiles: bit s of
//    m0..m3 (m_k holding s = 64k..64k+63) marks each super-tile s holding at
//    least one of the Gaussian's tiles.  Record word kStRecSet.
// A Gaussian that touches no tile, or a wide one on a larger grid, has record
// word 0.
//
// A fits record whose tile rectangle is at most 8x8 tiles, from tile (x0, y0)
// with x0, y0 < 4096, is stored compact: its tiles as one 8x8 board relative
// to (x0, y0) (bit (y - y0) * 8 + (x - x0)), record word
// x0 | y0 << 12 | kStRecCompact.  The 16-byte record (word, 0, board) is all
// the binning then gathers for it; st_expand_compact gives back the fits form.
// ---------------------------------------------------------------------------
constexpr int kStTiles = 8;
constexpr int kStMaxSet = 256;
constexpr uint32_t kStRecFits = 1u << 31;
constexpr uint32_t kStRecSet = 1u << 30;
constexpr uint32_t kStRecCompact = 1u << 29;

// 8x8 bit boards (byte r = row r, bit c = column c): the low n bits of every
// row, 0 <= n <= 8.
__device__ __forceinline__ uint64_t st_byte_mask(int n) {
  return 0x0101010101010101ull * (uint64_t)((1u << n) - 1u);
}

// The fits form (four boards of the 2x2 super-tiles from the one holding
// (x0, y0)) of a compact board M, with (ox, oy) = (x0 mod 8, y0 mod 8):
// board column c goes to column ox + c, left (m0, m2) or right (m1, m3);
// board row r to row oy + r, top (m0, m1) or bottom (m2, m3).
__device__ __forceinline__ void st_expand_compact(uint64_t M, int ox, int oy, uint64_t (&m)[4]) {
  const uint64_t lw = (M << ox) & ~st_byte_mask(ox);
  const uint64_t rw = ox ? ((M >> (8 - ox)) & st_byte_mask(ox)) : 0ull;
  m[0] = lw << (8 * oy);
  m[1] = rw << (8 * oy);
  m[2] = oy ? (lw >> (64 - 8 * oy)) : 0ull;
  m[3] = oy ? (rw >> (64 - 8 * oy)) : 0ull;
}

// bits [a, b) of one 8-bit mask row (0 <= a, b <= 8)
__device__ __forceinline__ uint64_t st_row_bits(int a, int b) {
  return b > a ? (((1ull << (b - a)) - 1ull) << a) : 0ull;
}

// rows [a, b) of mask column c (0 <= a, b <= 8)
__device__ __forceinline__ uint64_t st_col_bits(int a, int b, int c) {
  if (b <= a) return 0ull;
  const uint64_t hi = (b >= 8) ? ~0ull : ((1ull << (8 * b)) - 1ull);
  const uint64_t lo = (1ull << (8 * a)) - 1ull;
  return (hi & ~lo) & (0x0101010101010101ull << c);
}

// bits [lo, hi] of the 256-bit word lo..hi <= 255, as four 64-bit words:
// word k gets the part of the range inside [64k, 64k + 63]
__device__ __forceinline__ uint64_t st_set_word(int lo, int hi, int k) {
  const int a = imax(lo, 64 * k), z = imin(hi, 64 * k + 63);
  if (z < a) return 0ull;
  const int n = z - a + 1;
  return ((n >= 64) ? ~0ull : ((1ull << n) - 1ull)) << (a - 64 * k);
}

// The record bits of one walk span (tile row u, columns [vmin, vmax), or
// column u, rows [vmin, vmax)) for a Gaussian with the given record geometry
// (fits: the 2x2 super-tiles from (bx, by); otherwise, when set_ok, the
// super-tile set on a grid sgx super-tiles wide).  Every update is a select on
// all four words: a branch or an index here becomes a scratch access.
__device__ __forceinline__ void st_span_bits(bool fits, bool set_ok, int bx, int by, int sgx, int u,
                                             int vmin, int vmax, bool is_y, uint64_t (&d)[4]) {
  d[0] = d[1] = d[2] = d[3] = 0ull;
  if (fits) {
    if (is_y) {  // tile row u, columns [vmin, vmax)
      const int r = u - kStTiles * by;
      const int c0 = vmin - kStTiles * bx, c1 = vmax - kStTiles * bx;
      const int sh = (r & 7) * 8;
      const uint64_t a = st_row_bits(c0, imin(c1, 8)) << sh;
      const uint64_t b = st_row_bits(imax(c0, 8) - 8, c1 - 8) << sh;
      const bool top = r < 8;
      d[0] = top ? a : 0ull;
      d[1] = top ? b : 0ull;
      d[2] = top ? 0ull : a;
      d[3] = top ? 0ull : b;
    } else {  // tile column u, rows [vmin, vmax)
      const int c = u - kStTiles * bx;
      const int r0 = vmin - kStTiles * by, r1 = vmax - kStTiles * by;
      const uint64_t a = st_col_bits(r0, imin(r1, 8), c & 7);
      const uint64_t b = st_col_bits(imax(r0, 8) - 8, r1 - 8, c & 7);
      const bool left = c < 8;
      d[0] = left ? a : 0ull;
      d[2] = left ? b : 0ull;
      d[1] = left ? 0ull : a;
      d[3] = left ? 0ull : b;
    }
  } else if (set_ok) {
    const int b = u / kStTiles;
    const int c0 = vmin / kStTiles, c1 = (vmax - 1) / kStTiles;
    if (is_y) {  // row u: super-tiles b*sgx + c0 .. b*sgx + c1
      const int lo = b * sgx + c0, hi = b * sgx + c1;
      d[0] = st_set_word(lo, hi, 0);
      d[1] = st_set_word(lo, hi, 1);
      d[2] = st_set_word(lo, hi, 2);
      d[3] = st_set_word(lo, hi, 3);
    } else {  // column u: super-tiles c*sgx + b, c = c0..c1
      for (int c = c0; c <= c1; ++c) {
        const int sb = c * sgx + b;
        const uint64_t bit = 1ull << (sb & 63);
        const int k = sb >> 6;
        d[0] |= k == 0 ? bit : 0ull;
        d[1] |= k == 1 ? bit : 0ull;
        d[2] |= k == 2 ? bit : 0ull;
        d[3] |= k == 3 ? bit : 0ull;
      }
    }
  }
}

struct EmitStRecord {
  uint64_t m0 = 0ull, m1 = 0ull, m2 = 0ull, m3 = 0ull;
  int bx = 0, by = 0;
  int ox = 0, oy = 0;    // the rectangle's corner inside super-tile (bx, by)
  int sgx = 0;           // super-tile grid width
  bool set_ok = false;   // the grid has at most kStMaxSet super-tiles
  bool fits = false;
  bool compact = false;  // fits, in at most 8x8 tiles from a corner below 4096
  __device__ __forceinline__ EmitStRecord(int gx, int gy) {
    sgx = (gx + kStTiles - 1) / kStTiles;
    set_ok = sgx * ((gy + kStTiles - 1) / kStTiles) <= kStMaxSet;
  }
  __device__ __forceinline__ void rect(int x0, int x1, int y0, int y1) {
    bx = x0 / kStTiles;
    by = y0 / kStTiles;
    fits = (x1 - 1) / kStTiles - bx <= 1 && (y1 - 1) / kStTiles - by <= 1 && bx < 4096 &&
           by < 4096;
    ox = x0 - kStTiles * bx;
    oy = y0 - kStTiles * by;
    compact = fits && x1 - x0 <= kStTiles && y1 - y0 <= kStTiles && x0 < 4096 && y0 < 4096;
  }
  __device__ __forceinline__ void operator()(int u, int vmin, int vmax, bool is_y) {
    uint64_t d[4];
    st_span_bits(fits, set_ok, bx, by, sgx, u, vmin, vmax, is_y, d);
    m0 |= d[0];
    m1 |= d[1];
    m2 |= d[2];
    m3 |= d[3];
  }
  __device__ __forceinline__ uint32_t word() const {
    if (fits) return (uint32_t)bx | ((uint32_t)by << 12) | kStRecFits;
    return set_ok ? kStRecSet : 0u;
  }
  // compact form: the word and the 8x8 board from (ox, oy) of the 16x16
  // tiles m0..m3 cover (rows oy.., then columns ox..; every tile of a compact
  // rectangle lies there)
  __device__ __forceinline__ uint32_t compact_word() const {
    return (uint32_t)(kStTiles * bx + ox) | ((uint32_t)(kStTiles * by + oy) << 12) | kStRecCompact;
  }
  __device__ __forceinline__ uint64_t compact_board() const {
    const uint64_t l = oy ? ((m0 >> (8 * oy)) | (m2 << (64 - 8 * oy))) : m0;
    const uint64_t r = oy ? ((m1 >> (8 * oy)) | (m3 << (64 - 8 * oy))) : m1;
    const uint64_t keep = st_byte_mask(8 - ox);
    return ((l >> ox) & keep) | (ox ? ((r << (8 - ox)) & ~keep) : 0ull);
  }
  // OR of the four words over the wavefront (after tiles_walk_wave)
  __device__ __forceinline__ void wave_or() {
    uint32_t v[8] = {(uint32_t)m0, (uint32_t)(m0 >> 32), (uint32_t)m1, (uint32_t)(m1 >> 32),
                     (uint32_t)m2, (uint32_t)(m2 >> 32), (uint32_t)m3, (uint32_t)(m3 >> 32)};
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1)
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] |= (uint32_t)__shfl_xor((int)v[k], o, kWave);
    m0 = (uint64_t)v[0] | ((uint64_t)v[1] << 32);
    m1 = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
    m2 = (uint64_t)v[4] | ((uint64_t)v[5] << 32);
    m3 = (uint64_t)v[6] | ((uint64_t)v[7] << 32);
  }
};

// ---------------------------------------------------------------------------
// Wave64 primitives.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Workgroup barrier that orders LDS only.  __syncthreads() also makes every
// earlier global access of the thread complete (s_waitcnt vmcnt(0)), which
// drains loads issued ahead and fire-and-forget atomics; where the barrier
// guards nothing but LDS, this form lets them stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return (l == 0) ? 0ull : ((~0ull) >> (64 - l));
}

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t t = __shfl_up(v, (unsigned)o, kWave);
    if (l >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    const uint32_t t = __shfl_xor(v, o, kWave);
    v = v > t ? v : t;
  }
  return v;
}

// DPP lane move (GFX9 data-parallel primitives): lanes whose source is out of
// range, or whose row is masked off, read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes with DPP adds; the total is valid in lane 63 only.
// quad_perm(1,0,3,2), quad_perm(2,3,0,1), row_shr:4, row_shr:8 sum each row
// of 16 into its lane 15; row_bcast:15 and row_bcast:31 fold the four rows.
__device__ __forceinline__ float wave_sum_lane63(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x114>(v);
  v += dpp_mov<0x118>(v);
  v += dpp_mov<0x142, 0xA>(v);
  v += dpp_mov<0x143, 0xC>(v);
  return v;
}

// Block-wide exclusive scan of one u32 per thread (blockDim.x a multiple of
// 64, at most 1024).  Returns the exclusive prefix; *total gets the block sum.
// s_tmp needs blockDim.x/64 + 1 entries.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t* s_tmp, uint32_t* total) {
  const int nw = (int)(blockDim.x / kWave);
  const int w = (int)(threadIdx.x / kWave);
  const uint32_t incl = wave_incl_scan(v);
  if (lane_id() == kWave - 1) s_tmp[w] = incl;
  __syncthreads();
  if (w == 0) {
    uint32_t x = (lane_id() < nw) ? s_tmp[lane_id()] : 0u;
    const uint32_t xi = wave_incl_scan(x);
    if (lane_id() < nw) s_tmp[lane_id()] = xi - x;
    if (lane_id() == nw - 1) s_tmp[nw] = xi;
  }
  __syncthreads();
  const uint32_t r = s_tmp[w] + incl - v;
  if (total) *total = s_tmp[nw];
  __syncthreads();
  return r;
}

}  // namespace fgs
