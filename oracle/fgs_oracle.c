/*
 * fgs_oracle.c -- CPU restatement of the FastGS rasterizer (reference: the
 * Metal kernels of a1091150/fastgs_core) used as the PARITY ORACLE.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product path (fastgs_core_amd) never calls
 * it and fails loudly when the HIP library is missing.
 *
 * Build: compiled twice by oracle/Makefile.
 *   liborc_f32.so : real = float.  This is the parity oracle.  Arithmetic is
 *                   evaluated in the operation order written in the reference
 *                   Metal source, with -ffp-contract=off, correctly rounded
 *                   '/' and sqrt, and the deterministic orc_expf / orc_logf
 *                   below, which the HIP kernels implement with the same
 *                   operations.  Integer outputs are therefore bit-identical.
 *                   Two rasterizer steps are written in another order, each
 *                   stated where it is used: the blend exponent in base 2
 *                   (splat_power, orc_blend_exp2f: exp(power) = 2^t) and the
 *                   transmittance update T (1 - alpha) as fma(-alpha, T, T).
 *   liborc_f64.so : real = double, libm exp/log.  Used by the finite-difference
 *                   tests that pin the analytic backward.
 *
 * Every function cites the reference file:line it restates.  Where the
 * reference has a hazard (out-of-bounds read, uninitialised LDS, uint wrap,
 * NaN->int) the definition chosen is stated at the point of use.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#ifdef ORC_DOUBLE
typedef double real;
#define RSQRT(x) sqrt(x)
#define RFLOOR(x) floor(x)
#define RCEIL(x) ceil(x)
#define RABS(x) fabs(x)
#define RMIN(a, b) fmin(a, b)
#define RMAX(a, b) fmax(a, b)
#define REXP(x) exp(x)
#define RBEXP2(x) exp2(x)
#define ORC_LOG2E 1.4426950408889634
#define RFMA(a, b, c) fma(a, b, c)
#define RLOG(x) log(x)
#define REXP_LIBM(x) exp(x)
#else
typedef float real;
#define RSQRT(x) sqrtf(x)
#define RFLOOR(x) floorf(x)
#define RCEIL(x) ceilf(x)
#define RABS(x) fabsf(x)
#define RMIN(a, b) fminf(a, b)
#define RMAX(a, b) fmaxf(a, b)
#define REXP(x) orc_expf(x)
#define RBEXP2(x) orc_blend_exp2f(x)
#define ORC_LOG2E 1.44269504088896341f
#define RFMA(a, b, c) fmaf(a, b, c)
#define RLOG(x) orc_logf(x)
#define REXP_LIBM(x) expf(x)
#endif

#define ORC_TILE 16

/* ------------------------------------------------------------------------ */
/* Deterministic transcendental functions (float build).                     */
/* ------------------------------------------------------------------------ */

/* exp(x) by Cody-Waite reduction: n = floor(x*log2(e)), r = x - n*ln2 with
 * ln2 split in a float head and tail applied by fused multiply-adds, so r is
 * in [0, ln2) up to rounding; e^r = 1 + r*q(r) with q a degree-5 polynomial
 * fitted at 400 Chebyshev nodes on [-0.02, 0.72], Horner with correctly
 * rounded fused multiply-adds; scaled by ldexp (exact).  x is clamped at -87
 * so the result stays normal.  Max relative error 9.6e-8 on [-87, 0]. */
float orc_expf(float x) {
  x = fmaxf(x, -87.0f);
  const float t = x * 1.44269504088896341f;
  const float n = floorf(t);
  float r = fmaf(-n, 0.6931471824645996f, x);
  r = fmaf(-n, -1.9046542121259336e-09f, r);
  float q = 0.0018846612656489015f;
  q = fmaf(q, r, 0.00792612787336111f);
  q = fmaf(q, r, 0.041812896728515625f);
  q = fmaf(q, r, 0.16664455831050873f);
  q = fmaf(q, r, 0.5000009536743164f);
  q = fmaf(q, r, 1.0f);
  const float p = fmaf(r, q, 1.0f);
  return ldexpf(p, (int)n);
}

/* 2^t for the rasterizer's base-2 blend exponent t = log2(e) power (its
 * G = exp(power); the coefficients of splat_power carry log2(e)): t clamped
 * at -126, n = floor(t), f = min(t - n, 0x1.fffffep-1) in [0, 1) (t - n
 * rounds to 1 for t just below 0; the HIP kernels' v_fract_f32 returns this
 * clamped value and their v_cvt_flr_i32_f32 floor(t), checked for every float
 * in [-126, 8]); 2^f = 1 + f*q(f), q of degree 4 fitted to the relative error
 * at 400 Chebyshev nodes on [0, 1] by iteratively reweighted least squares,
 * Horner with correctly rounded fused multiply-adds; scaled by ldexp (exact).
 * Relative error at most 2e-7 against 2^t; tests/test_oracle_math.py pins it
 * against float64 exp2. */
float orc_blend_exp2f(float t) {
  t = fmaxf(t, -126.0f);
  const float n = floorf(t);
  const float f = fminf(t - n, 0x1.fffffep-1f);
  float q = 0x1.e86492p-10f;
  q = fmaf(q, f, 0x1.279248p-7f);
  q = fmaf(q, f, 0x1.c925b2p-5f);
  q = fmaf(q, f, 0x1.ebd92ep-3f);
  q = fmaf(q, f, 0x1.62e4d4p-1f);
  return ldexpf(fmaf(f, q, 1.0f), (int)n);
}

/* ln(x) for float x: x = m*2^e with m in [sqrt(1/2), sqrt(2)), then
 * ln(m) = 2*atanh(s), s = (m-1)/(m+1), by its Taylor series to s^19 in
 * double precision (|s| <= 0.1716, truncation < 2e-16), result rounded to
 * float.  Only IEEE basic operations are used, so the HIP kernels reproduce
 * it bit for bit. */
float orc_logf(float x) {
  if (!(x > 0.0f)) return (x == 0.0f) ? -INFINITY : NAN;
  if (isinf(x)) return x;
  int e;
  float m = frexpf(x, &e);
  if (m < 0.70710678118654752f) {
    m = m * 2.0f;
    e = e - 1;
  }
  double md = (double)m;
  double s = (md - 1.0) / (md + 1.0);
  double s2 = s * s;
  double poly = 0.052631578947368418;    /* 1/19 */
  poly = poly * s2 + 0.058823529411764705; /* 1/17 */
  poly = poly * s2 + 0.066666666666666666; /* 1/15 */
  poly = poly * s2 + 0.076923076923076927; /* 1/13 */
  poly = poly * s2 + 0.090909090909090912; /* 1/11 */
  poly = poly * s2 + 0.1111111111111111;   /* 1/9 */
  poly = poly * s2 + 0.14285714285714285;  /* 1/7 */
  poly = poly * s2 + 0.2;                  /* 1/5 */
  poly = poly * s2 + 0.33333333333333331;  /* 1/3 */
  poly = poly * s2 + 1.0;
  double r = (double)e * 0.69314718055994529 + 2.0 * s * poly;
  return (float)r;
}

/* float -> int conversion with truncation toward zero, NaN -> 0 and
 * saturation.  The reference (Metal) leaves NaN/out-of-range conversion
 * unspecified; NaN arises for opacity < 1/255 (fastgs_preprocess.metal:337). */
static inline int32_t orc_f2i(real v) {
  if (!(v == v)) return 0;
  if (v >= (real)2147483648.0) return INT32_MAX;
  if (v <= (real)-2147483648.0) return INT32_MIN;
  return (int32_t)v;
}

/* Base-2 exponent of a splat at offset (dx, dy) from its centre: t =
 * log2(e) power, power = -1/2 (a dx^2 + c dy^2) - b dx dy for the conic
 * (a, b, c) (the blend loops of fastgs_rasterize.metal:105-106 and
 * fastgs_rasterize_backward.metal:189-190, whose exp(power) is 2^t), written
 * as A dx^2 + B dx dy + C dy^2 with A = (-a/2) log2(e), B = -b log2(e),
 * C = (-c/2) log2(e) (one rounding each) and evaluated as
 * fma(dy, fma(C, dy, B dx), (A dx) dx), the HIP kernels' operation order.
 * t > 0 exactly where the reference's power > 0 up to these roundings. */
static inline real splat_power(const real* co, real dx, real dy) {
  const real A = ((real)-0.5 * co[0]) * ORC_LOG2E, B = -co[1] * ORC_LOG2E;
  const real C = ((real)-0.5 * co[2]) * ORC_LOG2E;
  return RFMA(dy, RFMA(C, dy, B * dx), (A * dx) * dx);
}

/* splat_power of the conic (a, b, c) at (dx, dy), exported for its error-bound
 * test (inputs and result converted to and from real). */
double orc_splat_power(double a, double b, double c, double dx, double dy) {
  const real co[4] = {(real)a, (real)b, (real)c, (real)0};
  return (double)splat_power(co, (real)dx, (real)dy);
}

static inline int imin(int a, int b) { return a < b ? a : b; }
static inline int imax(int a, int b) { return a > b ? a : b; }

/* ------------------------------------------------------------------------ */
/* Parameter block shared with oracle.py (ctypes).                           */
/* ------------------------------------------------------------------------ */
typedef struct {
  int32_t P;
  int32_t degree;
  int32_t max_sh_coeffs;
  int32_t image_width;
  int32_t image_height;
  int32_t grid_x;
  int32_t grid_y;
  int32_t use_cov3d_precomp;
  int32_t use_colors_precomp;
  float scale_modifier;
  float mult;
  float tan_fovx;
  float tan_fovy;
} orc_params;

static const real SH_C0 = (real)0.28209479177387814;
static const real SH_C1 = (real)0.4886025119029199;
static const real SH_C2[5] = {(real)1.0925484305920792, (real)-1.0925484305920792,
                              (real)0.31539156525252005, (real)-1.0925484305920792,
                              (real)0.5462742152960396};
static const real SH_C3[7] = {(real)-0.5900435899266435, (real)2.890611442640554,
                              (real)-0.4570457994644658, (real)0.3731763325901154,
                              (real)-0.4570457994644658, (real)1.445305721320277,
                              (real)-0.5900435899266435};

/* transform_point_4x3 (fastgs_preprocess.metal:81-86); matrices are 4x4
 * column-major flat arrays. */
static inline void xform43(const real* m, real x, real y, real z, real out[3]) {
  out[0] = m[0] * x + m[4] * y + m[8] * z + m[12];
  out[1] = m[1] * x + m[5] * y + m[9] * z + m[13];
  out[2] = m[2] * x + m[6] * y + m[10] * z + m[14];
}

/* transform_point_4x4 (fastgs_preprocess.metal:88-94). */
static inline void xform44(const real* m, real x, real y, real z, real out[4]) {
  out[0] = m[0] * x + m[4] * y + m[8] * z + m[12];
  out[1] = m[1] * x + m[5] * y + m[9] * z + m[13];
  out[2] = m[2] * x + m[6] * y + m[10] * z + m[14];
  out[3] = m[3] * x + m[7] * y + m[11] * z + m[15];
}

/* compute_cov3d (fastgs_preprocess.metal:207-231).  The Metal float3x3
 * constructor fills columns: rmat[c][r].  M = S*R, Sigma = M^T M.  Output
 * (Sigma00, Sigma01, Sigma02, Sigma11, Sigma12, Sigma22) in Metal indexing. */
static void cov3d_from_scale_rot(const real s3[3], real mod, const real q[4], real out[6]) {
  real r = q[0], x = q[1], y = q[2], z = q[3];
  real R[3][3]; /* R[col][row] */
  R[0][0] = (real)1 - (real)2 * (y * y + z * z);
  R[0][1] = (real)2 * (x * y - r * z);
  R[0][2] = (real)2 * (x * z + r * y);
  R[1][0] = (real)2 * (x * y + r * z);
  R[1][1] = (real)1 - (real)2 * (x * x + z * z);
  R[1][2] = (real)2 * (y * z - r * x);
  R[2][0] = (real)2 * (x * z - r * y);
  R[2][1] = (real)2 * (y * z + r * x);
  R[2][2] = (real)1 - (real)2 * (x * x + y * y);
  real s[3] = {mod * s3[0], mod * s3[1], mod * s3[2]};
  /* M = S*R with S diagonal: M[c][r] = s[r] * R[c][r] */
  real M[3][3];
  for (int c = 0; c < 3; ++c)
    for (int rr = 0; rr < 3; ++rr) M[c][rr] = s[rr] * R[c][rr];
  /* Sigma[i][j] = sum_k M^T[k][j]... as math: Sigma(j,i) = sum_k M(k,j) M(k,i);
   * M(k,j) = M[j][k].  Evaluated k = 0,1,2 left to right. */
#define SIG(i, j) (M[j][0] * M[i][0] + M[j][1] * M[i][1] + M[j][2] * M[i][2])
  out[0] = SIG(0, 0);
  out[1] = SIG(0, 1);
  out[2] = SIG(0, 2);
  out[3] = SIG(1, 1);
  out[4] = SIG(1, 2);
  out[5] = SIG(2, 2);
#undef SIG
}

/* compute_cov2d (fastgs_preprocess.metal:171-205) and its re-evaluation in
 * fastgs_preprocess_backward.metal:113-139.  W is built column-wise from
 * viewmatrix[0,1,2],[4,5,6],[8,9,10] (so W = R, the view rotation), J has the
 * EWA entries in its columns, T = W*J, cov = T^T Vrk T.  Tcol[c][r] holds T in
 * Metal indexing (column c, row r); the third column of T is zero.
 * Returns (cov00, cov01, cov11) without the +0.3, plus t, J and T for the
 * backward. */
typedef struct {
  real t[3];     /* view-space mean after the frustum clamp */
  real txtz, tytz, limx, limy;
  real j00, j02, j11, j12; /* Metal J[0][0], J[0][2], J[1][1], J[1][2] */
  real T[3][3];  /* T[col][row] */
  real cov00, cov01, cov11;
} orc_cov2d;

static void cov2d_eval(const real* view, const real mean[3], real focal_x, real focal_y,
                       real tan_fovx, real tan_fovy, const real c3[6], orc_cov2d* o) {
  real t[3];
  xform43(view, mean[0], mean[1], mean[2], t);
  real limx = (real)1.3 * tan_fovx;
  real limy = (real)1.3 * tan_fovy;
  real txtz = t[0] / t[2];
  real tytz = t[1] / t[2];
  t[0] = RMIN(limx, RMAX(-limx, txtz)) * t[2];
  t[1] = RMIN(limy, RMAX(-limy, tytz)) * t[2];
  o->t[0] = t[0];
  o->t[1] = t[1];
  o->t[2] = t[2];
  o->txtz = txtz;
  o->tytz = tytz;
  o->limx = limx;
  o->limy = limy;
  real j00 = focal_x / t[2];
  real j02 = -(focal_x * t[0]) / (t[2] * t[2]);
  real j11 = focal_y / t[2];
  real j12 = -(focal_y * t[1]) / (t[2] * t[2]);
  o->j00 = j00;
  o->j02 = j02;
  o->j11 = j11;
  o->j12 = j12;
  /* W[col][row] = view[4*col + row].  T = W*J (math): T(r,0) = W(r,0) J(0,0) +
   * W(r,2) J(2,0); T(r,1) = W(r,1) J(1,1) + W(r,2) J(2,1), where the math
   * J(2,0) is Metal J[0][2] and J(2,1) is Metal J[1][2].  Zero terms of the
   * 3x3 product are omitted. */
  for (int r = 0; r < 3; ++r) {
    o->T[0][r] = view[0 + r] * j00 + view[8 + r] * j02;
    o->T[1][r] = view[4 + r] * j11 + view[8 + r] * j12;
    o->T[2][r] = (real)0;
  }
  /* Vrk symmetric: V(r,s) */
  real V[3][3] = {{c3[0], c3[1], c3[2]}, {c3[1], c3[3], c3[4]}, {c3[2], c3[4], c3[5]}};
  /* U(c,s) = sum_r T(r,c) V(r,s), c in {0,1} */
  real U[2][3];
  for (int c = 0; c < 2; ++c)
    for (int s = 0; s < 3; ++s)
      U[c][s] = o->T[c][0] * V[0][s] + o->T[c][1] * V[1][s] + o->T[c][2] * V[2][s];
  /* cov(c,d) = sum_s U(c,s) T(s,d).  Metal cov[0][1] is math cov(1,0). */
  o->cov00 = U[0][0] * o->T[0][0] + U[0][1] * o->T[0][1] + U[0][2] * o->T[0][2];
  o->cov01 = U[1][0] * o->T[0][0] + U[1][1] * o->T[0][1] + U[1][2] * o->T[0][2];
  o->cov11 = U[1][0] * o->T[1][0] + U[1][1] * o->T[1][1] + U[1][2] * o->T[1][2];
}

/* ------------------------------------------------------------------------ */
/* Exact tile footprint (fastgs_preprocess.metal:247-382,                    */
/* fastgs_binning.metal:23-180).                                             */
/* ------------------------------------------------------------------------ */

/* compute_ellipse_intersection (fastgs_preprocess.metal:247-261). */
static inline void ellipse_isect(const real co[4], real disc, real t, real px, real py, int is_y,
                                 real coord, real* lo, real* hi) {
  real p_u = is_y ? py : px;
  real p_v = is_y ? px : py;
  real coeff = is_y ? co[0] : co[2];
  real h = coord - p_u;
  real sq = RSQRT(disc * h * h + t * coeff);
  *lo = (-co[1] * h - sq) / coeff + p_v;
  *hi = (-co[1] * h + sq) / coeff + p_v;
}

typedef void (*orc_emit_fn)(void* ctx, int tile_id);

/* duplicate_to_tiles_touched + process_tiles (fastgs_preprocess.metal:263-382)
 * and duplicate_with_keys + process_tiles (fastgs_binning.metal:39-180).
 * Walks the longer tile axis line by line.  When emit != NULL every touched
 * tile id (y*grid_x + x) is reported in sweep order.  Returns the count.
 * Definition (reference hazard): a line whose computed [min_tile_v,
 * max_tile_v) is empty or inverted contributes 0 (the reference adds the
 * uint-wrapped difference in the counting kernel while its emitting kernel
 * writes nothing for that line). */
static uint32_t tiles_walk(real px, real py, const real co[4], int gx, int gy, real mult,
                           orc_emit_fn emit, void* ctx) {
  real disc = co[1] * co[1] - co[0] * co[2];
  if (co[0] <= (real)0 || co[2] <= (real)0 || disc >= (real)0) return 0;
  real t = (real)2 * RLOG(co[3] * (real)255);
  t = (real)mult * t;
  real x_term = RSQRT(-(co[1] * co[1] * t) / (disc * co[0]));
  x_term = (co[1] < (real)0) ? x_term : -x_term;
  real y_term = RSQRT(-(co[1] * co[1] * t) / (disc * co[2]));
  y_term = (co[1] < (real)0) ? y_term : -y_term;
  real argmin[2] = {py - y_term, px - x_term};
  real argmax[2] = {py + y_term, px + x_term};
  real lo, hi, bmin[2], bmax[2];
  ellipse_isect(co, disc, t, px, py, 1, argmin[0], &lo, &hi);
  bmin[0] = lo;
  ellipse_isect(co, disc, t, px, py, 0, argmin[1], &lo, &hi);
  bmin[1] = lo;
  ellipse_isect(co, disc, t, px, py, 1, argmax[0], &lo, &hi);
  bmax[0] = hi;
  ellipse_isect(co, disc, t, px, py, 0, argmax[1], &lo, &hi);
  bmax[1] = hi;
  int rmin[2] = {imax(0, imin(gx, orc_f2i(bmin[0] / (real)ORC_TILE))),
                 imax(0, imin(gy, orc_f2i(bmin[1] / (real)ORC_TILE)))};
  int rmax[2] = {imax(0, imin(gx, orc_f2i(bmax[0] / (real)ORC_TILE + (real)1))),
                 imax(0, imin(gy, orc_f2i(bmax[1] / (real)ORC_TILE + (real)1)))};
  int y_span = rmax[1] - rmin[1];
  int x_span = rmax[0] - rmin[0];
  if (y_span * x_span == 0) return 0;
  int is_y = y_span < x_span;
  if (is_y) {
    int ti;
    real tr;
    ti = rmin[0]; rmin[0] = rmin[1]; rmin[1] = ti;
    ti = rmax[0]; rmax[0] = rmax[1]; rmax[1] = ti;
    tr = bmin[0]; bmin[0] = bmin[1]; bmin[1] = tr;
    tr = bmax[0]; bmax[0] = bmax[1]; bmax[1] = tr;
    tr = argmin[0]; argmin[0] = argmin[1]; argmin[1] = tr;
    tr = argmax[0]; argmax[0] = argmax[1]; argmax[1] = tr;
  }
  const real block_u = (real)ORC_TILE, block_v = (real)ORC_TILE;
  uint32_t count = 0;
  real imin_l[2], imax_l[2] = {bmax[1], bmin[1]};
  real min_line = (real)rmin[0] * block_u;
  if (bmin[0] <= min_line) {
    ellipse_isect(co, disc, t, px, py, is_y, (real)rmin[0] * block_u, &imin_l[0], &imin_l[1]);
  } else {
    imin_l[0] = imax_l[0];
    imin_l[1] = imax_l[1];
  }
  for (int u = rmin[0]; u < rmax[0]; ++u) {
    real max_line = min_line + block_u;
    if (max_line <= bmax[0]) {
      ellipse_isect(co, disc, t, px, py, is_y, max_line, &imax_l[0], &imax_l[1]);
    }
    real e_min, e_max;
    if (min_line <= argmin[1] && argmin[1] < max_line)
      e_min = bmin[1];
    else
      e_min = RMIN(imin_l[0], imax_l[0]);
    if (min_line <= argmax[1] && argmax[1] < max_line)
      e_max = bmax[1];
    else
      e_max = RMAX(imin_l[1], imax_l[1]);
    int min_tile_v = imax(rmin[1], imin(rmax[1], orc_f2i(e_min / block_v)));
    int max_tile_v = imin(rmax[1], imax(rmin[1], orc_f2i(e_max / block_v + (real)1)));
    if (max_tile_v > min_tile_v) {
      count += (uint32_t)(max_tile_v - min_tile_v);
      if (emit) {
        for (int v = min_tile_v; v < max_tile_v; ++v)
          emit(ctx, is_y ? (u * gx + v) : (v * gx + u));
      }
    }
    imin_l[0] = imax_l[0];
    imin_l[1] = imax_l[1];
    min_line = max_line;
  }
  return count;
}

uint32_t orc_tiles_touched_one(real px, real py, const real* co, int gx, int gy, real mult) {
  return tiles_walk(px, py, co, gx, gy, mult, NULL, NULL);
}

/* compute_color_from_sh (fastgs_preprocess.metal:117-169): real SH basis up
 * to degree 3 evaluated at dir = (mean - campos) / |mean - campos|, plus 0.5,
 * clamped at 0 with the clamp mask.  s points at the Gaussian's rest
 * coefficients s[k*3 + c], k = 0..14. */
void orc_color_from_sh(int degree, const real* mean, const real* campos, const real* d,
                       const real* s, real* col, uint8_t* clamped) {
  real v[3] = {mean[0] - campos[0], mean[1] - campos[1], mean[2] - campos[2]};
  real len = RSQRT(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  real x = v[0] / len, y = v[1] / len, z = v[2] / len;
  for (int c = 0; c < 3; ++c) {
    real res = SH_C0 * d[c];
    if (degree > 0) {
      res = res - SH_C1 * y * s[0 * 3 + c] + SH_C1 * z * s[1 * 3 + c] - SH_C1 * x * s[2 * 3 + c];
      if (degree > 1) {
        real xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
        res += SH_C2[0] * xy * s[3 * 3 + c] + SH_C2[1] * yz * s[4 * 3 + c] +
               SH_C2[2] * ((real)2 * zz - xx - yy) * s[5 * 3 + c] +
               SH_C2[3] * xz * s[6 * 3 + c] + SH_C2[4] * (xx - yy) * s[7 * 3 + c];
        if (degree > 2) {
          res += SH_C3[0] * y * ((real)3 * xx - yy) * s[8 * 3 + c] +
                 SH_C3[1] * xy * z * s[9 * 3 + c] +
                 SH_C3[2] * y * ((real)4 * zz - xx - yy) * s[10 * 3 + c] +
                 SH_C3[3] * z * ((real)2 * zz - (real)3 * xx - (real)3 * yy) * s[11 * 3 + c] +
                 SH_C3[4] * x * ((real)4 * zz - xx - yy) * s[12 * 3 + c] +
                 SH_C3[5] * z * (xx - yy) * s[13 * 3 + c] +
                 SH_C3[6] * x * (xx - (real)3 * yy) * s[14 * 3 + c];
        }
      }
    }
    res += (real)0.5;
    clamped[c] = res < (real)0;
    col[c] = RMAX(res, (real)0);
  }
}

/* ------------------------------------------------------------------------ */
/* Preprocess forward (fastgs_preprocess.metal:384-484).                     */
/* Outputs must be zero-filled by the caller (fastgs_preprocess.cpp:83-86).  */
/* ------------------------------------------------------------------------ */
void orc_preprocess_fwd(const orc_params* prm, const real* means3d, const real* dc,
                        const real* sh, const real* colors_precomp, const real* opacities,
                        const real* scales, const real* rotations, const real* cov3d_precomp,
                        const real* viewmatrix, const real* projmatrix, const real* campos,
                        const real* vsp_in, int32_t* radii, real* xys, real* depths,
                        real* cov3d, real* rgb, real* conic_opacity, uint32_t* tiles_touched,
                        uint8_t* clamped, real* vsp_out) {
  const int P = prm->P;
  /* focal = W / (2 tan_fov) (fastgs_preprocess.cpp:120-121), float */
  const real focal_x = (real)((float)prm->image_width / (2.0f * prm->tan_fovx));
  const real focal_y = (real)((float)prm->image_height / (2.0f * prm->tan_fovy));
#pragma omp parallel for schedule(dynamic, 1024)
  for (int i = 0; i < P; ++i) {
    radii[i] = 0;
    tiles_touched[i] = 0;
    const real* m = means3d + 3 * (size_t)i;
    real p_view[3];
    xform43(viewmatrix, m[0], m[1], m[2], p_view);
    if (p_view[2] <= (real)0.2) continue; /* in_frustum :96-115 */
    real p_hom[4];
    xform44(projmatrix, m[0], m[1], m[2], p_hom);
    real p_w = (real)1 / (p_hom[3] + (real)1.0e-7);
    real p_proj[3] = {p_hom[0] * p_w, p_hom[1] * p_w, p_hom[2] * p_w};
    real c3[6];
    if (prm->use_cov3d_precomp) {
      for (int k = 0; k < 6; ++k) c3[k] = cov3d_precomp[6 * (size_t)i + k];
    } else {
      cov3d_from_scale_rot(scales + 3 * (size_t)i, (real)prm->scale_modifier,
                           rotations + 4 * (size_t)i, c3);
    }
    for (int k = 0; k < 6; ++k) cov3d[6 * (size_t)i + k] = c3[k];
    orc_cov2d cv;
    cov2d_eval(viewmatrix, m, focal_x, focal_y, (real)prm->tan_fovx, (real)prm->tan_fovy, c3, &cv);
    real cx = cv.cov00 + (real)0.3, cy = cv.cov01, cz = cv.cov11 + (real)0.3;
    real det = cx * cz - cy * cy;
    if (det == (real)0) continue;
    real det_inv = (real)1 / det;
    real conic[3] = {cz * det_inv, -cy * det_inv, cx * det_inv};
    real mid = (real)0.5 * (cx + cz);
    real lambda1 = mid + RSQRT(RMAX((real)0.1, mid * mid - det));
    real lambda2 = mid - RSQRT(RMAX((real)0.1, mid * mid - det));
    real my_radius = RCEIL((real)3 * RSQRT(RMAX(lambda1, lambda2)));
    real ptx = ((p_proj[0] + (real)1) * (real)prm->image_width - (real)1) * (real)0.5;
    real pty = ((p_proj[1] + (real)1) * (real)prm->image_height - (real)1) * (real)0.5;
    real co[4] = {conic[0], conic[1], conic[2], opacities[i]};
    uint32_t cnt = tiles_walk(ptx, pty, co, prm->grid_x, prm->grid_y, (real)prm->mult, NULL, NULL);
    if (cnt == 0) continue;
    real col[3];
    if (prm->use_colors_precomp) {
      for (int c = 0; c < 3; ++c) col[c] = colors_precomp[3 * (size_t)i + c];
      clamped[3 * (size_t)i + 0] = 0;
      clamped[3 * (size_t)i + 1] = 0;
      clamped[3 * (size_t)i + 2] = 0;
    } else {
      orc_color_from_sh(prm->degree, m, campos, dc + 3 * (size_t)i,
                        sh + (size_t)i * (size_t)prm->max_sh_coeffs * 3, col,
                        clamped + 3 * (size_t)i);
    }
    for (int c = 0; c < 3; ++c) rgb[3 * (size_t)i + c] = col[c];
    depths[i] = p_view[2];
    radii[i] = orc_f2i(my_radius);
    xys[2 * (size_t)i + 0] = ptx;
    xys[2 * (size_t)i + 1] = pty;
    for (int k = 0; k < 4; ++k) conic_opacity[4 * (size_t)i + k] = co[k];
    tiles_touched[i] = cnt;
    vsp_out[4 * (size_t)i + 0] = p_view[0];
    vsp_out[4 * (size_t)i + 1] = p_view[1];
    vsp_out[4 * (size_t)i + 2] = p_view[2];
    vsp_out[4 * (size_t)i + 3] = vsp_in[4 * (size_t)i + 3];
  }
}

/* ------------------------------------------------------------------------ */
/* Scan (binding.cpp:153,211: mx::cumsum inclusive) and duplicate-with-keys  */
/* (fastgs_binning.metal:182-213).                                           */
/* ------------------------------------------------------------------------ */
void orc_inclusive_scan_u32(int64_t n, const uint32_t* in, uint32_t* out) {
  uint32_t acc = 0;
  for (int64_t i = 0; i < n; ++i) {
    acc += in[i];
    out[i] = acc;
  }
}

typedef struct {
  uint64_t* keys;
  uint32_t* vals;
  uint64_t off;
  uint64_t cap;
  uint32_t depth_bits;
  uint32_t idx;
} emit_ctx;

static void emit_key(void* vctx, int tile_id) {
  emit_ctx* c = (emit_ctx*)vctx;
  /* Bound check: the reference writes unconditionally (fastgs_binning.metal:107). */
  if (c->off < c->cap) {
    c->keys[c->off] = ((uint64_t)(uint32_t)tile_id << 32) | (uint64_t)c->depth_bits;
    c->vals[c->off] = c->idx;
  }
  c->off++;
}

/* keys/vals (length K) must be zero-filled by the caller
 * (fastgs_binning.cpp, eval_gpu memset). */
void orc_duplicate_with_keys(int32_t P, const real* xys, const real* depths,
                             const uint32_t* point_offsets, const real* conic_opacity,
                             const uint32_t* tiles_touched, float mult, int32_t gx, int32_t gy,
                             int64_t K, uint64_t* keys, uint32_t* vals) {
  for (int i = 0; i < P; ++i) {
    if (tiles_touched[i] == 0) continue;
    emit_ctx c;
    c.keys = keys;
    c.vals = vals;
    c.off = (i == 0) ? 0 : point_offsets[i - 1];
    c.cap = (uint64_t)K;
    float df = (float)depths[i];
    memcpy(&c.depth_bits, &df, 4);
    c.idx = (uint32_t)i;
    real co[4] = {conic_opacity[4 * (size_t)i], conic_opacity[4 * (size_t)i + 1],
                  conic_opacity[4 * (size_t)i + 2], conic_opacity[4 * (size_t)i + 3]};
    tiles_walk(xys[2 * (size_t)i], xys[2 * (size_t)i + 1], co, gx, gy, (real)mult, emit_key, &c);
  }
}

/* Stable ascending sort of (key, value) pairs by the full 64-bit key: LSD
 * radix sort, 8-bit digits, ties keep their input order.  This is the
 * definition of the reference's mx::argsort + take (binding.cpp:195-197),
 * whose tie order MLX leaves unspecified. */
void orc_sort_pairs_u64(int64_t n, uint64_t* keys, uint32_t* vals) {
  if (n <= 1) return;
  uint64_t* k2 = (uint64_t*)malloc((size_t)n * 8);
  uint32_t* v2 = (uint32_t*)malloc((size_t)n * 4);
  uint64_t* ka = keys;
  uint32_t* va = vals;
  uint64_t* kb = k2;
  uint32_t* vb = v2;
  for (int pass = 0; pass < 8; ++pass) {
    int shift = pass * 8;
    size_t cnt[257];
    memset(cnt, 0, sizeof(cnt));
    for (int64_t i = 0; i < n; ++i) cnt[((ka[i] >> shift) & 255) + 1]++;
    int trivial = 0;
    for (int d = 0; d < 256; ++d)
      if (cnt[d + 1] == (size_t)n) trivial = 1;
    if (trivial) continue;
    for (int d = 0; d < 256; ++d) cnt[d + 1] += cnt[d];
    for (int64_t i = 0; i < n; ++i) {
      size_t pos = cnt[(ka[i] >> shift) & 255]++;
      kb[pos] = ka[i];
      vb[pos] = va[i];
    }
    uint64_t* tk = ka; ka = kb; kb = tk;
    uint32_t* tv = va; va = vb; vb = tv;
  }
  if (ka != keys) {
    memcpy(keys, ka, (size_t)n * 8);
    memcpy(vals, va, (size_t)n * 4);
  }
  free(k2);
  free(v2);
}

/* identify_tile_ranges + per_tile_bucket_count (fastgs_tile_prep.metal:10-53).
 * ranges (2*T) zero-filled by the caller.  Keys whose tile id is
 * 0xFFFFFFFF are ignored (:21); tile ids >= T are ignored (the reference would
 * write out of bounds). */
void orc_tile_ranges(int64_t K, const uint64_t* keys, int32_t T, uint32_t* ranges,
                     uint32_t* bucket_count) {
  for (int64_t i = 0; i < K; ++i) {
    uint32_t cur = (uint32_t)(keys[i] >> 32);
    int valid = cur != 0xFFFFFFFFu;
    if (i == 0) {
      if (cur < (uint32_t)T) ranges[2 * (size_t)cur] = 0;
    } else {
      uint32_t prev = (uint32_t)(keys[i - 1] >> 32);
      if (cur != prev) {
        if (prev < (uint32_t)T) ranges[2 * (size_t)prev + 1] = (uint32_t)i;
        if (valid && cur < (uint32_t)T) ranges[2 * (size_t)cur] = (uint32_t)i;
      }
    }
    if (i == K - 1 && valid && cur < (uint32_t)T) ranges[2 * (size_t)cur + 1] = (uint32_t)K;
  }
  for (int t = 0; t < T; ++t) {
    int n = (int)(ranges[2 * t + 1] - ranges[2 * t]);
    bucket_count[t] = (uint32_t)((n + 31) / 32);
  }
}

/* ------------------------------------------------------------------------ */
/* Rasterize forward (fastgs_rasterize.metal:25-159).                        */
/* ------------------------------------------------------------------------ */
typedef struct {
  int32_t image_width;
  int32_t image_height;
  int32_t num_channels;
  int32_t num_tiles;
  int64_t bucket_sum;
  int32_t get_flag;
  int32_t write_sampled;
  /* 0: the blend in the HIP kernels' operation order (base-2 exponent,
   * orc_blend_exp2f, T (1 - alpha) as one fused multiply-add): the parity
   * oracle.  1: the reference's own order (fastgs_rasterize.metal:104-118):
   * power = -1/2 (a dx dx + c dy dy) - b dx dy, alpha = min(0.99, o exp(power))
   * with libm expf, test_T = T (1 - alpha) rounded twice.  Mode 1 exists to
   * measure how often the two orders take a different blend decision. */
  int32_t ref_order;
} orc_rparams;

/* All outputs zero-filled by the caller.  colors has row stride
 * num_channels; min(num_channels,3) channels are blended.  max_contrib is the
 * maximum n_contrib over the tile's in-image pixels (the reference reads
 * uninitialised threadgroup memory for out-of-image threads,
 * fastgs_rasterize.metal:142). */
void orc_rasterize_fwd(const orc_rparams* rp, const uint32_t* ranges, const uint32_t* point_list,
                       const uint32_t* bucket_offsets, const real* means2d, const real* colors,
                       const real* conic_opacity, const real* background,
                       const int32_t* metric_map, uint32_t* bucket_to_tile, real* sampled_t,
                       real* sampled_ar, real* final_t, uint32_t* n_contrib,
                       uint32_t* max_contrib, real* pixel_colors, real* out_color,
                       int32_t* metric_count) {
  const int W = rp->image_width, H = rp->image_height;
  const int gx = (W + ORC_TILE - 1) / ORC_TILE;
  const int gy = (H + ORC_TILE - 1) / ORC_TILE;
  const int NC = rp->num_channels;
  const int C = NC < 3 ? NC : 3;
  const size_t HW = (size_t)W * (size_t)H;
  const int ntiles = gx * gy < rp->num_tiles ? gx * gy : rp->num_tiles;
#pragma omp parallel for schedule(dynamic, 1)
  for (int tile = 0; tile < ntiles; ++tile) {
    int tx = tile % gx, ty = tile / gx;
    uint32_t start = ranges[2 * tile], end = ranges[2 * tile + 1];
    int to_do = (int)(end - start);
    int nb = (to_do + 31) / 32;
    uint32_t bbm0 = (tile == 0) ? 0 : bucket_offsets[tile - 1];
    for (int b = 0; b < nb; ++b)
      if ((int64_t)bbm0 + b < rp->bucket_sum) bucket_to_tile[bbm0 + b] = (uint32_t)tile;
    uint32_t maxc = 0;
    for (int ly = 0; ly < ORC_TILE; ++ly) {
      for (int lx = 0; lx < ORC_TILE; ++lx) {
        int px = tx * ORC_TILE + lx, py = ty * ORC_TILE + ly;
        if (px >= W || py >= H) continue;
        size_t pix = (size_t)py * W + px;
        int lr = ly * ORC_TILE + lx;
        real pxf = (real)px, pyf = (real)py;
        real T = 1;
        uint32_t contributor = 0, last = 0;
        real acc[3] = {0, 0, 0};
        uint32_t bbm = bbm0;
        for (uint32_t idx = start; idx < end; ++idx) {
          if (((idx - start) % 32u) == 0u) {
            if (rp->write_sampled && (int64_t)bbm < rp->bucket_sum) {
              sampled_t[(size_t)bbm * 256 + lr] = T;
              for (int c = 0; c < C; ++c) sampled_ar[(size_t)bbm * NC * 256 + c * 256 + lr] = acc[c];
            }
            bbm++;
          }
          contributor++;
          uint32_t g = point_list[idx];
          real dx = means2d[2 * (size_t)g] - pxf;
          real dy = means2d[2 * (size_t)g + 1] - pyf;
          const real* co = conic_opacity + 4 * (size_t)g;
          real alpha, test_t;
          if (rp->ref_order) {
            real power = (real)-0.5 * (co[0] * dx * dx + co[2] * dy * dy) - co[1] * dx * dy;
            if (power > (real)0) continue;
            alpha = RMIN((real)0.99, co[3] * REXP_LIBM(power));
            if (alpha < (real)1 / (real)255) continue;
            test_t = T * ((real)1 - alpha);
          } else {
            real t2 = splat_power(co, dx, dy); /* log2(e) power */
            if (t2 > (real)0) continue;
            alpha = RMIN((real)0.99, co[3] * RBEXP2(t2));
            if (alpha < (real)1 / (real)255) continue;
            /* T (1 - alpha) as one fused multiply-add, the HIP kernel's form */
            test_t = RFMA(-alpha, T, T);
          }
          if (test_t < (real)0.0001) break;
          for (int c = 0; c < C; ++c) acc[c] += colors[(size_t)g * NC + c] * alpha * T;
          if (rp->get_flag && metric_map[pix] == 1) {
#pragma omp atomic
            metric_count[g] += 1;
          }
          T = test_t;
          last = contributor;
        }
        final_t[pix] = T;
        n_contrib[pix] = last;
        for (int c = 0; c < C; ++c) {
          pixel_colors[c * HW + pix] = acc[c];
          out_color[c * HW + pix] = acc[c] + T * background[c];
        }
        if (last > maxc) maxc = last;
      }
    }
    max_contrib[tile] = maxc;
  }
}

/* ------------------------------------------------------------------------ */
/* Rasterize backward: the per-(pixel, splat) semantics of                   */
/* fastgs_rasterize_backward.metal:24-278, evaluated per pixel by replaying  */
/* the forward front to back and accumulating in reverse.                    */
/* Gradient arrays are accumulated into (zero them first).                   */
/* ------------------------------------------------------------------------ */
/* mag (optional, NULL: not computed): two magnitudes of every gradient entry,
 * accumulated in double and laid out [P][2][10 + NC], each row ordered as
 * (means2d x, y, viewspace x, y, |x|, |y|, conic a, b, c, opacity, colours):
 *  [0] the sum over its (pixel, splat) terms of the term's magnitude with every
 *      sum inside the term replaced by the sum of its summands' magnitudes
 *      (|a + b| -> |a| + |b|): an implementation that evaluates the same terms
 *      in another order, recovers T another way or sums them in another order
 *      differs from these gradients by a small multiple of float epsilon
 *      times it;
 *  [1] the sum over its terms of |term|. */
void orc_rasterize_bwd_mag(const orc_rparams* rp, const uint32_t* ranges,
                           const uint32_t* point_list, const real* means2d, const real* colors,
                           const real* conic_opacity, const real* background, const real* final_t,
                           const uint32_t* n_contrib, const real* dL_dout, real* dmeans2d,
                           real* dcolors, real* dconic, real* dvsp, double* mag, int64_t mag_rows) {
  const int W = rp->image_width, H = rp->image_height;
  const int gx = (W + ORC_TILE - 1) / ORC_TILE;
  const int gy = (H + ORC_TILE - 1) / ORC_TILE;
  const int NC = rp->num_channels;
  const int C = NC < 3 ? NC : 3;
  const size_t HW = (size_t)W * (size_t)H;
  const real ddelx_dx = (real)0.5 * (real)W;
  const real ddely_dy = (real)0.5 * (real)H;
  const int ntiles = gx * gy < rp->num_tiles ? gx * gy : rp->num_tiles;
  /* The per-Gaussian sums are accumulated in double and added to the outputs
   * once at the end: the parallel order of the additions (the reference's
   * float atomics have none either) then moves the result by far less than a
   * float ulp, so the oracle gives the same gradients on every run. */
  size_t lmax = 0;
  for (int tile = 0; tile < ntiles; ++tile)
    if (ranges[2 * tile + 1] > lmax) lmax = ranges[2 * tile + 1];
  uint32_t gn = 0;
  for (size_t i = 0; i < lmax; ++i)
    if (point_list[i] + 1 > gn) gn = point_list[i] + 1;
  const int AW = 10 + NC; /* means2d 2, vsp 4, conic 4, colours NC */
  double* acc = (double*)calloc((size_t)gn * AW + 1, sizeof(double));
  double* macc = mag ? (double*)calloc((size_t)gn * AW * 2 + 1, sizeof(double)) : NULL;
#pragma omp parallel
  {
    int cap = 0;
    uint32_t* rec_g = NULL;
    uint32_t* rec_j = NULL; /* the splat's position in the tile's list */
    real* rec = NULL; /* per contributing splat: alpha, G, T, dx, dy */
    size_t tcap = 0;
    double* tb = NULL; /* per list position: AW sums, then 2 AW magnitudes */
#pragma omp for schedule(dynamic, 1)
    for (int tile = 0; tile < ntiles; ++tile) {
      int tx = tile % gx, ty = tile / gx;
      uint32_t start = ranges[2 * tile], end = ranges[2 * tile + 1];
      if (end <= start) continue;
      /* the tile's terms are summed per list position here, then added to
       * the per-Gaussian sums once per (tile, splat) */
      const size_t tw = (size_t)(macc ? 3 : 1) * AW;
      const size_t tn = (size_t)(end - start) * tw;
      if (tn > tcap) {
        tcap = tn * 2;
        tb = (double*)realloc(tb, tcap * sizeof(double));
      }
      memset(tb, 0, tn * sizeof(double));
      for (int ly = 0; ly < ORC_TILE; ++ly) {
        for (int lx = 0; lx < ORC_TILE; ++lx) {
          int px = tx * ORC_TILE + lx, py = ty * ORC_TILE + ly;
          if (px >= W || py >= H) continue;
          size_t pix = (size_t)py * W + px;
          uint32_t n = n_contrib[pix];
          if (n == 0) continue;
          if ((int)n > cap) {
            cap = (int)n * 2;
            rec_g = (uint32_t*)realloc(rec_g, (size_t)cap * 4);
            rec_j = (uint32_t*)realloc(rec_j, (size_t)cap * 4);
            rec = (real*)realloc(rec, (size_t)cap * 5 * sizeof(real));
          }
          real pxf = (real)px, pyf = (real)py;
          real T = 1;
          int m = 0;
          for (uint32_t j = 0; j < n && start + j < end; ++j) {
            uint32_t g = point_list[start + j];
            real dx = means2d[2 * (size_t)g] - pxf;
            real dy = means2d[2 * (size_t)g + 1] - pyf;
            const real* co = conic_opacity + 4 * (size_t)g;
            real t2 = splat_power(co, dx, dy); /* log2(e) power */
            if (t2 > (real)0) continue;
            real G = RBEXP2(t2);
            real alpha = RMIN((real)0.99, co[3] * G);
            if (alpha < (real)1 / (real)255) continue;
            rec_g[m] = g;
            rec_j[m] = j;
            rec[5 * m + 0] = alpha;
            rec[5 * m + 1] = G;
            rec[5 * m + 2] = T;
            rec[5 * m + 3] = dx;
            rec[5 * m + 4] = dy;
            m++;
            T = RFMA(-alpha, T, T); /* the forward's transmittance */
          }
          real Tf = final_t[pix];
          real dL[3] = {0, 0, 0};
          for (int c = 0; c < C; ++c) dL[c] = dL_dout[c * HW + pix];
          real bg_dot = 0;
          double bg_abs = 0;
          for (int c = 0; c < C; ++c) {
            bg_dot += background[c] * dL[c];
            bg_abs += fabs((double)background[c] * (double)dL[c]);
          }
          real S[3] = {0, 0, 0}; /* sum over later splats of c*alpha*T */
          double Sm[3] = {0, 0, 0}; /* sum over later splats of |c|*alpha*T */
          for (int k = m - 1; k >= 0; --k) {
            uint32_t g = rec_g[k];
            double* ta = tb + (size_t)rec_j[k] * tw; /* sums of this splat's terms */
            double* tmg = ta + AW;                  /* and of their magnitudes */
            real alpha = rec[5 * k + 0], G = rec[5 * k + 1], Tj = rec[5 * k + 2];
            real dx = rec[5 * k + 3], dy = rec[5 * k + 4];
            const real* co = conic_opacity + 4 * (size_t)g;
            real rci = (real)1 / ((real)1 - alpha);
            real dL_dalpha = 0;
            double ma = 0; /* magnitude of dL_dalpha */
            for (int c = 0; c < C; ++c) {
              real col = colors[(size_t)g * NC + c];
              real dcol = alpha * Tj * dL[c];
              ta[10 + c] += (double)dcol;
              dL_dalpha += (col * Tj - rci * S[c]) * dL[c];
              S[c] += col * alpha * Tj;
              if (macc) {
                const double adl = fabs((double)dL[c]);
                tmg[10 + c] += (double)alpha * (double)Tj * adl;
                tmg[AW + 10 + c] += fabs((double)dcol);
                ma += (fabs((double)col) * (double)Tj + (double)rci * Sm[c]) * adl;
                Sm[c] += fabs((double)col) * (double)alpha * (double)Tj;
              }
            }
            dL_dalpha += (-Tf * rci) * bg_dot;
            ma += fabs((double)Tf * (double)rci) * bg_abs;
            if (co[3] * G > (real)0.99) continue;
            if (macc) {
              const double mG = fabs((double)co[3]) * ma; /* |dL_dG| */
              const double gx_ = fabs((double)G * (double)dx), gy_ = fabs((double)G * (double)dy);
              const double mx = mG * (gx_ * fabs((double)co[0]) + gy_ * fabs((double)co[1])) *
                                fabs((double)ddelx_dx);
              const double my = mG * (gy_ * fabs((double)co[2]) + gx_ * fabs((double)co[1])) *
                                fabs((double)ddely_dy);
              double* b = tmg;
              b[0] += mx;
              b[1] += my;
              b[2] += mx;
              b[3] += my;
              b[4] += mx;
              b[5] += my;
              b[6] += 0.5 * gx_ * fabs((double)dx) * mG;
              b[7] += 0.5 * gx_ * fabs((double)dy) * mG;
              b[8] += 0.5 * gy_ * fabs((double)dy) * mG;
              b[9] += (double)G * ma;
            }
            real dL_dG = co[3] * dL_dalpha;
            real gdx = G * dx, gdy = G * dy;
            real dG_ddelx = -gdx * co[0] - gdy * co[1];
            real dG_ddely = -gdy * co[2] - gdx * co[1];
            real tmp_x = dL_dG * dG_ddelx * ddelx_dx;
            real tmp_y = dL_dG * dG_ddely * ddely_dy;
            real v0 = (real)-0.5 * gdx * dx * dL_dG;
            real v1 = (real)-0.5 * gdx * dy * dL_dG;
            real v2 = (real)-0.5 * gdy * dy * dL_dG;
            real v3 = G * dL_dalpha;
            double* a = ta;
            a[0] += (double)tmp_x;
            a[1] += (double)tmp_y;
            a[2] += (double)tmp_x;
            a[3] += (double)tmp_y;
            a[4] += (double)RABS(tmp_x);
            a[5] += (double)RABS(tmp_y);
            a[6] += (double)v0;
            a[7] += (double)v1;
            a[8] += (double)v2;
            a[9] += (double)v3;
            if (macc) {
              double* t = tmg + AW;
              const double ax = fabs((double)tmp_x), ay = fabs((double)tmp_y);
              t[0] += ax;
              t[1] += ay;
              t[2] += ax;
              t[3] += ay;
              t[4] += ax;
              t[5] += ay;
              t[6] += fabs((double)v0);
              t[7] += fabs((double)v1);
              t[8] += fabs((double)v2);
              t[9] += fabs((double)v3);
            }
          }
        }
      }
      for (uint32_t j = 0; j < end - start; ++j) {
        const double* ta = tb + (size_t)j * tw;
        const uint32_t g = point_list[start + j];
        for (int q = 0; q < AW; ++q)
          if (ta[q] != 0.0) {
#pragma omp atomic
            acc[(size_t)g * AW + q] += ta[q];
          }
        if (macc)
          for (int q = 0; q < 2 * AW; ++q)
            if (ta[AW + q] != 0.0) {
#pragma omp atomic
              macc[(size_t)g * AW * 2 + q] += ta[AW + q];
            }
      }
    }
    free(rec_g);
    free(rec_j);
    free(rec);
    free(tb);
  }
  for (uint32_t g = 0; g < gn; ++g) {
    const double* a = acc + (size_t)g * AW;
    dmeans2d[2 * (size_t)g + 0] += (real)a[0];
    dmeans2d[2 * (size_t)g + 1] += (real)a[1];
    for (int q = 0; q < 4; ++q) dvsp[4 * (size_t)g + q] += (real)a[2 + q];
    for (int q = 0; q < 4; ++q) dconic[4 * (size_t)g + q] += (real)a[6 + q];
    for (int c = 0; c < C; ++c) dcolors[(size_t)g * NC + c] += (real)a[10 + c];
  }
  if (macc) {
    const int64_t rows = (int64_t)gn < mag_rows ? (int64_t)gn : mag_rows;
    for (int64_t g = 0; g < rows; ++g)
      for (int q = 0; q < 2 * AW; ++q) mag[(size_t)g * AW * 2 + q] += macc[(size_t)g * AW * 2 + q];
  }
  free(acc);
  free(macc);
}

void orc_rasterize_bwd(const orc_rparams* rp, const uint32_t* ranges, const uint32_t* point_list,
                       const real* means2d, const real* colors, const real* conic_opacity,
                       const real* background, const real* final_t, const uint32_t* n_contrib,
                       const real* dL_dout, real* dmeans2d, real* dcolors, real* dconic,
                       real* dvsp) {
  orc_rasterize_bwd_mag(rp, ranges, point_list, means2d, colors, conic_opacity, background,
                        final_t, n_contrib, dL_dout, dmeans2d, dcolors, dconic, dvsp, NULL, 0);
}

/* ------------------------------------------------------------------------ */
/* Preprocess backward (fastgs_preprocess_backward.metal:60-430).            */
/* Gradient outputs zero-filled by the caller (fastgs_preprocess_backward.cpp */
/* :91-94); rows with radii <= 0 stay zero.                                   */
/* ------------------------------------------------------------------------ */
void orc_preprocess_bwd(const orc_params* prm, const real* means3d, const real* scales,
                        const real* quats, const real* viewmat, const real* projmat,
                        const real* cam_pos, const real* sh, const real* cov3d_precomp,
                        const real* cov3d_fwd, const real* dL_dcov3d, const real* dL_drgb,
                        const real* dL_dxys, const real* dL_dconic_opacity,
                        const real* dL_dvsp_out, const int32_t* radii, const uint8_t* clamped,
                        real* dL_dmeans3d, real* dL_ddc, real* dL_dsh, real* dL_dcolors_precomp,
                        real* dL_dopacities, real* dL_dscales, real* dL_dquats,
                        real* dL_dvsp_in) {
  const int P = prm->P;
  /* 0.5*W/max(tan,1e-6) (fastgs_preprocess_backward.cpp:134-137), float */
  const real focal_x = (real)(0.5f * (float)prm->image_width / fmaxf(prm->tan_fovx, 1e-6f));
  const real focal_y = (real)(0.5f * (float)prm->image_height / fmaxf(prm->tan_fovy, 1e-6f));
#pragma omp parallel for schedule(static, 1024)
  for (int i = 0; i < P; ++i) {
    if (!(radii[i] > 0)) continue;
    const real* p = means3d + 3 * (size_t)i;
    real ph[4];
    xform44(projmat, p[0], p[1], p[2], ph);
    const real gx = dL_dxys[2 * (size_t)i + 0];
    const real gy = dL_dxys[2 * (size_t)i + 1];
    const real* cov_src = (prm->use_cov3d_precomp ? cov3d_precomp : cov3d_fwd) + 6 * (size_t)i;
    const real cg0 = dL_dconic_opacity[4 * (size_t)i + 0];
    const real cg1 = dL_dconic_opacity[4 * (size_t)i + 1];
    const real cg2 = dL_dconic_opacity[4 * (size_t)i + 2];
    real dcov_extra[6] = {0, 0, 0, 0, 0, 0};
    real dmean_cov[3];
    {
      orc_cov2d cv;
      cov2d_eval(viewmat, p, focal_x, focal_y, (real)prm->tan_fovx, (real)prm->tan_fovy, cov_src, &cv);
      const real x_grad_mul = (cv.txtz < -cv.limx || cv.txtz > cv.limx) ? (real)0 : (real)1;
      const real y_grad_mul = (cv.tytz < -cv.limy || cv.tytz > cv.limy) ? (real)0 : (real)1;
      /* Metal indexing: Tm[c][r], Vrk[c][r], W[c][r] = viewmat[4c + r] */
      real (*Tm)[3] = cv.T;
      const real Vrk[3][3] = {{cov_src[0], cov_src[1], cov_src[2]},
                              {cov_src[1], cov_src[3], cov_src[4]},
                              {cov_src[2], cov_src[4], cov_src[5]}};
      real Wm[3][3];
      for (int c = 0; c < 3; ++c)
        for (int r = 0; r < 3; ++r) Wm[c][r] = viewmat[4 * c + r];
      real a = cv.cov00 + (real)0.3;
      real b = cv.cov01;
      real c = cv.cov11 + (real)0.3;
      real denom = a * c - b * b;
      real denom2inv = (real)1 / ((denom * denom) + (real)1e-7);
      real dL_da = 0, dL_db = 0, dL_dc = 0;
      if (denom2inv != (real)0) {
        dL_da = denom2inv * (-c * c * cg0 + (real)2 * b * c * cg1 + (denom - a * c) * cg2);
        dL_dc = denom2inv * (-a * a * cg2 + (real)2 * a * b * cg1 + (denom - a * c) * cg0);
        dL_db = denom2inv * (real)2 * (b * c * cg0 - (denom + (real)2 * b * b) * cg1 + a * b * cg2);
        dcov_extra[0] = (Tm[0][0] * Tm[0][0] * dL_da + Tm[0][0] * Tm[1][0] * dL_db + Tm[1][0] * Tm[1][0] * dL_dc);
        dcov_extra[3] = (Tm[0][1] * Tm[0][1] * dL_da + Tm[0][1] * Tm[1][1] * dL_db + Tm[1][1] * Tm[1][1] * dL_dc);
        dcov_extra[5] = (Tm[0][2] * Tm[0][2] * dL_da + Tm[0][2] * Tm[1][2] * dL_db + Tm[1][2] * Tm[1][2] * dL_dc);
        dcov_extra[1] = (real)2 * Tm[0][0] * Tm[0][1] * dL_da + (Tm[0][0] * Tm[1][1] + Tm[0][1] * Tm[1][0]) * dL_db + (real)2 * Tm[1][0] * Tm[1][1] * dL_dc;
        dcov_extra[2] = (real)2 * Tm[0][0] * Tm[0][2] * dL_da + (Tm[0][0] * Tm[1][2] + Tm[0][2] * Tm[1][0]) * dL_db + (real)2 * Tm[1][0] * Tm[1][2] * dL_dc;
        dcov_extra[4] = (real)2 * Tm[0][2] * Tm[0][1] * dL_da + (Tm[0][1] * Tm[1][2] + Tm[0][2] * Tm[1][1]) * dL_db + (real)2 * Tm[1][1] * Tm[1][2] * dL_dc;
      }
      real dL_dT00 = (real)2 * (Tm[0][0] * Vrk[0][0] + Tm[0][1] * Vrk[0][1] + Tm[0][2] * Vrk[0][2]) * dL_da +
                     (Tm[1][0] * Vrk[0][0] + Tm[1][1] * Vrk[0][1] + Tm[1][2] * Vrk[0][2]) * dL_db;
      real dL_dT01 = (real)2 * (Tm[0][0] * Vrk[1][0] + Tm[0][1] * Vrk[1][1] + Tm[0][2] * Vrk[1][2]) * dL_da +
                     (Tm[1][0] * Vrk[1][0] + Tm[1][1] * Vrk[1][1] + Tm[1][2] * Vrk[1][2]) * dL_db;
      real dL_dT02 = (real)2 * (Tm[0][0] * Vrk[2][0] + Tm[0][1] * Vrk[2][1] + Tm[0][2] * Vrk[2][2]) * dL_da +
                     (Tm[1][0] * Vrk[2][0] + Tm[1][1] * Vrk[2][1] + Tm[1][2] * Vrk[2][2]) * dL_db;
      real dL_dT10 = (real)2 * (Tm[1][0] * Vrk[0][0] + Tm[1][1] * Vrk[0][1] + Tm[1][2] * Vrk[0][2]) * dL_dc +
                     (Tm[0][0] * Vrk[0][0] + Tm[0][1] * Vrk[0][1] + Tm[0][2] * Vrk[0][2]) * dL_db;
      real dL_dT11 = (real)2 * (Tm[1][0] * Vrk[1][0] + Tm[1][1] * Vrk[1][1] + Tm[1][2] * Vrk[1][2]) * dL_dc +
                     (Tm[0][0] * Vrk[1][0] + Tm[0][1] * Vrk[1][1] + Tm[0][2] * Vrk[1][2]) * dL_db;
      real dL_dT12 = (real)2 * (Tm[1][0] * Vrk[2][0] + Tm[1][1] * Vrk[2][1] + Tm[1][2] * Vrk[2][2]) * dL_dc +
                     (Tm[0][0] * Vrk[2][0] + Tm[0][1] * Vrk[2][1] + Tm[0][2] * Vrk[2][2]) * dL_db;
      real dL_dJ00 = Wm[0][0] * dL_dT00 + Wm[0][1] * dL_dT01 + Wm[0][2] * dL_dT02;
      real dL_dJ02 = Wm[2][0] * dL_dT00 + Wm[2][1] * dL_dT01 + Wm[2][2] * dL_dT02;
      real dL_dJ11 = Wm[1][0] * dL_dT10 + Wm[1][1] * dL_dT11 + Wm[1][2] * dL_dT12;
      real dL_dJ12 = Wm[2][0] * dL_dT10 + Wm[2][1] * dL_dT11 + Wm[2][2] * dL_dT12;
      const real tz = (real)1 / cv.t[2];
      const real tz2 = tz * tz;
      const real tz3 = tz2 * tz;
      const real dL_dtx = x_grad_mul * -focal_x * tz2 * dL_dJ02;
      const real dL_dty = y_grad_mul * -focal_y * tz2 * dL_dJ12;
      const real dL_dtz = -focal_x * tz2 * dL_dJ00 - focal_y * tz2 * dL_dJ11 +
                          ((real)2 * focal_x * cv.t[0]) * tz3 * dL_dJ02 +
                          ((real)2 * focal_y * cv.t[1]) * tz3 * dL_dJ12;
      /* transform_vec4x3_transpose (:47-52) */
      dmean_cov[0] = viewmat[0] * dL_dtx + viewmat[1] * dL_dty + viewmat[2] * dL_dtz;
      dmean_cov[1] = viewmat[4] * dL_dtx + viewmat[5] * dL_dty + viewmat[6] * dL_dtz;
      dmean_cov[2] = viewmat[8] * dL_dtx + viewmat[9] * dL_dty + viewmat[10] * dL_dtz;
    }
    /* projective mean gradient (:187-204) */
    const real m_w = (real)1 / (ph[3] + (real)1.0e-7);
    const real mul1 = (projmat[0] * p[0] + projmat[4] * p[1] + projmat[8] * p[2] + projmat[12]) * m_w * m_w;
    const real mul2 = (projmat[1] * p[0] + projmat[5] * p[1] + projmat[9] * p[2] + projmat[13]) * m_w * m_w;
    const real dmx = (projmat[0] * m_w - projmat[3] * mul1) * gx + (projmat[1] * m_w - projmat[3] * mul2) * gy;
    const real dmy = (projmat[4] * m_w - projmat[7] * mul1) * gx + (projmat[5] * m_w - projmat[7] * mul2) * gy;
    const real dmz = (projmat[8] * m_w - projmat[11] * mul1) * gx + (projmat[9] * m_w - projmat[11] * mul2) * gy;
    real dm[3] = {dmx + dmean_cov[0], dmy + dmean_cov[1], dmz + dmean_cov[2]};
    dL_dopacities[i] = dL_dconic_opacity[4 * (size_t)i + 3];
    if (prm->use_colors_precomp) {
      for (int c = 0; c < 3; ++c) dL_dcolors_precomp[3 * (size_t)i + c] = dL_drgb[3 * (size_t)i + c];
    } else {
      real dRGB[3];
      for (int c = 0; c < 3; ++c) dRGB[c] = clamped[3 * (size_t)i + c] ? (real)0 : dL_drgb[3 * (size_t)i + c];
      for (int c = 0; c < 3; ++c) dL_ddc[3 * (size_t)i + c] = SH_C0 * dRGB[c];
      for (int c = 0; c < 3; ++c) dL_dcolors_precomp[3 * (size_t)i + c] = 0;
      const int msh = prm->max_sh_coeffs;
      if (prm->degree > 0 && msh >= 3) {
        real dir_orig[3] = {p[0] - cam_pos[0], p[1] - cam_pos[1], p[2] - cam_pos[2]};
        real len = RSQRT(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]);
        real x = dir_orig[0] / len, y = dir_orig[1] / len, z = dir_orig[2] / len;
        const real* s = sh + (size_t)i * (size_t)msh * 3;
        real* ds = dL_dsh + (size_t)i * (size_t)msh * 3;
        real dRGBdx[3], dRGBdy[3], dRGBdz[3];
        for (int c = 0; c < 3; ++c) {
          ds[0 * 3 + c] = (-SH_C1 * y) * dRGB[c];
          ds[1 * 3 + c] = (SH_C1 * z) * dRGB[c];
          ds[2 * 3 + c] = (-SH_C1 * x) * dRGB[c];
          dRGBdx[c] = -SH_C1 * s[2 * 3 + c];
          dRGBdy[c] = -SH_C1 * s[0 * 3 + c];
          dRGBdz[c] = SH_C1 * s[1 * 3 + c];
        }
        if (prm->degree > 1 && msh >= 8) {
          real xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
          for (int c = 0; c < 3; ++c) {
            ds[3 * 3 + c] = (SH_C2[0] * xy) * dRGB[c];
            ds[4 * 3 + c] = (SH_C2[1] * yz) * dRGB[c];
            ds[5 * 3 + c] = (SH_C2[2] * ((real)2 * zz - xx - yy)) * dRGB[c];
            ds[6 * 3 + c] = (SH_C2[3] * xz) * dRGB[c];
            ds[7 * 3 + c] = (SH_C2[4] * (xx - yy)) * dRGB[c];
            const real s3 = s[3 * 3 + c], s4 = s[4 * 3 + c], s5 = s[5 * 3 + c], s6 = s[6 * 3 + c], s7 = s[7 * 3 + c];
            dRGBdx[c] += SH_C2[0] * y * s3 + SH_C2[2] * (real)2 * -x * s5 + SH_C2[3] * z * s6 + SH_C2[4] * (real)2 * x * s7;
            dRGBdy[c] += SH_C2[0] * x * s3 + SH_C2[1] * z * s4 + SH_C2[2] * (real)2 * -y * s5 + SH_C2[4] * (real)2 * -y * s7;
            dRGBdz[c] += SH_C2[1] * y * s4 + SH_C2[2] * (real)4 * z * s5 + SH_C2[3] * x * s6;
          }
          if (prm->degree > 2 && msh >= 15) {
            for (int c = 0; c < 3; ++c) {
              ds[8 * 3 + c] = (SH_C3[0] * y * ((real)3 * xx - yy)) * dRGB[c];
              ds[9 * 3 + c] = (SH_C3[1] * xy * z) * dRGB[c];
              ds[10 * 3 + c] = (SH_C3[2] * y * ((real)4 * zz - xx - yy)) * dRGB[c];
              ds[11 * 3 + c] = (SH_C3[3] * z * ((real)2 * zz - (real)3 * xx - (real)3 * yy)) * dRGB[c];
              ds[12 * 3 + c] = (SH_C3[4] * x * ((real)4 * zz - xx - yy)) * dRGB[c];
              ds[13 * 3 + c] = (SH_C3[5] * z * (xx - yy)) * dRGB[c];
              ds[14 * 3 + c] = (SH_C3[6] * x * (xx - (real)3 * yy)) * dRGB[c];
              const real s8 = s[8 * 3 + c], s9 = s[9 * 3 + c], s10 = s[10 * 3 + c], s11 = s[11 * 3 + c];
              const real s12 = s[12 * 3 + c], s13 = s[13 * 3 + c], s14 = s[14 * 3 + c];
              dRGBdx[c] += (SH_C3[0] * s8 * (real)6 * xy + SH_C3[1] * s9 * yz + SH_C3[2] * s10 * (real)-2 * xy +
                            SH_C3[3] * s11 * (real)-6 * xz + SH_C3[4] * s12 * ((real)-3 * xx + (real)4 * zz - yy) +
                            SH_C3[5] * s13 * (real)2 * xz + SH_C3[6] * s14 * (real)3 * (xx - yy));
              dRGBdy[c] += (SH_C3[0] * s8 * (real)3 * (xx - yy) + SH_C3[1] * s9 * xz +
                            SH_C3[2] * s10 * ((real)-3 * yy + (real)4 * zz - xx) + SH_C3[3] * s11 * (real)-6 * yz +
                            SH_C3[4] * s12 * (real)-2 * xy + SH_C3[5] * s13 * (real)-2 * yz +
                            SH_C3[6] * s14 * (real)-6 * xy);
              dRGBdz[c] += (SH_C3[1] * s9 * xy + SH_C3[2] * s10 * (real)8 * yz +
                            SH_C3[3] * s11 * (real)3 * ((real)2 * zz - xx - yy) + SH_C3[4] * s12 * (real)8 * xz +
                            SH_C3[5] * s13 * (xx - yy));
            }
          }
        }
        real ddir[3] = {dRGBdx[0] * dRGB[0] + dRGBdx[1] * dRGB[1] + dRGBdx[2] * dRGB[2],
                        dRGBdy[0] * dRGB[0] + dRGBdy[1] * dRGB[1] + dRGBdy[2] * dRGB[2],
                        dRGBdz[0] * dRGB[0] + dRGBdz[1] * dRGB[1] + dRGBdz[2] * dRGB[2]};
        /* dnormvdv (:54-58) */
        real l = RMAX(RSQRT(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]), (real)1e-6);
        real nv[3] = {dir_orig[0] / l, dir_orig[1] / l, dir_orig[2] / l};
        real nd = nv[0] * ddir[0] + nv[1] * ddir[1] + nv[2] * ddir[2];
        for (int k = 0; k < 3; ++k) dm[k] += (ddir[k] - nv[k] * nd) / l;
      }
    }
    for (int k = 0; k < 3; ++k) dL_dmeans3d[3 * (size_t)i + k] = dm[k];
    if (!prm->use_cov3d_precomp) {
      const real* sc = scales + 3 * (size_t)i;
      const real* q = quats + 4 * (size_t)i;
      const real r = q[0], x = q[1], y = q[2], z = q[3];
      real R[3][3]; /* R[col][row] */
      R[0][0] = (real)1 - (real)2 * (y * y + z * z);
      R[0][1] = (real)2 * (x * y - r * z);
      R[0][2] = (real)2 * (x * z + r * y);
      R[1][0] = (real)2 * (x * y + r * z);
      R[1][1] = (real)1 - (real)2 * (x * x + z * z);
      R[1][2] = (real)2 * (y * z - r * x);
      R[2][0] = (real)2 * (x * z - r * y);
      R[2][1] = (real)2 * (y * z + r * x);
      R[2][2] = (real)1 - (real)2 * (x * x + y * y);
      real s[3] = {(real)prm->scale_modifier * sc[0], (real)prm->scale_modifier * sc[1],
                   (real)prm->scale_modifier * sc[2]};
      real M[3][3]; /* M[col][row] = s[row] * R[col][row] */
      for (int c = 0; c < 3; ++c)
        for (int rr = 0; rr < 3; ++rr) M[c][rr] = s[rr] * R[c][rr];
      real cc[6];
      for (int k = 0; k < 6; ++k) cc[k] = dL_dcov3d[6 * (size_t)i + k] + dcov_extra[k];
      /* dSigma[col][row] */
      real dS[3][3] = {{cc[0], (real)0.5 * cc[1], (real)0.5 * cc[2]},
                       {(real)0.5 * cc[1], cc[3], (real)0.5 * cc[4]},
                       {(real)0.5 * cc[2], (real)0.5 * cc[4], cc[5]}};
      /* dM = 2 M dSigma (math): dM(r,c) = sum_k 2 M(r,k) dS(k,c);
       * Metal dM[c][r]; M(r,k) = M[k][r]; dS(k,c) = dS[c][k]. */
      real dM[3][3];
      for (int c = 0; c < 3; ++c)
        for (int rr = 0; rr < 3; ++rr)
          dM[c][rr] = ((real)2 * M[0][rr]) * dS[c][0] + ((real)2 * M[1][rr]) * dS[c][1] +
                      ((real)2 * M[2][rr]) * dS[c][2];
      /* Rt[i][j] = R[j][i]; dMt[i][j] = dM[j][i] */
      real dMt[3][3];
      for (int a = 0; a < 3; ++a)
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] = dM[bb][a];
      real dsv[3];
      for (int a = 0; a < 3; ++a)
        dsv[a] = R[0][a] * dMt[a][0] + R[1][a] * dMt[a][1] + R[2][a] * dMt[a][2];
      for (int a = 0; a < 3; ++a) dL_dscales[3 * (size_t)i + a] = dsv[a];
      for (int a = 0; a < 3; ++a)
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] *= s[a];
      real dq0 = (real)2 * z * (dMt[0][1] - dMt[1][0]) + (real)2 * y * (dMt[2][0] - dMt[0][2]) + (real)2 * x * (dMt[1][2] - dMt[2][1]);
      real dq1 = (real)2 * y * (dMt[1][0] + dMt[0][1]) + (real)2 * z * (dMt[2][0] + dMt[0][2]) + (real)2 * r * (dMt[1][2] - dMt[2][1]) - (real)4 * x * (dMt[2][2] + dMt[1][1]);
      real dq2 = (real)2 * x * (dMt[1][0] + dMt[0][1]) + (real)2 * r * (dMt[2][0] - dMt[0][2]) + (real)2 * z * (dMt[1][2] + dMt[2][1]) - (real)4 * y * (dMt[2][2] + dMt[0][0]);
      real dq3 = (real)2 * r * (dMt[0][1] - dMt[1][0]) + (real)2 * x * (dMt[2][0] + dMt[0][2]) + (real)2 * y * (dMt[1][2] + dMt[2][1]) - (real)4 * z * (dMt[1][1] + dMt[0][0]);
      dL_dquats[4 * (size_t)i + 0] = dq0;
      dL_dquats[4 * (size_t)i + 1] = dq1;
      dL_dquats[4 * (size_t)i + 2] = dq2;
      dL_dquats[4 * (size_t)i + 3] = dq3;
    }
    for (int k = 0; k < 4; ++k) dL_dvsp_in[4 * (size_t)i + k] = dL_dvsp_out[4 * (size_t)i + k];
  }
}

/* Sums of term magnitudes through the preprocess backward (orc_preprocess_bwd,
 * fastgs_preprocess_backward.metal:60-430).  The backward is linear in its
 * cotangents; every output entry is a sum of products of forward-derived
 * scalars (T, the covariances, the conic's denominators, R, s, the SH
 * coefficients and direction, ...) with cotangents.  This evaluates the same
 * expression tree with each sum replaced by the sum of its summands'
 * magnitudes and each product by the product of magnitudes: the forward
 * scalars enter as |value|, the cotangents as the given magnitudes m_* (the
 * sums of their own terms' magnitudes, from orc_rasterize_bwd_mag).  The
 * result is, per entry, the sum of |term| over the fully expanded chain rule:
 * the scale of the rounding differences of two evaluations of these sums
 * that order or round them differently.  Outputs (double, accumulated with
 * +=): the magnitudes of dL_dmeans3d, dL_ddc, dL_dsh, dL_dcolors_precomp,
 * dL_dopacities, dL_dscales, dL_dquats, dL_dvsp_in. */
#define AB(x) fabs((double)(x))
void orc_preprocess_bwd_mag(const orc_params* prm, const real* means3d, const real* scales,
                            const real* quats, const real* viewmat, const real* projmat,
                            const real* cam_pos, const real* sh, const real* cov3d_precomp,
                            const real* cov3d_fwd, const double* m_cov3d, const double* m_rgb,
                            const double* m_xys, const double* m_conic, const double* m_vsp,
                            const int32_t* radii, const uint8_t* clamped, double* o_means3d,
                            double* o_dc, double* o_sh, double* o_colors_precomp,
                            double* o_opacities, double* o_scales, double* o_quats,
                            double* o_vsp) {
  const int P = prm->P;
  const real focal_x = (real)(0.5f * (float)prm->image_width / fmaxf(prm->tan_fovx, 1e-6f));
  const real focal_y = (real)(0.5f * (float)prm->image_height / fmaxf(prm->tan_fovy, 1e-6f));
#pragma omp parallel for schedule(static, 1024)
  for (int i = 0; i < P; ++i) {
    if (!(radii[i] > 0)) continue;
    const real* p = means3d + 3 * (size_t)i;
    real ph[4];
    xform44(projmat, p[0], p[1], p[2], ph);
    const double gx = m_xys[2 * (size_t)i + 0], gy = m_xys[2 * (size_t)i + 1];
    const real* cov_src = (prm->use_cov3d_precomp ? cov3d_precomp : cov3d_fwd) + 6 * (size_t)i;
    const double cg0 = m_conic[4 * (size_t)i + 0];
    const double cg1 = m_conic[4 * (size_t)i + 1];
    const double cg2 = m_conic[4 * (size_t)i + 2];
    double dce[6] = {0, 0, 0, 0, 0, 0};
    double dmc[3] = {0, 0, 0};
    {
      orc_cov2d cv;
      cov2d_eval(viewmat, p, focal_x, focal_y, (real)prm->tan_fovx, (real)prm->tan_fovy, cov_src,
                 &cv);
      const double xg = (cv.txtz < -cv.limx || cv.txtz > cv.limx) ? 0.0 : 1.0;
      const double yg = (cv.tytz < -cv.limy || cv.tytz > cv.limy) ? 0.0 : 1.0;
      double T[3][3], V[3][3], Wm[3][3];
      for (int c = 0; c < 3; ++c)
        for (int r = 0; r < 3; ++r) {
          T[c][r] = AB(cv.T[c][r]);
          Wm[c][r] = AB(viewmat[4 * c + r]);
        }
      const double vv[6] = {AB(cov_src[0]), AB(cov_src[1]), AB(cov_src[2]),
                            AB(cov_src[3]), AB(cov_src[4]), AB(cov_src[5])};
      V[0][0] = vv[0]; V[0][1] = vv[1]; V[0][2] = vv[2];
      V[1][0] = vv[1]; V[1][1] = vv[3]; V[1][2] = vv[4];
      V[2][0] = vv[2]; V[2][1] = vv[4]; V[2][2] = vv[5];
      const real a_ = cv.cov00 + (real)0.3, b_ = cv.cov01, c_ = cv.cov11 + (real)0.3;
      const real den_ = a_ * c_ - b_ * b_;
      const double a = AB(a_), b = AB(b_), c = AB(c_), den = AB(den_);
      const double d2i = AB((real)1 / ((den_ * den_) + (real)1e-7));
      double da = 0, db = 0, dc = 0;
      if (d2i != 0.0) {
        const double dm_ac = den + a * c; /* |denom| + |a c| */
        da = d2i * (c * c * cg0 + 2 * b * c * cg1 + dm_ac * cg2);
        dc = d2i * (a * a * cg2 + 2 * a * b * cg1 + dm_ac * cg0);
        db = d2i * 2 * (b * c * cg0 + (den + 2 * b * b) * cg1 + a * b * cg2);
        dce[0] = T[0][0] * T[0][0] * da + T[0][0] * T[1][0] * db + T[1][0] * T[1][0] * dc;
        dce[3] = T[0][1] * T[0][1] * da + T[0][1] * T[1][1] * db + T[1][1] * T[1][1] * dc;
        dce[5] = T[0][2] * T[0][2] * da + T[0][2] * T[1][2] * db + T[1][2] * T[1][2] * dc;
        dce[1] = 2 * T[0][0] * T[0][1] * da + (T[0][0] * T[1][1] + T[0][1] * T[1][0]) * db +
                 2 * T[1][0] * T[1][1] * dc;
        dce[2] = 2 * T[0][0] * T[0][2] * da + (T[0][0] * T[1][2] + T[0][2] * T[1][0]) * db +
                 2 * T[1][0] * T[1][2] * dc;
        dce[4] = 2 * T[0][2] * T[0][1] * da + (T[0][1] * T[1][2] + T[0][2] * T[1][1]) * db +
                 2 * T[1][1] * T[1][2] * dc;
      }
      double dT0[3], dT1[3];
      for (int k = 0; k < 3; ++k) {
        const double u0 = T[0][0] * V[k][0] + T[0][1] * V[k][1] + T[0][2] * V[k][2];
        const double u1 = T[1][0] * V[k][0] + T[1][1] * V[k][1] + T[1][2] * V[k][2];
        dT0[k] = 2 * u0 * da + u1 * db;
        dT1[k] = 2 * u1 * dc + u0 * db;
      }
      const double dJ00 = Wm[0][0] * dT0[0] + Wm[0][1] * dT0[1] + Wm[0][2] * dT0[2];
      const double dJ02 = Wm[2][0] * dT0[0] + Wm[2][1] * dT0[1] + Wm[2][2] * dT0[2];
      const double dJ11 = Wm[1][0] * dT1[0] + Wm[1][1] * dT1[1] + Wm[1][2] * dT1[2];
      const double dJ12 = Wm[2][0] * dT1[0] + Wm[2][1] * dT1[1] + Wm[2][2] * dT1[2];
      const real tzr = (real)1 / cv.t[2];
      const double tz = AB(tzr), tz2 = AB(tzr * tzr), tz3 = AB(tzr * tzr * tzr);
      const double fx = AB(focal_x), fy = AB(focal_y);
      const double dtx = xg * fx * tz2 * dJ02;
      const double dty = yg * fy * tz2 * dJ12;
      const double dtz = fx * tz2 * dJ00 + fy * tz2 * dJ11 + (2 * fx * AB(cv.t[0])) * tz3 * dJ02 +
                         (2 * fy * AB(cv.t[1])) * tz3 * dJ12;
      (void)tz;
      for (int k = 0; k < 3; ++k)
        dmc[k] = AB(viewmat[4 * k]) * dtx + AB(viewmat[4 * k + 1]) * dty +
                 AB(viewmat[4 * k + 2]) * dtz;
    }
    const real m_w_ = (real)1 / (ph[3] + (real)1.0e-7);
    const double mw = AB(m_w_);
    const double mul1 = (AB(projmat[0] * p[0]) + AB(projmat[4] * p[1]) + AB(projmat[8] * p[2]) +
                         AB(projmat[12])) * mw * mw;
    const double mul2 = (AB(projmat[1] * p[0]) + AB(projmat[5] * p[1]) + AB(projmat[9] * p[2]) +
                         AB(projmat[13])) * mw * mw;
    double dm[3];
    for (int k = 0; k < 3; ++k)
      dm[k] = (AB(projmat[4 * k]) * mw + AB(projmat[4 * k + 3]) * mul1) * gx +
              (AB(projmat[4 * k + 1]) * mw + AB(projmat[4 * k + 3]) * mul2) * gy + dmc[k];
    o_opacities[i] += m_conic[4 * (size_t)i + 3];
    if (prm->use_colors_precomp) {
      for (int c = 0; c < 3; ++c) o_colors_precomp[3 * (size_t)i + c] += m_rgb[3 * (size_t)i + c];
    } else {
      double dRGB[3];
      for (int c = 0; c < 3; ++c) dRGB[c] = clamped[3 * (size_t)i + c] ? 0.0 : m_rgb[3 * (size_t)i + c];
      for (int c = 0; c < 3; ++c) o_dc[3 * (size_t)i + c] += AB(SH_C0) * dRGB[c];
      const int msh = prm->max_sh_coeffs;
      if (prm->degree > 0 && msh >= 3) {
        real dir_orig[3] = {p[0] - cam_pos[0], p[1] - cam_pos[1], p[2] - cam_pos[2]};
        real len = RSQRT(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]);
        const double x = AB(dir_orig[0] / len), y = AB(dir_orig[1] / len), z = AB(dir_orig[2] / len);
        const real* sr = sh + (size_t)i * (size_t)msh * 3;
        double* ds = o_sh + (size_t)i * (size_t)msh * 3;
        double ex[3], ey[3], ez[3];
        const double C1 = AB(SH_C1);
        for (int c = 0; c < 3; ++c) {
          ds[0 * 3 + c] += C1 * y * dRGB[c];
          ds[1 * 3 + c] += C1 * z * dRGB[c];
          ds[2 * 3 + c] += C1 * x * dRGB[c];
          ex[c] = C1 * AB(sr[2 * 3 + c]);
          ey[c] = C1 * AB(sr[0 * 3 + c]);
          ez[c] = C1 * AB(sr[1 * 3 + c]);
        }
        if (prm->degree > 1 && msh >= 8) {
          const double xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
          double C2[5], C3[7];
          for (int k = 0; k < 5; ++k) C2[k] = AB(SH_C2[k]);
          for (int k = 0; k < 7; ++k) C3[k] = AB(SH_C3[k]);
          for (int c = 0; c < 3; ++c) {
            ds[3 * 3 + c] += C2[0] * xy * dRGB[c];
            ds[4 * 3 + c] += C2[1] * yz * dRGB[c];
            ds[5 * 3 + c] += C2[2] * (2 * zz + xx + yy) * dRGB[c];
            ds[6 * 3 + c] += C2[3] * xz * dRGB[c];
            ds[7 * 3 + c] += C2[4] * (xx + yy) * dRGB[c];
            const double s3 = AB(sr[3 * 3 + c]), s4 = AB(sr[4 * 3 + c]), s5 = AB(sr[5 * 3 + c]),
                         s6 = AB(sr[6 * 3 + c]), s7 = AB(sr[7 * 3 + c]);
            ex[c] += C2[0] * y * s3 + C2[2] * 2 * x * s5 + C2[3] * z * s6 + C2[4] * 2 * x * s7;
            ey[c] += C2[0] * x * s3 + C2[1] * z * s4 + C2[2] * 2 * y * s5 + C2[4] * 2 * y * s7;
            ez[c] += C2[1] * y * s4 + C2[2] * 4 * z * s5 + C2[3] * x * s6;
          }
          if (prm->degree > 2 && msh >= 15) {
            for (int c = 0; c < 3; ++c) {
              ds[8 * 3 + c] += C3[0] * y * (3 * xx + yy) * dRGB[c];
              ds[9 * 3 + c] += C3[1] * xy * z * dRGB[c];
              ds[10 * 3 + c] += C3[2] * y * (4 * zz + xx + yy) * dRGB[c];
              ds[11 * 3 + c] += C3[3] * z * (2 * zz + 3 * xx + 3 * yy) * dRGB[c];
              ds[12 * 3 + c] += C3[4] * x * (4 * zz + xx + yy) * dRGB[c];
              ds[13 * 3 + c] += C3[5] * z * (xx + yy) * dRGB[c];
              ds[14 * 3 + c] += C3[6] * x * (xx + 3 * yy) * dRGB[c];
              const double s8 = AB(sr[8 * 3 + c]), s9 = AB(sr[9 * 3 + c]), s10 = AB(sr[10 * 3 + c]),
                           s11 = AB(sr[11 * 3 + c]), s12 = AB(sr[12 * 3 + c]),
                           s13 = AB(sr[13 * 3 + c]), s14 = AB(sr[14 * 3 + c]);
              ex[c] += C3[0] * s8 * 6 * xy + C3[1] * s9 * yz + C3[2] * s10 * 2 * xy +
                       C3[3] * s11 * 6 * xz + C3[4] * s12 * (3 * xx + 4 * zz + yy) +
                       C3[5] * s13 * 2 * xz + C3[6] * s14 * 3 * (xx + yy);
              ey[c] += C3[0] * s8 * 3 * (xx + yy) + C3[1] * s9 * xz +
                       C3[2] * s10 * (3 * yy + 4 * zz + xx) + C3[3] * s11 * 6 * yz +
                       C3[4] * s12 * 2 * xy + C3[5] * s13 * 2 * yz + C3[6] * s14 * 6 * xy;
              ez[c] += C3[1] * s9 * xy + C3[2] * s10 * 8 * yz +
                       C3[3] * s11 * 3 * (2 * zz + xx + yy) + C3[4] * s12 * 8 * xz +
                       C3[5] * s13 * (xx + yy);
            }
          }
        }
        const double dd[3] = {ex[0] * dRGB[0] + ex[1] * dRGB[1] + ex[2] * dRGB[2],
                              ey[0] * dRGB[0] + ey[1] * dRGB[1] + ey[2] * dRGB[2],
                              ez[0] * dRGB[0] + ez[1] * dRGB[1] + ez[2] * dRGB[2]};
        real l_ = RMAX(RSQRT(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]), (real)1e-6);
        const double l = AB(l_);
        const double nv[3] = {AB(dir_orig[0] / l_), AB(dir_orig[1] / l_), AB(dir_orig[2] / l_)};
        const double nd = nv[0] * dd[0] + nv[1] * dd[1] + nv[2] * dd[2];
        for (int k = 0; k < 3; ++k) dm[k] += (dd[k] + nv[k] * nd) / l;
      }
    }
    for (int k = 0; k < 3; ++k) o_means3d[3 * (size_t)i + k] += dm[k];
    if (!prm->use_cov3d_precomp) {
      const real* sc = scales + 3 * (size_t)i;
      const real* q = quats + 4 * (size_t)i;
      const real r_ = q[0], x_ = q[1], y_ = q[2], z_ = q[3];
      real R_[3][3];
      R_[0][0] = (real)1 - (real)2 * (y_ * y_ + z_ * z_);
      R_[0][1] = (real)2 * (x_ * y_ - r_ * z_);
      R_[0][2] = (real)2 * (x_ * z_ + r_ * y_);
      R_[1][0] = (real)2 * (x_ * y_ + r_ * z_);
      R_[1][1] = (real)1 - (real)2 * (x_ * x_ + z_ * z_);
      R_[1][2] = (real)2 * (y_ * z_ - r_ * x_);
      R_[2][0] = (real)2 * (x_ * z_ - r_ * y_);
      R_[2][1] = (real)2 * (y_ * z_ + r_ * x_);
      R_[2][2] = (real)1 - (real)2 * (x_ * x_ + y_ * y_);
      double R[3][3], M[3][3];
      const double s3[3] = {AB((real)prm->scale_modifier * sc[0]), AB((real)prm->scale_modifier * sc[1]),
                            AB((real)prm->scale_modifier * sc[2])};
      for (int c = 0; c < 3; ++c)
        for (int rr = 0; rr < 3; ++rr) {
          R[c][rr] = AB(R_[c][rr]);
          M[c][rr] = AB((real)s3[rr] * R_[c][rr]);
        }
      double cc[6];
      for (int k = 0; k < 6; ++k) cc[k] = (m_cov3d ? m_cov3d[6 * (size_t)i + k] : 0.0) + dce[k];
      const double dS[3][3] = {{cc[0], 0.5 * cc[1], 0.5 * cc[2]},
                               {0.5 * cc[1], cc[3], 0.5 * cc[4]},
                               {0.5 * cc[2], 0.5 * cc[4], cc[5]}};
      double dM[3][3], dMt[3][3];
      for (int c = 0; c < 3; ++c)
        for (int rr = 0; rr < 3; ++rr)
          dM[c][rr] = 2 * M[0][rr] * dS[c][0] + 2 * M[1][rr] * dS[c][1] + 2 * M[2][rr] * dS[c][2];
      for (int a = 0; a < 3; ++a)
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] = dM[bb][a];
      for (int a = 0; a < 3; ++a)
        o_scales[3 * (size_t)i + a] += R[0][a] * dMt[a][0] + R[1][a] * dMt[a][1] + R[2][a] * dMt[a][2];
      for (int a = 0; a < 3; ++a)
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] *= s3[a];
      const double r = AB(r_), x = AB(x_), y = AB(y_), z = AB(z_);
      double* oq = o_quats + 4 * (size_t)i;
      oq[0] += 2 * z * (dMt[0][1] + dMt[1][0]) + 2 * y * (dMt[2][0] + dMt[0][2]) + 2 * x * (dMt[1][2] + dMt[2][1]);
      oq[1] += 2 * y * (dMt[1][0] + dMt[0][1]) + 2 * z * (dMt[2][0] + dMt[0][2]) + 2 * r * (dMt[1][2] + dMt[2][1]) + 4 * x * (dMt[2][2] + dMt[1][1]);
      oq[2] += 2 * x * (dMt[1][0] + dMt[0][1]) + 2 * r * (dMt[2][0] + dMt[0][2]) + 2 * z * (dMt[1][2] + dMt[2][1]) + 4 * y * (dMt[2][2] + dMt[0][0]);
      oq[3] += 2 * r * (dMt[0][1] + dMt[1][0]) + 2 * x * (dMt[2][0] + dMt[0][2]) + 2 * y * (dMt[1][2] + dMt[2][1]) + 4 * z * (dMt[1][1] + dMt[0][0]);
    }
    for (int k = 0; k < 4; ++k) o_vsp[4 * (size_t)i + k] += m_vsp[4 * (size_t)i + k];
  }
}
#undef AB

int orc_sizeof_real(void) { return (int)sizeof(real); }

/* Threads the OpenMP loops use (1 without OpenMP). */
void orc_set_num_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
