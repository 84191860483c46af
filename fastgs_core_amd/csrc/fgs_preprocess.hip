// fgs_preprocess.hip -- per-Gaussian projection, covariance, SH colour and
// exact tile-footprint count (forward), and the chain rule back to the 3D
// parameters (backward).  One thread per Gaussian, 128-thread workgroups;
// every output row is written (zeros for culled rows), so no separate clear
// pass is needed.
//
// Forward restates fastgs_preprocess.metal:384-484, backward
// fastgs_preprocess_backward.metal:60-430.  Matrices arrive as 16 floats,
// column-major; the Metal float3x3 constructor fills columns, so X[c][r]
// below is column c, row r of the Metal matrix.
#include <cstdio>

#include "fgs_common.hpp"

namespace fgs {

__constant__ float kSH_C0 = 0.28209479177387814f;
__constant__ float kSH_C1 = 0.4886025119029199f;
__constant__ float kSH_C2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                                -1.0925484305920792f, 0.5462742152960396f};
__constant__ float kSH_C3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                                0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                                -0.5900435899266435f};

struct Mat16 {
  float m[16];
};

__device__ __forceinline__ Mat16 load_mat(const float* __restrict__ p) {
  Mat16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r.m[i] = p[i];
  return r;
}

// cov3d from scale and rotation (fastgs_preprocess.metal:207-231).
__device__ __forceinline__ void cov3d_from_sr(float sx, float sy, float sz, float mod, float4 q,
                                              float out[6]) {
  const float r = q.x, x = q.y, y = q.z, z = q.w;
  float R[3][3];
  R[0][0] = 1.0f - 2.0f * (y * y + z * z);
  R[0][1] = 2.0f * (x * y - r * z);
  R[0][2] = 2.0f * (x * z + r * y);
  R[1][0] = 2.0f * (x * y + r * z);
  R[1][1] = 1.0f - 2.0f * (x * x + z * z);
  R[1][2] = 2.0f * (y * z - r * x);
  R[2][0] = 2.0f * (x * z - r * y);
  R[2][1] = 2.0f * (y * z + r * x);
  R[2][2] = 1.0f - 2.0f * (x * x + y * y);
  const float s[3] = {mod * sx, mod * sy, mod * sz};
  float M[3][3];
#pragma unroll
  for (int c = 0; c < 3; ++c)
#pragma unroll
    for (int rr = 0; rr < 3; ++rr) M[c][rr] = s[rr] * R[c][rr];
#define FGS_SIG(i, j) (M[j][0] * M[i][0] + M[j][1] * M[i][1] + M[j][2] * M[i][2])
  out[0] = FGS_SIG(0, 0);
  out[1] = FGS_SIG(0, 1);
  out[2] = FGS_SIG(0, 2);
  out[3] = FGS_SIG(1, 1);
  out[4] = FGS_SIG(1, 2);
  out[5] = FGS_SIG(2, 2);
#undef FGS_SIG
}

struct Cov2D {
  float t0, t1, t2;
  float txtz, tytz, limx, limy;
  float T[2][3];  // T[col][row]; third column is zero
  float cov00, cov01, cov11;
};

// EWA cov2D (fastgs_preprocess.metal:171-205).  W = R (columns of the view
// rotation), T = W*J, cov = T^T Vrk T; zero terms of the products omitted.
__device__ __forceinline__ void cov2d_eval(const Mat16& V, float mx, float my, float mz, float fx,
                                           float fy, float tan_fovx, float tan_fovy,
                                           const float c3[6], Cov2D& o) {
  float t0 = V.m[0] * mx + V.m[4] * my + V.m[8] * mz + V.m[12];
  float t1 = V.m[1] * mx + V.m[5] * my + V.m[9] * mz + V.m[13];
  const float t2 = V.m[2] * mx + V.m[6] * my + V.m[10] * mz + V.m[14];
  const float limx = 1.3f * tan_fovx;
  const float limy = 1.3f * tan_fovy;
  const float txtz = t0 / t2;
  const float tytz = t1 / t2;
  t0 = fminf(limx, fmaxf(-limx, txtz)) * t2;
  t1 = fminf(limy, fmaxf(-limy, tytz)) * t2;
  o.t0 = t0;
  o.t1 = t1;
  o.t2 = t2;
  o.txtz = txtz;
  o.tytz = tytz;
  o.limx = limx;
  o.limy = limy;
  const float j00 = fx / t2;
  const float j02 = -(fx * t0) / (t2 * t2);
  const float j11 = fy / t2;
  const float j12 = -(fy * t1) / (t2 * t2);
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    o.T[0][r] = V.m[0 + r] * j00 + V.m[8 + r] * j02;
    o.T[1][r] = V.m[4 + r] * j11 + V.m[8 + r] * j12;
  }
  const float Vr[3][3] = {{c3[0], c3[1], c3[2]}, {c3[1], c3[3], c3[4]}, {c3[2], c3[4], c3[5]}};
  float U[2][3];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int s = 0; s < 3; ++s)
      U[c][s] = o.T[c][0] * Vr[0][s] + o.T[c][1] * Vr[1][s] + o.T[c][2] * Vr[2][s];
  o.cov00 = U[0][0] * o.T[0][0] + U[0][1] * o.T[0][1] + U[0][2] * o.T[0][2];
  o.cov01 = U[1][0] * o.T[0][0] + U[1][1] * o.T[0][1] + U[1][2] * o.T[0][2];
  o.cov11 = U[1][0] * o.T[1][0] + U[1][1] * o.T[1][1] + U[1][2] * o.T[1][2];
}

// Block-cooperative copy of the SH rows of Gaussians [b0, b0+kB) into LDS
// (kB threads per block, a multiple of 64).  The block's rows are one
// contiguous range of kB*kRow floats that starts on a 16-byte boundary
// (b0*kRow*4 is a multiple of 256 and the base is 16-byte aligned), so it
// moves as 16-byte loads, all in flight before the first LDS write, then a
// tail of fewer than 4 floats.
// Threads per block of the preprocess kernels.  With the SH rows staged
// (kRow floats per Gaussian, 180 bytes at SH degree 3) the LDS bounds the
// Gaussians in flight per CU, and 128-thread blocks pack that bound more
// closely than 256-thread ones (the backward 121 -> 117 us at 1M Gaussians).
constexpr int kShBlock = 128;
// The colour half runs beside the depth sort: at 256 threads per block it
// holds fewer waves per CU and slows the sort less (forward at 1M Gaussians
// 3,455 Mpix/s with 128-thread blocks, 3,495 with 256).
constexpr int kColourBlock = 256;
// ... and walks the Gaussians with a grid of at most 256 workgroups, one per
// CU's worth, so it takes a smaller share of each CU from the sort (forward
// 3,646 -> 3,684 Mpix/s at 1M Gaussians; the step rate unchanged).
constexpr int kColourGrid = 256;

// radii (optional): the rows of Gaussians with radius 0 (which no caller
// reads) are not loaded; a 16-byte piece is loaded when either row it
// touches is needed, so the bytes skipped are those of culled rows alone.
template <int kRow, int kB = kShBlock>
__device__ __forceinline__ void stage_sh_rows(const float* __restrict__ sh, int P,
                                              float* __restrict__ s_sh,
                                              int blk = (int)blockIdx.x,
                                              const int32_t* __restrict__ radii = nullptr) {
  constexpr int kIters = (kRow + 3) / 4;  // ceil(kB*kRow/4 / kB)
  const int b0 = blk * kB;
  const int nb = (P - b0) < kB ? (P - b0) : kB;
  const int n = nb * kRow;
  const int n4 = n >> 2;
  const float* __restrict__ src = sh + (size_t)b0 * kRow;
  // n4 >= 2 (nb >= 1, kRow >= 9). Indexes past the range are clamped to its
  // last element (several lanes then copy the same value), so the copy is
  // branch-free and every load issues before the first wait.
  const int t = 4 * n4 + (int)threadIdx.x;  // tail float of this thread
  float4 v[kIters];
  float tv;
  if (radii) {  // uniform
    __shared__ uint32_t s_need[kB];
    if ((int)threadIdx.x < nb) s_need[threadIdx.x] = radii[b0 + (int)threadIdx.x] > 0 ? 1u : 0u;
    __syncthreads();
    const int tc = t < n ? t : n - 1;
    tv = s_need[tc / kRow] ? src[tc] : 0.0f;
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
      int e = (int)threadIdx.x + kB * j;
      e = e < n4 ? e : n4 - 1;
      const bool need = (s_need[(4 * e) / kRow] | s_need[(4 * e + 3) / kRow]) != 0u;
      v[j] = need ? reinterpret_cast<const float4*>(src)[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  } else {
    tv = src[t < n ? t : n - 1];
#pragma unroll
    for (int j = 0; j < kIters; ++j) {
      const int e = (int)threadIdx.x + kB * j;
      v[j] = reinterpret_cast<const float4*>(src)[e < n4 ? e : n4 - 1];
    }
  }
#pragma unroll
  for (int j = 0; j < kIters; ++j) {
    const int e = (int)threadIdx.x + kB * j;
    reinterpret_cast<float4*>(s_sh)[e < n4 ? e : n4 - 1] = v[j];
  }
  if (t < n) s_sh[t] = tv;
  __syncthreads();
}

// The reverse copy: LDS rows of the block's Gaussians to global memory.
template <int kRow, int kB = kShBlock>
__device__ __forceinline__ void store_sh_rows(const float* __restrict__ s_sh, int P,
                                              float* __restrict__ dst_base) {
  constexpr int kIters = (kRow + 3) / 4;
  const int b0 = (int)blockIdx.x * kB;
  const int nb = (P - b0) < kB ? (P - b0) : kB;
  const int n = nb * kRow;
  const int n4 = n >> 2;
  float* __restrict__ dst = dst_base + (size_t)b0 * kRow;
#pragma unroll
  for (int j = 0; j < kIters; ++j) {
    const int e = (int)threadIdx.x + kB * j;
    if (e < n4) reinterpret_cast<float4*>(dst)[e] = reinterpret_cast<const float4*>(s_sh)[e];
  }
  const int t = 4 * n4 + (int)threadIdx.x;
  if (t < n) dst[t] = s_sh[t];
}

// Scale, rotation and opacity of Gaussian I: the activated inputs, or the
// raw parameters activated here (the training-step form).
__device__ __forceinline__ float3 load_scale(const float* scales, const float* log_scales,
                                             size_t I) {
  if (log_scales)
    return make_float3(act_scale(log_scales[3 * I + 0]), act_scale(log_scales[3 * I + 1]),
                       act_scale(log_scales[3 * I + 2]));
  return make_float3(scales[3 * I + 0], scales[3 * I + 1], scales[3 * I + 2]);
}
__device__ __forceinline__ float4 load_rotation(const float* rotations, const float* raw, size_t I) {
  if (raw) return act_rotation(*reinterpret_cast<const float4*>(raw + 4 * I));
  return make_float4(rotations[4 * I + 0], rotations[4 * I + 1], rotations[4 * I + 2],
                     rotations[4 * I + 3]);
}
__device__ __forceinline__ float load_opacity(const float* opacities, const float* logits,
                                              size_t I) {
  return logits ? act_opacity(logits[I]) : opacities[I];
}

// Colour of Gaussian I (fastgs_preprocess.metal:117-169 through computeColorFromSH):
// colors_precomp, or the SH colour toward the camera centre clamped at 0
// (clamp[c] = the unclamped value was negative).  s: its SH rest
// coefficients (3 floats each), in LDS or global memory.
__device__ __forceinline__ void gaussian_colour(const fgs_preprocess_params& prm,
                                                const float* __restrict__ colors_precomp,
                                                const float* __restrict__ campos,
                                                const float* __restrict__ dc,
                                                const float* __restrict__ s, size_t I, float mx,
                                                float my, float mz, float col[3],
                                                uint8_t clamp[3]) {
  if (prm.use_colors_precomp) {
#pragma unroll
    for (int c = 0; c < 3; ++c) col[c] = colors_precomp[3 * I + c];
    return;
  }
  const float v0 = mx - campos[0], v1 = my - campos[1], v2 = mz - campos[2];
  const float len = __builtin_sqrtf(v0 * v0 + v1 * v1 + v2 * v2);
  const float x = v0 / len, y = v1 / len, z = v2 / len;
  const float* __restrict__ d = dc + 3 * I;
  const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    float res = kSH_C0 * d[c];
    if (prm.degree > 0) {
      res = res - kSH_C1 * y * s[0 * 3 + c] + kSH_C1 * z * s[1 * 3 + c] -
            kSH_C1 * x * s[2 * 3 + c];
      if (prm.degree > 1) {
        res += kSH_C2[0] * xy * s[3 * 3 + c] + kSH_C2[1] * yz * s[4 * 3 + c] +
               kSH_C2[2] * (2.0f * zz - xx - yy) * s[5 * 3 + c] +
               kSH_C2[3] * xz * s[6 * 3 + c] + kSH_C2[4] * (xx - yy) * s[7 * 3 + c];
        if (prm.degree > 2) {
          res += kSH_C3[0] * y * (3.0f * xx - yy) * s[8 * 3 + c] +
                 kSH_C3[1] * xy * z * s[9 * 3 + c] +
                 kSH_C3[2] * y * (4.0f * zz - xx - yy) * s[10 * 3 + c] +
                 kSH_C3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy) * s[11 * 3 + c] +
                 kSH_C3[4] * x * (4.0f * zz - xx - yy) * s[12 * 3 + c] +
                 kSH_C3[5] * z * (xx - yy) * s[13 * 3 + c] +
                 kSH_C3[6] * x * (xx - 3.0f * yy) * s[14 * 3 + c];
        }
      }
    }
    res += 0.5f;
    clamp[c] = res < 0.0f;
    col[c] = fmaxf(res, 0.0f);
  }
}

// Tile walks longer than this many lines are taken by the whole wavefront
// (tiles_walk_wave), so one wide Gaussian does not hold its 63 neighbours
// for its full walk (the kernel form with the SH rows staged; the other forms
// pack every walk, PackedWalk below).
constexpr int kWaveWalkLines = 16;

// The tile walks of a wavefront's Gaussians packed over its lanes.  Each lane
// stages its Gaussian's walk set-up (WalkSetup, the near-edge state of its
// first line, its record geometry) in LDS; the wavefront's lines, numbered
// Gaussian by Gaussian (an exclusive scan of the line counts), are then taken
// 64 at a time, one per lane.  A lane finds the Gaussian of its line as the
// largest starting line at or below it (each Gaussian's start written into a
// 64-slot table, then a prefix maximum over the lanes), intersects the line's
// far edge as walk_lines does, takes its near edge from the lane below (the
// previous line of the same Gaussian; the first line's from the set-up), and
// adds the span's tiles and record bits into its Gaussian's LDS counters
// (atomics).  The spans and their sums are those of walk_lines, so
// tiles_touched and the records are bit-identical; the lanes no longer wait
// for the longest walk of their wavefront (at 1M Gaussians / 1080p it ran 7.4
// lines against 2.9 on average, at 3M with 2 % large Gaussians 14.5 plus 3.7
// whole-wavefront walks against 6.1 rounds).
// 6.5 KB per wavefront, so that six wavefronts per SIMD fit in the LDS (the
// discriminant is recomputed from the conic; the integers are packed).
struct PackedWalk {
  enum { kPx, kPy, kCa, kCb, kCc, kT, kAm1, kAM1, kBmax0, kBmin1, kBmax1, kIl0, kIl1, kNF };
  // kOff: rmin0 - start (line u of position p is p + kOff); kR1: rmin1 | rmax1 << 16;
  // kGeo: is_y | fits << 1 | bx << 2 | by << 17 (the record's corner super-tile)
  enum { kOff, kR1, kGeo, kSlot, kCnt, kNI };
  float f[kNF][kWave];
  int i[kNI][kWave];
  unsigned long long rec[4][kWave];
};

__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int wave_incl_max(int v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(v, (unsigned)o, kWave);
    if (l >= o) v = v > t ? v : t;
  }
  return v;
}

// Called by every lane of the wavefront.  nl: the lane's line count (0 for
// no walk); ws, px, py, co, st: its walk set-up and record (st's geometry
// from rect()).  Returns the lane's tile count and ORs its record bits into st.
__device__ __forceinline__ uint32_t packed_walk(PackedWalk& S, int nl, const WalkSetup& ws,
                                                float px, float py, float4 co, EmitStRecord& st) {
  const int l = lane_id();
  const int incl = (int)wave_incl_scan((uint32_t)nl);
  const int start = incl - nl;
  const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
  if (total == 0) return 0u;  // uniform
  if (nl > 0) {
    // the near edge of the first line, as walk_lines starts it
    float il0 = ws.bmax1, il1 = ws.bmin1;
    if (ws.bmin0 <= (float)ws.rmin0 * 16.0f)
      ellipse_isect(co, ws.disc, ws.t, px, py, ws.is_y, (float)ws.rmin0 * 16.0f, il0, il1);
    S.f[PackedWalk::kPx][l] = px;
    S.f[PackedWalk::kPy][l] = py;
    S.f[PackedWalk::kCa][l] = co.x;
    S.f[PackedWalk::kCb][l] = co.y;
    S.f[PackedWalk::kCc][l] = co.z;
    S.f[PackedWalk::kT][l] = ws.t;
    S.f[PackedWalk::kAm1][l] = ws.am1;
    S.f[PackedWalk::kAM1][l] = ws.aM1;
    S.f[PackedWalk::kBmax0][l] = ws.bmax0;
    S.f[PackedWalk::kBmin1][l] = ws.bmin1;
    S.f[PackedWalk::kBmax1][l] = ws.bmax1;
    S.f[PackedWalk::kIl0][l] = il0;
    S.f[PackedWalk::kIl1][l] = il1;
    S.i[PackedWalk::kOff][l] = ws.rmin0 - start;
    S.i[PackedWalk::kR1][l] = (int)((uint32_t)ws.rmin1 | ((uint32_t)ws.rmax1 << 16));
    S.i[PackedWalk::kGeo][l] = (int)((ws.is_y ? 1u : 0u) | (st.fits ? 2u : 0u) |
                                     ((uint32_t)st.bx << 2) | ((uint32_t)st.by << 17));
  }
  S.i[PackedWalk::kCnt][l] = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) S.rec[k][l] = 0ull;
  int carry_owner = 0;
  float carry0 = 0.0f, carry1 = 0.0f;  // far edge of the previous round's last line
  for (int base = 0; base < total; base += kWave) {  // uniform
    S.i[PackedWalk::kSlot][l] = -1;
    wave_lds_order();
    if (nl > 0 && start >= base && start < base + kWave) S.i[PackedWalk::kSlot][start - base] = l;
    wave_lds_order();
    int v = S.i[PackedWalk::kSlot][l];
    // a Gaussian's walk starts at this line: the largest start at or below it
    // is that Gaussian's, so it is g below
    const bool first = v >= 0;
    if (l == 0 && v < 0) v = carry_owner;
    const int g = wave_incl_max(v);  // the Gaussian of line base + l
    carry_owner = __builtin_amdgcn_readlane(g, kWave - 1);
    const int p = base + l;
    const bool valid = p < total;
    WalkSetup w;
    w.am1 = S.f[PackedWalk::kAm1][g];
    w.aM1 = S.f[PackedWalk::kAM1][g];
    w.bmin1 = S.f[PackedWalk::kBmin1][g];
    w.bmax1 = S.f[PackedWalk::kBmax1][g];
    const uint32_t r1 = (uint32_t)S.i[PackedWalk::kR1][g];
    w.rmin1 = (int)(r1 & 0xFFFFu);
    w.rmax1 = (int)(r1 >> 16);
    const uint32_t geo = (uint32_t)S.i[PackedWalk::kGeo][g];
    const bool is_y = (geo & 1u) != 0u;
    const int u = p + S.i[PackedWalk::kOff][g];
    const float min_line = (float)u * 16.0f;
    const float max_line = min_line + 16.0f;
    const bool far = valid && max_line <= S.f[PackedWalk::kBmax0][g];
    float iM0 = 0.0f, iM1 = 0.0f;
    if (far) {
      const float4 gco = make_float4(S.f[PackedWalk::kCa][g], S.f[PackedWalk::kCb][g],
                                     S.f[PackedWalk::kCc][g], 0.0f);
      const float disc = gco.y * gco.y - gco.x * gco.z;  // as walk_setup forms it
      ellipse_isect(gco, disc, S.f[PackedWalk::kT][g], S.f[PackedWalk::kPx][g],
                    S.f[PackedWalk::kPy][g], is_y, max_line, iM0, iM1);
    }
    float il0 = __shfl_up(iM0, 1u, kWave), il1 = __shfl_up(iM1, 1u, kWave);
    if (l == 0) {
      il0 = carry0;
      il1 = carry1;
    }
    if (first) {
      il0 = S.f[PackedWalk::kIl0][g];
      il1 = S.f[PackedWalk::kIl1][g];
    }
    if (!far) {  // the last line: walk_lines keeps the previous far edge there
      iM0 = first ? w.bmax1 : il0;
      iM1 = first ? w.bmin1 : il1;
    }
    carry0 = __shfl(iM0, kWave - 1, kWave);
    carry1 = __shfl(iM1, kWave - 1, kWave);
    if (valid) {
      int vmin, vmax;
      walk_line_span(w, min_line, max_line, il0, il1, iM0, iM1, vmin, vmax);
      if (vmax > vmin) {
        atomicAdd(&S.i[PackedWalk::kCnt][g], vmax - vmin);
        uint64_t d[4];
        st_span_bits((geo & 2u) != 0u, st.set_ok, (int)((geo >> 2) & 0x7FFFu), (int)(geo >> 17),
                     st.sgx, u, vmin, vmax, is_y, d);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (d[k]) atomicOr(&S.rec[k][g], (unsigned long long)d[k]);
      }
    }
    wave_lds_order();  // the table is rewritten in the next round
  }
  if (nl == 0) return 0u;
  st.m0 |= S.rec[0][l];
  st.m1 |= S.rec[1][l];
  st.m2 |= S.rec[2][l];
  st.m3 |= S.rec[3][l];
  return (uint32_t)S.i[PackedWalk::kCnt][l];
}

// kRow = 0: SH rows are read from global memory where needed; kRow > 0: the
// rows (kRow = 3 * max_sh_coeffs floats) of the block are staged through LDS.
// kColour = false: the geometry only (rgb and clamped are not written;
// preprocess_colour_kernel writes them, possibly on another stream).
template <int kRow, bool kColour = true>
__global__ void __launch_bounds__(kShBlock)
preprocess_fwd_kernel(const fgs_preprocess_params prm, const fgs_preprocess_fwd_io io,
                      float focal_x, float focal_y) {
  extern __shared__ float4 s_sh4[];
  float* __restrict__ s_sh = reinterpret_cast<float*>(s_sh4);
  const int row = kRow > 0 ? kRow : prm.max_sh_coeffs * 3;
  if constexpr (kRow > 0) stage_sh_rows<kRow>(io.sh, prm.P, s_sh);
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  // every lane stays to the end: the wide Gaussians' walks below take the
  // whole wavefront
  const bool live = i < prm.P;
  const size_t I = live ? (size_t)i : 0;
  const float mx = io.means3d[3 * I + 0];
  const float my = io.means3d[3 * I + 1];
  const float mz = io.means3d[3 * I + 2];
  const Mat16 V = load_mat(io.viewmatrix);
  int32_t radius = 0;
  uint32_t cnt = 0;
  float xy0 = 0.f, xy1 = 0.f, depth = 0.f;
  float4 co = make_float4(0.f, 0.f, 0.f, 0.f);
  float col[3] = {0.f, 0.f, 0.f};
  uint8_t clamp[3] = {0, 0, 0};
  float4 vsp = make_float4(0.f, 0.f, 0.f, 0.f);
  float c3[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  EmitStRecord st(prm.grid_x, prm.grid_y);  // super-tile record, built by the tile walk
  // without SH rows in LDS every walk is packed over the wavefront
  // (packed_walk); otherwise a walk longer than kWaveWalkLines lines is left
  // to the whole wavefront.  Either way the lane keeps the walk's inputs and
  // takes the rest of the path as if the Gaussian touched a tile, undone
  // below if it touches none
  constexpr bool kPacked = kRow == 0;
  bool wide = false;
  int nl = 0;  // kPacked: the lines of the lane's walk
  WalkSetup wsv;
  wsv.empty = true;
  float wpx = 0.f, wpy = 0.f;
  float4 wco = make_float4(0.f, 0.f, 0.f, 0.f);
  // p_view (in_frustum, :96-115)
  const float pv0 = V.m[0] * mx + V.m[4] * my + V.m[8] * mz + V.m[12];
  const float pv1 = V.m[1] * mx + V.m[5] * my + V.m[9] * mz + V.m[13];
  const float pv2 = V.m[2] * mx + V.m[6] * my + V.m[10] * mz + V.m[14];
  if (live && pv2 > 0.2f) {
    const Mat16 Pm = load_mat(io.projmatrix);
    const float ph0 = Pm.m[0] * mx + Pm.m[4] * my + Pm.m[8] * mz + Pm.m[12];
    const float ph1 = Pm.m[1] * mx + Pm.m[5] * my + Pm.m[9] * mz + Pm.m[13];
    const float ph3 = Pm.m[3] * mx + Pm.m[7] * my + Pm.m[11] * mz + Pm.m[15];
    const float p_w = 1.0f / (ph3 + 1.0e-7f);
    const float pp0 = ph0 * p_w;
    const float pp1 = ph1 * p_w;
    if (prm.use_cov3d_precomp) {
#pragma unroll
      for (int k = 0; k < 6; ++k) c3[k] = io.cov3d_precomp[6 * I + k];
    } else {
      const float4 q = load_rotation(io.rotations, io.raw_rotations, I);
      const float3 sc = load_scale(io.scales, io.log_scales, I);
      cov3d_from_sr(sc.x, sc.y, sc.z, prm.scale_modifier, q, c3);
    }
    Cov2D cv;
    cov2d_eval(V, mx, my, mz, focal_x, focal_y, prm.tan_fovx, prm.tan_fovy, c3, cv);
    const float cx = cv.cov00 + 0.3f, cy = cv.cov01, cz = cv.cov11 + 0.3f;
    const float det = cx * cz - cy * cy;
    if (det != 0.0f) {
      const float det_inv = 1.0f / det;
      const float conic0 = cz * det_inv, conic1 = -cy * det_inv, conic2 = cx * det_inv;
      const float mid = 0.5f * (cx + cz);
      const float lambda1 = mid + __builtin_sqrtf(fmaxf(0.1f, mid * mid - det));
      const float lambda2 = mid - __builtin_sqrtf(fmaxf(0.1f, mid * mid - det));
      const float my_radius = ceilf(3.0f * __builtin_sqrtf(fmaxf(lambda1, lambda2)));
      const float px = ((pp0 + 1.0f) * (float)prm.image_width - 1.0f) * 0.5f;
      const float py = ((pp1 + 1.0f) * (float)prm.image_height - 1.0f) * 0.5f;
      const float4 con_o =
          make_float4(conic0, conic1, conic2, load_opacity(io.opacities, io.opacity_logits, I));
      const WalkSetup ws = walk_setup(px, py, con_o, prm.grid_x, prm.grid_y, prm.mult, st);
      uint32_t n = 0u;
      if (!ws.empty) {
        if (kPacked) {
          nl = ws.rmax0 - ws.rmin0;
          wsv = ws;
          wpx = px;
          wpy = py;
          wco = con_o;
          n = 1u;  // provisional
        } else if (ws.rmax0 - ws.rmin0 > kWaveWalkLines) {
          wide = true;
          wpx = px;
          wpy = py;
          wco = con_o;
          n = 1u;  // provisional
        } else {
          n = walk_lines(ws, px, py, con_o, ws.rmin0, ws.rmax0, st);
        }
      }
      if (n != 0u) {
        if constexpr (kColour)
          gaussian_colour(prm, io.colors_precomp, io.campos, io.dc,
                          kRow > 0 ? s_sh + threadIdx.x * kRow
                                   : (io.sh ? io.sh + I * (size_t)row : nullptr),
                          I, mx, my, mz, col, clamp);
        depth = pv2;
        radius = f2i(my_radius);
        xy0 = px;
        xy1 = py;
        co = con_o;
        cnt = n;
        vsp = make_float4(pv0, pv1, pv2, io.viewspace_in[4 * I + 3]);
      }
    }
  }
  if constexpr (kPacked) {
    __shared__ PackedWalk s_pw[kShBlock / kWave];
    const uint32_t nw = packed_walk(s_pw[threadIdx.x / kWave], nl, wsv, wpx, wpy, wco, st);
    if (nl > 0) {
      cnt = nw;
      if (nw == 0u) {  // it touches no tile: the outputs of a Gaussian that touches none
        radius = 0;
        depth = 0.f;
        xy0 = xy1 = 0.f;
        co = make_float4(0.f, 0.f, 0.f, 0.f);
        vsp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          col[c] = 0.f;
          clamp[c] = 0;
        }
      }
    }
  }
  // the wide Gaussians of this wavefront, one at a time by all its lanes
  for (uint64_t wm = __ballot(wide); wm != 0ull; wm &= wm - 1ull) {  // uniform
    const int src = __builtin_ctzll(wm);
    const float sx = __shfl(wpx, src, kWave), sy = __shfl(wpy, src, kWave);
    const float4 sco = make_float4(__shfl(wco.x, src, kWave), __shfl(wco.y, src, kWave),
                                   __shfl(wco.z, src, kWave), __shfl(wco.w, src, kWave));
    EmitStRecord sw(prm.grid_x, prm.grid_y);
    const uint32_t nw = tiles_walk_wave(sx, sy, sco, prm.grid_x, prm.grid_y, prm.mult, sw);
    sw.wave_or();
    if (lane_id() == src) {
      st = sw;
      cnt = nw;
      if (nw == 0u) {  // it touches no tile: the outputs of a Gaussian that touches none
        radius = 0;
        depth = 0.f;
        xy0 = xy1 = 0.f;
        co = make_float4(0.f, 0.f, 0.f, 0.f);
        vsp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          col[c] = 0.f;
          clamp[c] = 0;
        }
      }
    }
  }
  if (!live) return;
  io.radii[I] = radius;
  io.tiles_touched[I] = cnt;
  io.depths[I] = depth;
  *reinterpret_cast<float2*>(io.xys + 2 * I) = make_float2(xy0, xy1);
  *reinterpret_cast<float4*>(io.conic_opacity + 4 * I) = co;
  *reinterpret_cast<float4*>(io.viewspace_out + 4 * I) = vsp;
  float2* c3o = reinterpret_cast<float2*>(io.cov3d + 6 * I);
  c3o[0] = make_float2(c3[0], c3[1]);
  c3o[1] = make_float2(c3[2], c3[3]);
  c3o[2] = make_float2(c3[4], c3[5]);
  if constexpr (kColour) {
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      io.rgb[3 * I + c] = col[c];
      io.clamped[3 * I + c] = clamp[c];
    }
  }
  if (io.st_rec) {
    // a compact record is the 16 bytes alone; the others add their four
    // words in st_masks
    uint4 rec = make_uint4(0u, 0u, 0u, 0u);
    if (cnt != 0u && st.compact) {
      const uint64_t b = st.compact_board();
      rec = make_uint4(st.compact_word(), 0u, (uint32_t)b, (uint32_t)(b >> 32));
    } else if (cnt != 0u) {
      rec.x = st.word();
      if (rec.x != 0u) {
        uint4* dst = reinterpret_cast<uint4*>(io.st_masks + 4 * I);
        dst[0] = make_uint4((uint32_t)st.m0, (uint32_t)(st.m0 >> 32), (uint32_t)st.m1,
                            (uint32_t)(st.m1 >> 32));
        dst[1] = make_uint4((uint32_t)st.m2, (uint32_t)(st.m2 >> 32), (uint32_t)st.m3,
                            (uint32_t)(st.m3 >> 32));
      }
    }
    reinterpret_cast<uint4*>(io.st_rec)[I] = rec;
  }
}

// The colour half of preprocess_fwd_kernel (the rgb and clamped rows), after
// the geometry half: Gaussians with radius > 0 (those that touch a tile) get
// gaussian_colour, the others zeros.  kRow as in preprocess_fwd_kernel.
template <int kRow>
__global__ void __launch_bounds__(kColourBlock)
preprocess_colour_kernel(const fgs_preprocess_params prm, const fgs_preprocess_fwd_io io) {
  extern __shared__ float4 s_sh4[];
  float* __restrict__ s_sh = reinterpret_cast<float*>(s_sh4);
  const int row = kRow > 0 ? kRow : prm.max_sh_coeffs * 3;
  const int nblk = (prm.P + kColourBlock - 1) / kColourBlock;
  // a bounded grid walks the blocks of Gaussians in turn (uniform loop)
  for (int blk = (int)blockIdx.x; blk < nblk; blk += (int)gridDim.x) {
    if constexpr (kRow > 0) stage_sh_rows<kRow, kColourBlock>(io.sh, prm.P, s_sh, blk, io.radii);
    const int i = blk * kColourBlock + (int)threadIdx.x;
    if (i < prm.P) {
      const size_t I = (size_t)i;
      float col[3] = {0.f, 0.f, 0.f};
      uint8_t clamp[3] = {0, 0, 0};
      if (io.radii[I] > 0)
        gaussian_colour(prm, io.colors_precomp, io.campos, io.dc,
                        kRow > 0 ? s_sh + threadIdx.x * kRow
                                 : (io.sh ? io.sh + I * (size_t)row : nullptr),
                        I, io.means3d[3 * I + 0], io.means3d[3 * I + 1], io.means3d[3 * I + 2],
                        col, clamp);
#pragma unroll
      for (int c = 0; c < 3; ++c) {
        io.rgb[3 * I + c] = col[c];
        io.clamped[3 * I + c] = clamp[c];
      }
    }
    if constexpr (kRow > 0) __syncthreads();  // the next block's staging reuses the rows
  }
}

// kRow as in preprocess_fwd_kernel. Staged, the SH coefficients are copied
// into registers so the LDS rows can be reused for the gradient rows, which
// leave as one coalesced block store at the end.
template <int kRow>
__global__ void __launch_bounds__(kShBlock)
preprocess_bwd_kernel(const fgs_preprocess_params prm, const fgs_preprocess_bwd_io io,
                      float focal_x, float focal_y) {
  extern __shared__ float4 s_sh4[];
  float* __restrict__ s_sh = reinterpret_cast<float*>(s_sh4);
  constexpr bool kStaged = kRow > 0;
  const int msh = kStaged ? kRow / 3 : prm.max_sh_coeffs;
  // (all rows staged: waiting for the radii before the row loads, to skip the
  // culled ones, measured 2 us slower here at 1M Gaussians)
  if constexpr (kStaged) stage_sh_rows<kRow>(io.sh, prm.P, s_sh);
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  const bool valid = i < prm.P;
  const size_t I = valid ? (size_t)i : 0;
  float shv[45];
  float dsv[45];
#pragma unroll
  for (int k = 0; k < 45; ++k) {
    shv[k] = (kStaged && k < kRow) ? s_sh[threadIdx.x * kRow + k] : 0.0f;
    dsv[k] = 0.0f;
  }
  float dm[3] = {0.f, 0.f, 0.f};
  float ddc[3] = {0.f, 0.f, 0.f};
  float dcol[3] = {0.f, 0.f, 0.f};
  float dop = 0.f;
  float dsc[3] = {0.f, 0.f, 0.f};
  float3 sc_act = make_float3(0.f, 0.f, 0.f);  // the (activated) scales, once read
  float dq[4] = {0.f, 0.f, 0.f, 0.f};
  float4 dvsp = make_float4(0.f, 0.f, 0.f, 0.f);
  float* __restrict__ ds = kStaged ? dsv : (io.dL_dsh ? io.dL_dsh + I * (size_t)msh * 3 : nullptr);
  int sh_written = 0;  // number of rest coefficients written below
  if (valid && io.radii[I] > 0) {
    const float px = io.means3d[3 * I + 0], py = io.means3d[3 * I + 1], pz = io.means3d[3 * I + 2];
    const Mat16 V = load_mat(io.viewmatrix);
    const Mat16 Pm = load_mat(io.projmatrix);
    const float ph3 = Pm.m[3] * px + Pm.m[7] * py + Pm.m[11] * pz + Pm.m[15];
    const size_t xs = io.dL_dxys_stride > 0 ? (size_t)io.dL_dxys_stride : 2u;
    const float gx = io.dL_dxys ? io.dL_dxys[xs * I + 0] : 0.f;
    const float gy = io.dL_dxys ? io.dL_dxys[xs * I + 1] : 0.f;
    float cg0 = 0.f, cg1 = 0.f, cg2 = 0.f, cg3 = 0.f;
    if (io.dL_dconic_opacity) {
      const float4 g = *reinterpret_cast<const float4*>(io.dL_dconic_opacity + 4 * I);
      cg0 = g.x;
      cg1 = g.y;
      cg2 = g.z;
      cg3 = g.w;
    }
    const float* __restrict__ cs =
        (prm.use_cov3d_precomp ? io.cov3d_precomp : io.cov3d_fwd) + 6 * I;
    float c3[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) c3[k] = cs[k];
    float dcov_extra[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float dmc[3];
    {
      Cov2D cv;
      cov2d_eval(V, px, py, pz, focal_x, focal_y, prm.tan_fovx, prm.tan_fovy, c3, cv);
      const float x_grad_mul = (cv.txtz < -cv.limx || cv.txtz > cv.limx) ? 0.0f : 1.0f;
      const float y_grad_mul = (cv.tytz < -cv.limy || cv.tytz > cv.limy) ? 0.0f : 1.0f;
      // Metal indexing Tm[c][r]; the third column is zero.
      float Tm[3][3];
#pragma unroll
      for (int r = 0; r < 3; ++r) {
        Tm[0][r] = cv.T[0][r];
        Tm[1][r] = cv.T[1][r];
        Tm[2][r] = 0.0f;
      }
      const float Vrk[3][3] = {{c3[0], c3[1], c3[2]}, {c3[1], c3[3], c3[4]}, {c3[2], c3[4], c3[5]}};
      float Wm[3][3];
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int r = 0; r < 3; ++r) Wm[c][r] = V.m[4 * c + r];
      const float a = cv.cov00 + 0.3f;
      const float b = cv.cov01;
      const float c = cv.cov11 + 0.3f;
      const float denom = a * c - b * b;
      const float denom2inv = 1.0f / ((denom * denom) + 1e-7f);
      float dL_da = 0.f, dL_db = 0.f, dL_dc = 0.f;
      if (denom2inv != 0.0f) {
        dL_da = denom2inv * (-c * c * cg0 + 2.0f * b * c * cg1 + (denom - a * c) * cg2);
        dL_dc = denom2inv * (-a * a * cg2 + 2.0f * a * b * cg1 + (denom - a * c) * cg0);
        dL_db = denom2inv * 2.0f * (b * c * cg0 - (denom + 2.0f * b * b) * cg1 + a * b * cg2);
        dcov_extra[0] = (Tm[0][0] * Tm[0][0] * dL_da + Tm[0][0] * Tm[1][0] * dL_db + Tm[1][0] * Tm[1][0] * dL_dc);
        dcov_extra[3] = (Tm[0][1] * Tm[0][1] * dL_da + Tm[0][1] * Tm[1][1] * dL_db + Tm[1][1] * Tm[1][1] * dL_dc);
        dcov_extra[5] = (Tm[0][2] * Tm[0][2] * dL_da + Tm[0][2] * Tm[1][2] * dL_db + Tm[1][2] * Tm[1][2] * dL_dc);
        dcov_extra[1] = 2.0f * Tm[0][0] * Tm[0][1] * dL_da + (Tm[0][0] * Tm[1][1] + Tm[0][1] * Tm[1][0]) * dL_db + 2.0f * Tm[1][0] * Tm[1][1] * dL_dc;
        dcov_extra[2] = 2.0f * Tm[0][0] * Tm[0][2] * dL_da + (Tm[0][0] * Tm[1][2] + Tm[0][2] * Tm[1][0]) * dL_db + 2.0f * Tm[1][0] * Tm[1][2] * dL_dc;
        dcov_extra[4] = 2.0f * Tm[0][2] * Tm[0][1] * dL_da + (Tm[0][1] * Tm[1][2] + Tm[0][2] * Tm[1][1]) * dL_db + 2.0f * Tm[1][1] * Tm[1][2] * dL_dc;
      }
      const float dL_dT00 = 2.0f * (Tm[0][0] * Vrk[0][0] + Tm[0][1] * Vrk[0][1] + Tm[0][2] * Vrk[0][2]) * dL_da +
                            (Tm[1][0] * Vrk[0][0] + Tm[1][1] * Vrk[0][1] + Tm[1][2] * Vrk[0][2]) * dL_db;
      const float dL_dT01 = 2.0f * (Tm[0][0] * Vrk[1][0] + Tm[0][1] * Vrk[1][1] + Tm[0][2] * Vrk[1][2]) * dL_da +
                            (Tm[1][0] * Vrk[1][0] + Tm[1][1] * Vrk[1][1] + Tm[1][2] * Vrk[1][2]) * dL_db;
      const float dL_dT02 = 2.0f * (Tm[0][0] * Vrk[2][0] + Tm[0][1] * Vrk[2][1] + Tm[0][2] * Vrk[2][2]) * dL_da +
                            (Tm[1][0] * Vrk[2][0] + Tm[1][1] * Vrk[2][1] + Tm[1][2] * Vrk[2][2]) * dL_db;
      const float dL_dT10 = 2.0f * (Tm[1][0] * Vrk[0][0] + Tm[1][1] * Vrk[0][1] + Tm[1][2] * Vrk[0][2]) * dL_dc +
                            (Tm[0][0] * Vrk[0][0] + Tm[0][1] * Vrk[0][1] + Tm[0][2] * Vrk[0][2]) * dL_db;
      const float dL_dT11 = 2.0f * (Tm[1][0] * Vrk[1][0] + Tm[1][1] * Vrk[1][1] + Tm[1][2] * Vrk[1][2]) * dL_dc +
                            (Tm[0][0] * Vrk[1][0] + Tm[0][1] * Vrk[1][1] + Tm[0][2] * Vrk[1][2]) * dL_db;
      const float dL_dT12 = 2.0f * (Tm[1][0] * Vrk[2][0] + Tm[1][1] * Vrk[2][1] + Tm[1][2] * Vrk[2][2]) * dL_dc +
                            (Tm[0][0] * Vrk[2][0] + Tm[0][1] * Vrk[2][1] + Tm[0][2] * Vrk[2][2]) * dL_db;
      const float dL_dJ00 = Wm[0][0] * dL_dT00 + Wm[0][1] * dL_dT01 + Wm[0][2] * dL_dT02;
      const float dL_dJ02 = Wm[2][0] * dL_dT00 + Wm[2][1] * dL_dT01 + Wm[2][2] * dL_dT02;
      const float dL_dJ11 = Wm[1][0] * dL_dT10 + Wm[1][1] * dL_dT11 + Wm[1][2] * dL_dT12;
      const float dL_dJ12 = Wm[2][0] * dL_dT10 + Wm[2][1] * dL_dT11 + Wm[2][2] * dL_dT12;
      const float tz = 1.0f / cv.t2;
      const float tz2 = tz * tz;
      const float tz3 = tz2 * tz;
      const float dL_dtx = x_grad_mul * -focal_x * tz2 * dL_dJ02;
      const float dL_dty = y_grad_mul * -focal_y * tz2 * dL_dJ12;
      const float dL_dtz = -focal_x * tz2 * dL_dJ00 - focal_y * tz2 * dL_dJ11 +
                           (2.0f * focal_x * cv.t0) * tz3 * dL_dJ02 +
                           (2.0f * focal_y * cv.t1) * tz3 * dL_dJ12;
      dmc[0] = V.m[0] * dL_dtx + V.m[1] * dL_dty + V.m[2] * dL_dtz;
      dmc[1] = V.m[4] * dL_dtx + V.m[5] * dL_dty + V.m[6] * dL_dtz;
      dmc[2] = V.m[8] * dL_dtx + V.m[9] * dL_dty + V.m[10] * dL_dtz;
    }
    const float m_w = 1.0f / (ph3 + 1.0e-7f);
    const float mul1 = (Pm.m[0] * px + Pm.m[4] * py + Pm.m[8] * pz + Pm.m[12]) * m_w * m_w;
    const float mul2 = (Pm.m[1] * px + Pm.m[5] * py + Pm.m[9] * pz + Pm.m[13]) * m_w * m_w;
    const float dmx = (Pm.m[0] * m_w - Pm.m[3] * mul1) * gx + (Pm.m[1] * m_w - Pm.m[3] * mul2) * gy;
    const float dmy = (Pm.m[4] * m_w - Pm.m[7] * mul1) * gx + (Pm.m[5] * m_w - Pm.m[7] * mul2) * gy;
    const float dmz = (Pm.m[8] * m_w - Pm.m[11] * mul1) * gx + (Pm.m[9] * m_w - Pm.m[11] * mul2) * gy;
    dm[0] = dmx + dmc[0];
    dm[1] = dmy + dmc[1];
    dm[2] = dmz + dmc[2];
    dop = cg3;
    float drgb[3] = {0.f, 0.f, 0.f};
    if (io.dL_drgb) {
#pragma unroll
      for (int c = 0; c < 3; ++c) drgb[c] = io.dL_drgb[3 * I + c];
    }
    if (prm.use_colors_precomp) {
#pragma unroll
      for (int c = 0; c < 3; ++c) dcol[c] = drgb[c];
    } else {
      float dRGB[3];
#pragma unroll
      for (int c = 0; c < 3; ++c) dRGB[c] = io.clamped[3 * I + c] ? 0.0f : drgb[c];
#pragma unroll
      for (int c = 0; c < 3; ++c) ddc[c] = kSH_C0 * dRGB[c];
      if (prm.degree > 0 && msh >= 3) {
        const float d0 = px - io.campos[0], d1 = py - io.campos[1], d2 = pz - io.campos[2];
        const float len = __builtin_sqrtf(d0 * d0 + d1 * d1 + d2 * d2);
        const float x = d0 / len, y = d1 / len, z = d2 / len;
        const float* __restrict__ s = kStaged ? shv : io.sh + I * (size_t)msh * 3;
        float dRGBdx[3], dRGBdy[3], dRGBdz[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          ds[0 * 3 + c] = (-kSH_C1 * y) * dRGB[c];
          ds[1 * 3 + c] = (kSH_C1 * z) * dRGB[c];
          ds[2 * 3 + c] = (-kSH_C1 * x) * dRGB[c];
          dRGBdx[c] = -kSH_C1 * s[2 * 3 + c];
          dRGBdy[c] = -kSH_C1 * s[0 * 3 + c];
          dRGBdz[c] = kSH_C1 * s[1 * 3 + c];
        }
        sh_written = 3;
        if (prm.degree > 1 && msh >= 8) {
          const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
#pragma unroll
          for (int c = 0; c < 3; ++c) {
            ds[3 * 3 + c] = (kSH_C2[0] * xy) * dRGB[c];
            ds[4 * 3 + c] = (kSH_C2[1] * yz) * dRGB[c];
            ds[5 * 3 + c] = (kSH_C2[2] * (2.0f * zz - xx - yy)) * dRGB[c];
            ds[6 * 3 + c] = (kSH_C2[3] * xz) * dRGB[c];
            ds[7 * 3 + c] = (kSH_C2[4] * (xx - yy)) * dRGB[c];
            const float s3 = s[3 * 3 + c], s4 = s[4 * 3 + c], s5 = s[5 * 3 + c], s6 = s[6 * 3 + c],
                        s7 = s[7 * 3 + c];
            dRGBdx[c] += kSH_C2[0] * y * s3 + kSH_C2[2] * 2.0f * -x * s5 + kSH_C2[3] * z * s6 +
                         kSH_C2[4] * 2.0f * x * s7;
            dRGBdy[c] += kSH_C2[0] * x * s3 + kSH_C2[1] * z * s4 + kSH_C2[2] * 2.0f * -y * s5 +
                         kSH_C2[4] * 2.0f * -y * s7;
            dRGBdz[c] += kSH_C2[1] * y * s4 + kSH_C2[2] * 4.0f * z * s5 + kSH_C2[3] * x * s6;
          }
          sh_written = 8;
          if (prm.degree > 2 && msh >= 15) {
#pragma unroll
            for (int c = 0; c < 3; ++c) {
              ds[8 * 3 + c] = (kSH_C3[0] * y * (3.0f * xx - yy)) * dRGB[c];
              ds[9 * 3 + c] = (kSH_C3[1] * xy * z) * dRGB[c];
              ds[10 * 3 + c] = (kSH_C3[2] * y * (4.0f * zz - xx - yy)) * dRGB[c];
              ds[11 * 3 + c] = (kSH_C3[3] * z * (2.0f * zz - 3.0f * xx - 3.0f * yy)) * dRGB[c];
              ds[12 * 3 + c] = (kSH_C3[4] * x * (4.0f * zz - xx - yy)) * dRGB[c];
              ds[13 * 3 + c] = (kSH_C3[5] * z * (xx - yy)) * dRGB[c];
              ds[14 * 3 + c] = (kSH_C3[6] * x * (xx - 3.0f * yy)) * dRGB[c];
              const float s8 = s[8 * 3 + c], s9 = s[9 * 3 + c], s10 = s[10 * 3 + c],
                          s11 = s[11 * 3 + c], s12 = s[12 * 3 + c], s13 = s[13 * 3 + c],
                          s14 = s[14 * 3 + c];
              dRGBdx[c] += (kSH_C3[0] * s8 * 6.0f * xy + kSH_C3[1] * s9 * yz +
                            kSH_C3[2] * s10 * -2.0f * xy + kSH_C3[3] * s11 * -6.0f * xz +
                            kSH_C3[4] * s12 * (-3.0f * xx + 4.0f * zz - yy) +
                            kSH_C3[5] * s13 * 2.0f * xz + kSH_C3[6] * s14 * 3.0f * (xx - yy));
              dRGBdy[c] += (kSH_C3[0] * s8 * 3.0f * (xx - yy) + kSH_C3[1] * s9 * xz +
                            kSH_C3[2] * s10 * (-3.0f * yy + 4.0f * zz - xx) +
                            kSH_C3[3] * s11 * -6.0f * yz + kSH_C3[4] * s12 * -2.0f * xy +
                            kSH_C3[5] * s13 * -2.0f * yz + kSH_C3[6] * s14 * -6.0f * xy);
              dRGBdz[c] += (kSH_C3[1] * s9 * xy + kSH_C3[2] * s10 * 8.0f * yz +
                            kSH_C3[3] * s11 * 3.0f * (2.0f * zz - xx - yy) +
                            kSH_C3[4] * s12 * 8.0f * xz + kSH_C3[5] * s13 * (xx - yy));
            }
            sh_written = 15;
          }
        }
        const float ddir0 = dRGBdx[0] * dRGB[0] + dRGBdx[1] * dRGB[1] + dRGBdx[2] * dRGB[2];
        const float ddir1 = dRGBdy[0] * dRGB[0] + dRGBdy[1] * dRGB[1] + dRGBdy[2] * dRGB[2];
        const float ddir2 = dRGBdz[0] * dRGB[0] + dRGBdz[1] * dRGB[1] + dRGBdz[2] * dRGB[2];
        const float l = fmaxf(__builtin_sqrtf(d0 * d0 + d1 * d1 + d2 * d2), 1e-6f);
        const float n0 = d0 / l, n1 = d1 / l, n2 = d2 / l;
        const float nd = n0 * ddir0 + n1 * ddir1 + n2 * ddir2;
        dm[0] += (ddir0 - n0 * nd) / l;
        dm[1] += (ddir1 - n1 * nd) / l;
        dm[2] += (ddir2 - n2 * nd) / l;
      }
    }
    if (!prm.use_cov3d_precomp) {
      const float4 rq = load_rotation(io.rotations, io.rotations ? nullptr : io.quats_raw, I);
      const float r = rq.x, x = rq.y, y = rq.z, z = rq.w;
      float R[3][3];
      R[0][0] = 1.0f - 2.0f * (y * y + z * z);
      R[0][1] = 2.0f * (x * y - r * z);
      R[0][2] = 2.0f * (x * z + r * y);
      R[1][0] = 2.0f * (x * y + r * z);
      R[1][1] = 1.0f - 2.0f * (x * x + z * z);
      R[1][2] = 2.0f * (y * z - r * x);
      R[2][0] = 2.0f * (x * z - r * y);
      R[2][1] = 2.0f * (y * z + r * x);
      R[2][2] = 1.0f - 2.0f * (x * x + y * y);
      sc_act = load_scale(io.scales, io.log_scales, I);
      const float s[3] = {prm.scale_modifier * sc_act.x, prm.scale_modifier * sc_act.y,
                          prm.scale_modifier * sc_act.z};
      float M[3][3];
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int rr = 0; rr < 3; ++rr) M[c][rr] = s[rr] * R[c][rr];
      float cc[6];
#pragma unroll
      for (int k = 0; k < 6; ++k) cc[k] = (io.dL_dcov3d ? io.dL_dcov3d[6 * I + k] : 0.0f) + dcov_extra[k];
      const float dS[3][3] = {{cc[0], 0.5f * cc[1], 0.5f * cc[2]},
                              {0.5f * cc[1], cc[3], 0.5f * cc[4]},
                              {0.5f * cc[2], 0.5f * cc[4], cc[5]}};
      float dM[3][3];
#pragma unroll
      for (int c = 0; c < 3; ++c)
#pragma unroll
        for (int rr = 0; rr < 3; ++rr)
          dM[c][rr] = (2.0f * M[0][rr]) * dS[c][0] + (2.0f * M[1][rr]) * dS[c][1] +
                      (2.0f * M[2][rr]) * dS[c][2];
      float dMt[3][3];
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] = dM[bb][a];
#pragma unroll
      for (int a = 0; a < 3; ++a)
        dsc[a] = R[0][a] * dMt[a][0] + R[1][a] * dMt[a][1] + R[2][a] * dMt[a][2];
#pragma unroll
      for (int a = 0; a < 3; ++a)
#pragma unroll
        for (int bb = 0; bb < 3; ++bb) dMt[a][bb] *= s[a];
      dq[0] = 2.0f * z * (dMt[0][1] - dMt[1][0]) + 2.0f * y * (dMt[2][0] - dMt[0][2]) + 2.0f * x * (dMt[1][2] - dMt[2][1]);
      dq[1] = 2.0f * y * (dMt[1][0] + dMt[0][1]) + 2.0f * z * (dMt[2][0] + dMt[0][2]) + 2.0f * r * (dMt[1][2] - dMt[2][1]) - 4.0f * x * (dMt[2][2] + dMt[1][1]);
      dq[2] = 2.0f * x * (dMt[1][0] + dMt[0][1]) + 2.0f * r * (dMt[2][0] - dMt[0][2]) + 2.0f * z * (dMt[1][2] + dMt[2][1]) - 4.0f * y * (dMt[2][2] + dMt[0][0]);
      dq[3] = 2.0f * r * (dMt[0][1] - dMt[1][0]) + 2.0f * x * (dMt[2][0] + dMt[0][2]) + 2.0f * y * (dMt[1][2] + dMt[2][1]) - 4.0f * z * (dMt[1][1] + dMt[0][0]);
    }
    if (io.dL_dviewspace_out) dvsp = *reinterpret_cast<const float4*>(io.dL_dviewspace_out + 4 * I);
  }
  if constexpr (kStaged) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kRow; ++k) s_sh[threadIdx.x * kRow + k] = dsv[k];
    __syncthreads();
    store_sh_rows<kRow>(s_sh, prm.P, io.dL_dsh);
  }
  if (!valid) return;
  // Write every element of every gradient row.
#pragma unroll
  for (int k = 0; k < 3; ++k) io.dL_dmeans3d[3 * I + k] = dm[k];
  if (io.dL_ddc)
#pragma unroll
    for (int k = 0; k < 3; ++k) io.dL_ddc[3 * I + k] = ddc[k];
  if (io.dL_dcolors_precomp)
#pragma unroll
    for (int k = 0; k < 3; ++k) io.dL_dcolors_precomp[3 * I + k] = dcol[k];
  if (io.dL_dopacities) io.dL_dopacities[I] = dop;
  if (io.dL_dscales)
#pragma unroll
    for (int k = 0; k < 3; ++k) io.dL_dscales[3 * I + k] = dsc[k];
  if (io.dL_drotations)
    *reinterpret_cast<float4*>(io.dL_drotations + 4 * I) = make_float4(dq[0], dq[1], dq[2], dq[3]);
  // the activations' backward, with the operations of activations_bwd_kernel
  // (fgs_train.hip), so the fused and the separate forms agree bit for bit
  if (io.dL_dlogits) {
    const float o = load_opacity(io.act_opacities, io.act_opacities ? nullptr : io.opacity_logits, I);
    io.dL_dlogits[I] = dop * (1.0f - o) * o;
  }
  if (io.dL_dlog_scales) {
    if (!(valid && io.radii[I] > 0)) sc_act = load_scale(io.scales, io.log_scales, I);
    io.dL_dlog_scales[3 * I + 0] = dsc[0] * sc_act.x;
    io.dL_dlog_scales[3 * I + 1] = dsc[1] * sc_act.y;
    io.dL_dlog_scales[3 * I + 2] = dsc[2] * sc_act.z;
  }
  if (io.dL_dquats) {
    const float4 q = *reinterpret_cast<const float4*>(io.quats_raw + 4 * I);
    *reinterpret_cast<float4*>(io.dL_dquats + 4 * I) =
        quat_normalize_grad(q, make_float4(dq[0], dq[1], dq[2], dq[3]));
  }
  *reinterpret_cast<float4*>(io.dL_dviewspace_in + 4 * I) = dvsp;
  if (!kStaged && ds) {
    for (int k = sh_written * 3; k < msh * 3; ++k) ds[k] = 0.0f;
  }
}

}  // namespace fgs

using namespace fgs;

// Row length (floats) of the LDS-staged SH path, or 0 for direct reads. Rows
// are staged when the SH colour path is active, the row is one of the three
// sizes of degrees 1-3 with 3, 8 or 15 rest coefficients (at most 45 floats:
// 45 KB of LDS per workgroup) and the arrays are 16-byte aligned.
// (The forward passes sh as both arrays.)
static int staged_sh_row(const fgs_preprocess_params* p, const float* sh, const float* dsh) {
  if (p->use_colors_precomp || p->degree <= 0 || !sh || !dsh) return 0;
  if ((reinterpret_cast<uintptr_t>(sh) | reinterpret_cast<uintptr_t>(dsh)) & 15u) return 0;
  const int m = p->max_sh_coeffs;
  return (m == 3 || m == 8 || m == 15) ? 3 * m : 0;
}

// Arguments of the preprocess forward, checked once for the fused call and
// for each of its two halves.
static int32_t preprocess_fwd_check(const fgs_preprocess_params* p, const fgs_preprocess_fwd_io* io,
                                    const char* who) {
  char msg[160];
  auto fail = [&](const char* what) {
    std::snprintf(msg, sizeof(msg), "%s: %s", who, what);
    return set_error(FGS_ERR_INVALID_ARGUMENT, msg);
  };
  if (!p || !io) return fail("null argument");
  if (p->P < 0) return fail("P < 0");
  if (p->P == 0) return FGS_OK;
  if (!io->means3d || !(io->opacities || io->opacity_logits) || !io->viewmatrix ||
      !io->projmatrix || !io->campos ||
      !io->viewspace_in || !io->radii || !io->xys || !io->depths || !io->cov3d || !io->rgb ||
      !io->conic_opacity || !io->tiles_touched || !io->clamped || !io->viewspace_out)
    return fail("missing tensor");
  if (p->use_cov3d_precomp ? !io->cov3d_precomp
                           : (!(io->scales || io->log_scales) || !(io->rotations || io->raw_rotations)))
    return fail("missing geometry tensors");
  if (p->use_colors_precomp ? !io->colors_precomp : (!io->dc || (p->degree > 0 && !io->sh)))
    return fail("missing colour tensors");
  if (!p->use_colors_precomp && p->degree > 0) {
    const int d = p->degree > 3 ? 3 : p->degree;
    if (p->max_sh_coeffs < (d + 1) * (d + 1) - 1)
      return fail("sh has fewer coefficients than the degree needs");
  }
  if (p->image_width <= 0 || p->image_height <= 0 || p->grid_x <= 0 || p->grid_y <= 0)
    return fail("bad image size");
  // the packed tile walks keep tile coordinates in 16 bits
  if (p->grid_x > 65535 || p->grid_y > 65535) return fail("more than 65535 tiles on a side");
  if (!io->st_rec != !io->st_masks || (reinterpret_cast<uintptr_t>(io->st_masks) & 15u) ||
      (reinterpret_cast<uintptr_t>(io->st_rec) & 15u))
    return fail("st_rec and st_masks must both be set (16-byte aligned) or both NULL");
  return FGS_OK;
}

// part: 0 the fused kernel, 1 the geometry half, 2 the colour half.
static int32_t preprocess_fwd_launch(const fgs_preprocess_params* p,
                                     const fgs_preprocess_fwd_io* io, void* stream, int part,
                                     const char* who) {
  if (const int32_t e = preprocess_fwd_check(p, io, who)) return e;
  if (p->P == 0) return FGS_OK;
  const float fx = (float)p->image_width / (2.0f * p->tan_fovx);
  const float fy = (float)p->image_height / (2.0f * p->tan_fovy);
  const unsigned blocks = (unsigned)((p->P + kShBlock - 1) / kShBlock);
  // Staging moves every row of the block, visible or not, but as coalesced
  // 16-byte loads; the direct path reads 4-byte elements 180 bytes apart.
  const hipStream_t st = (hipStream_t)stream;
  const dim3 grid(blocks), block(kShBlock);
  if (part == 2) {
    const unsigned nblk = ceil_div_u(p->P, kColourBlock);
    const dim3 grid(kColourGrid > 0 && nblk > (unsigned)kColourGrid ? (unsigned)kColourGrid : nblk),
        block(kColourBlock);
    if (const int32_t e = launch_mark(kLaunchPreprocessColour, st, 0)) return e;
    switch (staged_sh_row(p, io->sh, io->sh)) {
      case 9:
        hipLaunchKernelGGL(preprocess_colour_kernel<9>, grid, block,
                           kColourBlock * 9 * sizeof(float), st, *p, *io);
        break;
      case 24:
        hipLaunchKernelGGL(preprocess_colour_kernel<24>, grid, block,
                           kColourBlock * 24 * sizeof(float), st, *p, *io);
        break;
      case 45:
        hipLaunchKernelGGL(preprocess_colour_kernel<45>, grid, block,
                           kColourBlock * 45 * sizeof(float), st, *p, *io);
        break;
      default:
        hipLaunchKernelGGL(preprocess_colour_kernel<0>, grid, block, 0, st, *p, *io);
    }
    if (check_launch("preprocess_colour_kernel") != FGS_OK) return FGS_ERR_LAUNCH;
    return launch_mark(kLaunchPreprocessColour, st, 1);
  }
  if (const int32_t e = launch_mark(kLaunchPreprocessFwd, st, 0)) return e;
  if (part == 1) {
    hipLaunchKernelGGL((preprocess_fwd_kernel<0, false>), grid, block, 0, st, *p, *io, fx, fy);
  } else {
    switch (staged_sh_row(p, io->sh, io->sh)) {
      case 9:
        hipLaunchKernelGGL(preprocess_fwd_kernel<9>, grid, block, kShBlock * 9 * sizeof(float), st, *p,
                           *io, fx, fy);
        break;
      case 24:
        hipLaunchKernelGGL(preprocess_fwd_kernel<24>, grid, block, kShBlock * 24 * sizeof(float), st,
                           *p, *io, fx, fy);
        break;
      case 45:
        hipLaunchKernelGGL(preprocess_fwd_kernel<45>, grid, block, kShBlock * 45 * sizeof(float), st,
                           *p, *io, fx, fy);
        break;
      default:
        hipLaunchKernelGGL(preprocess_fwd_kernel<0>, grid, block, 0, st, *p, *io, fx, fy);
    }
  }
  if (check_launch("preprocess_fwd_kernel") != FGS_OK) return FGS_ERR_LAUNCH;
  return launch_mark(kLaunchPreprocessFwd, st, 1);
}

extern "C" int32_t fgs_preprocess_fwd(const fgs_preprocess_params* p,
                                      const fgs_preprocess_fwd_io* io, void* stream) {
  return preprocess_fwd_launch(p, io, stream, 0, "fgs_preprocess_fwd");
}

extern "C" int32_t fgs_preprocess_geometry_fwd(const fgs_preprocess_params* p,
                                               const fgs_preprocess_fwd_io* io, void* stream) {
  return preprocess_fwd_launch(p, io, stream, 1, "fgs_preprocess_geometry_fwd");
}

extern "C" int32_t fgs_preprocess_colour_fwd(const fgs_preprocess_params* p,
                                             const fgs_preprocess_fwd_io* io, void* stream) {
  return preprocess_fwd_launch(p, io, stream, 2, "fgs_preprocess_colour_fwd");
}

extern "C" int32_t fgs_preprocess_bwd(const fgs_preprocess_params* p,
                                      const fgs_preprocess_bwd_io* io, void* stream) {
  if (!p || !io) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_preprocess_bwd: null argument");
  if (p->P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_preprocess_bwd: P < 0");
  if (p->P == 0) return FGS_OK;
  if (!io->means3d || !io->viewmatrix || !io->projmatrix || !io->campos || !io->radii ||
      !io->clamped || !io->dL_dmeans3d || !io->dL_dviewspace_in ||
      !(io->dL_dopacities || (io->dL_dlogits && (io->act_opacities || io->opacity_logits))))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_preprocess_bwd: missing tensor");
  if (p->use_cov3d_precomp ? !io->cov3d_precomp
                           : (!io->cov3d_fwd || !(io->scales || io->log_scales) ||
                              !(io->rotations || io->quats_raw)))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_preprocess_bwd: missing geometry tensors");
  if (!p->use_colors_precomp && p->degree > 0 && p->max_sh_coeffs >= 3 && (!io->sh || !io->dL_dsh))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_preprocess_bwd: missing sh tensors");
  if ((io->dL_dlogits && !(io->act_opacities || io->opacity_logits)) ||
      (io->dL_dquats && !io->quats_raw) ||
      ((io->dL_dlog_scales || io->dL_dquats) && p->use_cov3d_precomp))
    return set_error(FGS_ERR_INVALID_ARGUMENT,
                     "fgs_preprocess_bwd: fused activation gradients need act_opacities, "
                     "quats_raw and the scale/rotation path");
  if (io->dL_dxys_stride < 0 || io->dL_dxys_stride == 1)
    return set_error(FGS_ERR_INVALID_ARGUMENT,
                     "fgs_preprocess_bwd: dL_dxys_stride must be 0 or at least 2");
  const float fx = 0.5f * (float)p->image_width / fmaxf(p->tan_fovx, 1e-6f);
  const float fy = 0.5f * (float)p->image_height / fmaxf(p->tan_fovy, 1e-6f);
  const unsigned blocks = (unsigned)((p->P + kShBlock - 1) / kShBlock);
  const hipStream_t st = (hipStream_t)stream;
  const dim3 grid(blocks), block(kShBlock);
  if (const int32_t e = launch_mark(kLaunchPreprocessBwd, st, 0)) return e;
  switch (staged_sh_row(p, io->sh, io->dL_dsh)) {
    case 9:
      hipLaunchKernelGGL(preprocess_bwd_kernel<9>, grid, block, kShBlock * 9 * sizeof(float), st,
                         *p, *io, fx, fy);
      break;
    case 24:
      hipLaunchKernelGGL(preprocess_bwd_kernel<24>, grid, block, kShBlock * 24 * sizeof(float),
                         st, *p, *io, fx, fy);
      break;
    case 45:
      hipLaunchKernelGGL(preprocess_bwd_kernel<45>, grid, block, kShBlock * 45 * sizeof(float),
                         st, *p, *io, fx, fy);
      break;
    default:
      hipLaunchKernelGGL(preprocess_bwd_kernel<0>, grid, block, 0, st, *p, *io, fx, fy);
  }
  if (check_launch("preprocess_bwd_kernel") != FGS_OK) return FGS_ERR_LAUNCH;
  return launch_mark(kLaunchPreprocessBwd, st, 1);
}
