// fgs_raster.hip -- tile rasterization forward and backward (gfx950, wave64).
//
// Forward (semantics of fastgs_rasterize.metal:25-159): one 256-thread
// workgroup per 16x16 tile, one pixel per thread, wavefront w owning the 8x8
// quarter (w & 1, w >> 1).  The tile's sorted splat list is streamed through
// LDS in batches
// of 256 (each thread stages one splat: 2D mean, conic, opacity, colour and
// opacity), then every pixel blends the batch front to back.  Pixels stop at
// T < 1e-4; a wavefront whose pixels have all stopped skips the blend loop,
// and the workgroup leaves as soon as every pixel has stopped
// (__syncthreads_count).  Batches whose colours are all finite blend without
// the selects that keep a non-finite colour out of non-taking pixels.  (A
// one-wavefront-per-tile form with per-strip row
// culling measured slower: at 1M splats over 1080p most splats reach every
// row of the tiles they touch, so culling removes little work and one
// wavefront per tile hides less latency.)
//
// Backward (per-(pixel, splat) semantics of
// fastgs_rasterize_backward.metal:24-278): one wavefront per tile, each lane
// owning four pixels (one per 16x4 strip); splats are walked back to front
// from the tile's max_contrib in LDS batches of 64.  Each pixel recovers
// T_j = T_{j+1} / (1 - alpha_j) starting from final_T and carries one scalar
// for the colour behind the splat, so no per-bucket sampled state is needed.
// Strips a splat cannot reach (conservative alpha >= 1/255 row extent) are
// skipped wave-uniformly; the pixel terms are computed without branches.  Per
// splat, the 11 gradient terms are summed over the wave by permlane swaps and
// DPP adds into an LDS record; each batch is flushed with global float
// atomics whose lanes cover consecutive terms of a few splats.  Given a
// tile-order scratch, the tiles run heaviest first (by max_contrib), so the
// light ones fill the end of the launch.
#include "fgs_common.hpp"

namespace fgs {

struct RasterShape {
  int W, H, gx, gy;
};

// Splat record staged in LDS: a = (x, y, conic.a, conic.b),
// b = (conic.c, opacity, r, g), c = (b, -, -, -) and the Gaussian index.
template <int NCH>
__device__ __forceinline__ void stage_splat(uint32_t g, uint32_t P, const float* __restrict__ means2d,
                                            const float* __restrict__ colors, int stride,
                                            const float* __restrict__ conic_opacity, float4& a,
                                            float4& b, float& c) {
  if (g >= P) {  // out-of-range list entry: an empty splat (opacity 0)
    a = make_float4(0.f, 0.f, 0.f, 0.f);
    b = make_float4(0.f, 0.f, 0.f, 0.f);
    c = 0.f;
    return;
  }
  const float2 xy = *reinterpret_cast<const float2*>(means2d + 2 * (size_t)g);
  const float4 co = *reinterpret_cast<const float4*>(conic_opacity + 4 * (size_t)g);
  const float* col = colors + (size_t)g * stride;
  a = make_float4(xy.x, xy.y, co.x, co.y);
  b = make_float4(co.z, co.w, col[0], NCH > 1 ? col[1] : 0.0f);
  c = NCH > 2 ? col[2] : 0.0f;
}

// Rows [lo, hi] outside which no pixel of a splat can reach alpha >= 1/255.
// alpha >= 1/255 needs o*exp(power) >= 1/255, i.e. q(d) = d^T Conic d <= tau =
// 2 ln(255 o).  The row extent of {q <= tau} is sqrt(tau * a / det).  Margins:
// the float base-2 exponent of a pixel (splat_power on splat_log2_coeffs)
// differs from t = -log2(e) q/2 by at most (4 * 2^-24 + 1.4e-8) log2(e)
// (a dx^2/2 + |b dx dy| + c dy^2/2) <= 2.6e-7 |t| (1 + |rho|) / (1 - |rho|),
// under 1.1e-3 |t| for the conics culled here (det > 1e-3 a c, rho =
// b / sqrt(a c)); the exp (blend_exp2f, relative error < 2e-7), the hardware
// log and the product o*G move the threshold by ~1e-6; det loses at most
// ~6e-5 to cancellation.  tau' = 1.01 tau + 0.05 and hy * 1.001 + 0.25 px
// cover all of these.  Ill-conditioned or non-positive conics, NaN
// opacities and non-finite centres are not culled; o < 0.999/255 never
// blends.
__device__ __forceinline__ float2 splat_rows(float y, float a, float b, float c, float o) {
  const float inf = __builtin_huge_valf();
  float2 r = make_float2(-inf, inf);
  if (!(o == o) || !__builtin_isfinite(y)) return r;
  if (!(255.0f * o >= 0.999f)) return make_float2(inf, -inf);  // alpha <= o < 1/255
  const float tau = 2.0f * __logf(255.0f * o);
  const float det = a * c - b * b;
  if (!(a > 0.f) || !(c > 0.f) || !(det > 1e-3f * a * c)) return r;
  const float tq = fmaxf(tau, 0.0f) * 1.01f + 0.05f;
  const float hy = __builtin_sqrtf(tq * a / det) * 1.001f + 0.25f;
  return make_float2(y - hy, y + hy);
}

template <bool B>
struct FiniteTag {
  static constexpr bool value = B;
};

// Eight waves per SIMD: under that bound the compiler keeps the unrolled loop
// in 54 VGPRs without spills (at six waves it used 80 and spilled 7), and the
// forward ran 221-224 -> 215-218 us at 1M / 1080p.
// kMode bit 0: write the sampled state; bit 1: count metric hits (get_flag);
// bit 2: write each pixel's loop iterations under the reference loop (the
// splats it visits, the one it stops at included: the stop index + 1, or the
// tile's list length if it never stops), a measurement output.
template <int NCH, int kMode>
__global__ void __launch_bounds__(256, 8)
raster_fwd_kernel(const fgs_raster_params prm, const fgs_raster_fwd_io io, RasterShape sh) {
  constexpr bool kSampled = (kMode & 1) != 0;
  constexpr bool kMetric = (kMode & 2) != 0;
  constexpr bool kIters = (kMode & 4) != 0;
  __shared__ float4 s_a[256];
  __shared__ float4 s_b[256];
  __shared__ float s_c[256];
  __shared__ uint32_t s_g[256];
  __shared__ uint32_t s_max[4];
  const int tile = (int)blockIdx.x;
  const int tx = tile % sh.gx, ty = tile / sh.gx;
  const int t = (int)threadIdx.x;
  // wavefront w blends the 8x8 quarter (w & 1, w >> 1) of the tile: compact
  // blocks stop at more similar times than 16x4 strips
  const int w8 = t >> 6;
  const int lx = ((w8 & 1) << 3) | (t & 7), ly = ((w8 >> 1) << 3) | ((t >> 3) & 7);
  const int tp = ly * 16 + lx;  // the pixel's index in the tile
  const int px = tx * kTile + lx, py = ty * kTile + ly;
  const bool inside = px < sh.W && py < sh.H;
  const size_t HW = (size_t)sh.W * (size_t)sh.H;
  const size_t pix = inside ? (size_t)py * sh.W + px : 0;
  uint32_t end = io.ranges[2 * tile + 1];
  if ((int64_t)end > prm.list_len) end = (uint32_t)prm.list_len;
  uint32_t start = io.ranges[2 * tile];
  if (start > end) start = end;
  const int n = (int)(end - start);
  const uint32_t bbm0 = (tile == 0) ? 0u : io.bucket_offsets[tile - 1];
  {
    const int nb = (n + 31) / 32;
    for (int b = t; b < nb; b += 256)
      if ((int64_t)bbm0 + b < prm.bucket_sum) io.bucket_to_tile[bbm0 + b] = (uint32_t)tile;
  }
  const bool count_metric = kMetric && inside && io.metric_map[pix] == 1;
  const float pxf = (float)px, pyf = (float)py;
  float T = 1.0f;
  uint32_t last = 0;
  uint32_t iters = 0;  // kIters: the stop index + 1 once the pixel stops
  float acc[3] = {0.0f, 0.0f, 0.0f};
  int done = inside ? 0 : 1;
  const int rounds = (n + 255) / 256;
  for (int r = 0; r < rounds; ++r) {
    if (__syncthreads_count(done) == 256) break;
    const int base = r * 256;
    const int cnt = (n - base) < 256 ? (n - base) : 256;
    const int cnt8 = (cnt + 7) & ~7;  // padded with splats of opacity 0 (never blended)
    bool fin = true;  // the staged colour is finite
    if (base + t < n) {
      const uint32_t g = io.point_list[start + base + t];
      float4 a, b;
      float c;
      stage_splat<NCH>(g, (uint32_t)prm.num_points, io.means2d, io.colors, prm.num_channels, io.conic_opacity, a, b, c);
      // staged as (x, y, A, B) and (C, o, ...) with the base-2 exponent
      // coefficients of splat_log2_coeffs, the operands of splat_power
      const float3 k2 = splat_log2_coeffs(a.z, a.w, b.x);
      a.z = k2.x;
      a.w = k2.y;
      b.x = k2.z;
      s_a[t] = a;
      s_b[t] = b;
      s_c[t] = c;
      s_g[t] = g;
      fin = __builtin_isfinite(b.z) && (NCH < 2 || __builtin_isfinite(b.w)) &&
            (NCH < 3 || __builtin_isfinite(c));
    } else if (t < cnt8) {
      s_a[t] = make_float4(0.f, 0.f, 0.f, 0.f);
      s_b[t] = make_float4(0.f, 0.f, 0.f, 0.f);
      s_c[t] = 0.0f;
      s_g[t] = 0xFFFFFFFFu;
    }
    const bool colours_finite = __syncthreads_and(fin ? 1 : 0) != 0;
    // Branch-free per splat: blend / stop / take are lane predicates and the
    // state moves by selects, so the wave runs one straight path, eight
    // splats at a time; it leaves the batch once no lane is live.  A lane
    // that stops takes nothing more, as the reference loop's break.
    bool live = !done;
    auto walk = [&](auto finite_tag) {
      constexpr bool kFinite = decltype(finite_tag)::value;
      for (int j0 = 0; j0 < cnt8; j0 += 8) {
        int lg = 0;  // u + 1 of the group's last splat the pixel takes (0: none)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int j = j0 + u;
          const int jj = base + j;
          if (kSampled && (jj & 31) == 0 && jj < n && live) {
            const size_t bk = (size_t)bbm0 + (size_t)(jj >> 5);
            if ((int64_t)bk < prm.bucket_sum) {
              io.sampled_t[bk * 256 + tp] = T;
#pragma unroll
              for (int c = 0; c < NCH; ++c)
                io.sampled_ar[bk * (size_t)prm.num_channels * 256 + (size_t)c * 256 + tp] = acc[c];
            }
          }
          const float4 a = s_a[j];
          const float4 b = s_b[j];
          const float dx = a.x - pxf;
          const float dy = a.y - pyf;
          const float t2 = splat_power(a.z, a.w, b.x, dx, dy);  // log2(e) power
          const float alpha = fminf(0.99f, b.y * blend_exp2f(t2));
          const float test_t = __builtin_fmaf(-alpha, T, T);  // T (1 - alpha), one rounding
          const bool blend = live && !(t2 > 0.0f) && !(alpha < 1.0f / 255.0f);
          const bool stop = blend && test_t < 0.0001f;
          const bool take = blend && !stop;
          live = live && !stop;
          // colour by fused multiply-adds (no decision depends on it), with
          // the weight alpha T taken as T - T (1 - alpha): the transmittance
          // the splat removes, one subtraction instead of a product and a
          // select (it differs from the product by the rounding of test_t,
          // below 2^-24 T, and the weights of a pixel sum to at most
          // 1 - T_final).  aT is exactly 0 where the pixel does not take the
          // splat; with a non-finite colour in the batch the colour is
          // selected to 0 there as well (0 * inf would be NaN), otherwise
          // c * 0 adds an exact zero.
          const float Tn = take ? test_t : T;
          const float aT = T - Tn;
          const float c2 = NCH > 2 ? s_c[j] : 0.0f;
          if (kFinite) {
            acc[0] = __builtin_fmaf(b.z, aT, acc[0]);
            if (NCH > 1) acc[1] = __builtin_fmaf(b.w, aT, acc[1]);
            if (NCH > 2) acc[2] = __builtin_fmaf(c2, aT, acc[2]);
          } else {
            acc[0] = __builtin_fmaf(take ? b.z : 0.0f, aT, acc[0]);
            if (NCH > 1) acc[1] = __builtin_fmaf(take ? b.w : 0.0f, aT, acc[1]);
            if (NCH > 2) acc[2] = __builtin_fmaf(take ? c2 : 0.0f, aT, acc[2]);
          }
          if (kMetric && take && count_metric && s_g[j] < (uint32_t)prm.num_points)
            atomicAdd(&io.metric_count[s_g[j]], 1);
          T = Tn;
          lg = take ? u + 1 : lg;
          if (kIters) iters = stop ? (uint32_t)(jj + 1) : iters;
        }
        last = lg ? (uint32_t)(base + j0 + lg) : last;
        if (__ballot(live) == 0ull) break;  // uniform
      }
    };
    if (__ballot(live) != 0ull) {  // wave-uniform
      if (colours_finite)
        walk(FiniteTag<true>{});
      else
        walk(FiniteTag<false>{});
    }
    done = live ? 0 : 1;
    // the next round's __syncthreads_count is the barrier before its staging
    // overwrites the batch; after the last round the batch is not read again
  }
  if (inside) {
    io.final_t[pix] = T;
    io.n_contrib[pix] = last;
    if (kIters) io.n_iter[pix] = iters ? iters : (uint32_t)n;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      io.pixel_colors[(size_t)c * HW + pix] = acc[c];
      io.out_color[(size_t)c * HW + pix] = acc[c] + T * io.background[c];
    }
  }
  const uint32_t m = wave_max_u32(inside ? last : 0u);
  if (lane_id() == 0) s_max[t / kWave] = m;
  __syncthreads();
  if (t == 0) {
    uint32_t mm = s_max[0];
    for (int k = 1; k < 4; ++k) mm = s_max[k] > mm ? s_max[k] : mm;
    io.max_contrib[tile] = mm;
  }
}

constexpr int kGradTerms = 11;
constexpr int kRec = 12;  // per-splat gradient record in LDS (11 terms + 1 pad)
constexpr int kBwdBatch = 64;

// Gradient record terms: 0..3 viewspace (dx, dy, |dx|, |dy|), 4..7 conic and
// opacity, 8..10 colour.
__device__ __forceinline__ void permlane32_swap(float& d, float& s) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(d), __float_as_uint(s), false, false);
  d = __uint_as_float(r[0]);
  s = __uint_as_float(r[1]);
}
__device__ __forceinline__ void permlane16_swap(float& d, float& s) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(d), __float_as_uint(s), false, false);
  d = __uint_as_float(r[0]);
  s = __uint_as_float(r[1]);
}

// Sums the 11 terms over the 64 lanes and writes them into rec[0..11].
// Stage 1 swaps the upper half of term 2i with the lower half of term 2i+1
// (v_permlane32_swap), so one add halves two terms at once: u[i] holds term 2i
// in lanes 0-31 and term 2i+1 in lanes 32-63.  Stage 2 does the same across
// odd/even 16-lane rows (v_permlane16_swap): row r of w[m] then holds term
// 4m + {0,2,1,3}[r].  Stage 3 sums each 16-lane row with four DPP adds; lane 15
// of each row holds its row's term.
__device__ __forceinline__ void wave_reduce_terms(float (&v)[kGradTerms], float* rec, int l) {
  float u[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    float d = v[2 * i];
    float s = (2 * i + 1 < kGradTerms) ? v[2 * i + 1] : 0.0f;
    permlane32_swap(d, s);
    u[i] = d + s;
  }
  float w[3];
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    float d = u[2 * m], s = u[2 * m + 1];
    permlane16_swap(d, s);
    w[m] = d + s;
  }
#pragma unroll
  for (int m = 0; m < 3; ++m) {
    w[m] += dpp_mov<0xB1>(w[m]);
    w[m] += dpp_mov<0x4E>(w[m]);
    w[m] += dpp_mov<0x114>(w[m]);
    w[m] += dpp_mov<0x118>(w[m]);
    // the sums are formed here, by every lane: sunk into the lane-15 branch
    // below, the last add could not take its DPP operand directly (a zeroed
    // register, a DPP move and a plain add instead of one DPP add)
    asm volatile("" : "+v"(w[m]));
  }
  if ((l & 15) == 15) {
    const int r = l >> 4;
    const int t = ((r & 1) << 1) | (r >> 1);
#pragma unroll
    for (int m = 0; m < 3; ++m) rec[4 * m + t] = w[m];
  }
}

// Gradient terms of one splat for the lane's four pixels (one per 16x4
// strip), accumulated into v.  The blend decisions repeat the forward's
// operations exactly (same power, exp and thresholds), so T recovery and the
// set of contributing splats match it.  (The hardware exp2 with an exact
// fallback next to the thresholds measured slower: v_exp_f32 issues at a
// quarter of the rate and the threshold test costs what it saves.)
//
// Per pixel the colour behind the splat enters only through
// SdL = T_final * (bg . dL) + sum_c S_c dL_c (S_c: colour accumulated behind
// the splat), so one scalar is carried instead of S_c:
//   dL/dalpha = T_j (col . dL) - SdL / (1 - alpha),  SdL += alpha T_j (col . dL).
// With w = G o dL/dalpha and h = (a W/2, b W/2, c H/2, b H/2) from the conic
// (a, b, c):  d/dmean2d = -w (h.x dx + h.y dy, h.z dy + h.w dx),
// d/dconic = -w/2 (dx^2, dx dy, dy^2), d/dopacity = G dL/dalpha.  The
// pixels' sums are taken without the splat's factor o (-o, -o/2), which
// multiplies each sum once when the record is flushed.
//
// kSafe = false is the fast form: the terms of pixels that do not blend the
// splat are driven to exact zeros by three selects, which needs every operand
// finite (the caller checks the splat records, the loss gradients and the
// carried T and SdL).
// kSafe = true selects every accumulated term, so non-finite values reach only
// pixels that blend the splat, as in the per-pixel definition.  Returns
// whether any pixel of the wave blends the splat (wave-uniform); v is left
// untouched otherwise.
template <int NCH, bool kSafe>
__device__ __forceinline__ bool bwd_splat_terms(const float4 a, const float4 b, const float4 cu,
                                                const float4 h, const int jj, const float pxf,
                                                const float pyf0, const uint32_t reach,
                                                const int (&nc)[4], const int (&nc_max)[4],
                                                float (&T)[4],
                                                float (&SdL)[4], const float (&dL)[4][3],
                                                float (&v)[kGradTerms]) {
  bool any = false;
  const float dx = a.x - pxf;
  const float dxdx = dx * dx;
  // the forward's base-2 exponent (a.z, a.w, b.x hold the coefficients of
  // splat_log2_coeffs), with its per-splat parts kept for the four strips
  const float Bdx = a.w * dx;
  const float Adxdx = (a.z * dx) * dx;
  const float Cc = b.x;
  // the means2d terms' parts in dx, the same for the lane's four strips
  const float hxdx = h.x * dx, hwdx = h.w * dx;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (jj >= nc_max[k]) continue;  // every pixel of the strip ends before this splat
    if (!((reach >> k) & 1u)) continue;  // outside the splat's rows (scalar test)
    const float dy = a.y - (pyf0 + (float)(4 * k));
    const float t2 = splat_power_rows(Bdx, Adxdx, Cc, dy);
    const float G = blend_exp2f(t2);
    const float oG = b.y * G;
    const float alpha = fminf(0.99f, oG);
    const bool act = jj < nc[k] && !(t2 > 0.0f) && !(alpha < 1.0f / 255.0f);
    if (__ballot(act) == 0ull) continue;  // wave-uniform
    any = true;
    // 1/(1-alpha) by the hardware reciprocal (1 ulp): the backward takes no
    // decision from T, so IEEE division is not needed here.
    const float rci = __builtin_amdgcn_rcpf(1.0f - alpha);
    const float Tp = T[k];
    // alpha T_j; in the fast form as T_j - T_{j+1} = T_{j+1} / (1 - alpha) -
    // T_{j+1}, the transmittance the splat removes (exactly 0 where the pixel
    // does not blend it), and T_j = T_{j+1} + that, so T is updated in place
    const float aTf = act ? __builtin_fmaf(Tp, rci, -Tp) : 0.0f;
    const float Tj = kSafe ? (act ? Tp * rci : Tp) : Tp + aTf;
    T[k] = Tj;
    {
#pragma clang fp contract(fast)
      const float aT = kSafe ? (act ? alpha * Tj : 0.0f) : aTf;
      const float col[3] = {b.z, b.w, cu.w};
      float cdl = col[0] * dL[k][0];
#pragma unroll
      for (int c = 1; c < NCH; ++c) cdl += col[c] * dL[k][c];
      const float dL_dalpha = Tj * cdl - rci * SdL[k];
      if (kSafe) {
        SdL[k] += act ? aT * cdl : 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) v[8 + c] += act ? aT * dL[k][c] : 0.0f;
      } else {
        SdL[k] += aT * cdl;
#pragma unroll
        for (int c = 0; c < NCH; ++c) v[8 + c] += aT * dL[k][c];
      }
      const bool geo = act && !(oG > 0.99f);
      const float gm = geo ? G : 0.0f;
      // q = G dL/dalpha is the opacity term.  w = o q; the splat's factor
      // -o/2 (cu.z) is applied when its record is flushed, so here the conic
      // terms are q (dx^2, dx dy, dy^2) and the means2d terms
      // q (h.x dx + h.y dy, h.z dy + h.w dx) and their magnitudes.
      const float qg = gm * dL_dalpha;
      const float mx = h.x * dx + h.y * dy;
      const float my = h.z * dy + h.w * dx;
      const float qdy = qg * dy;
      if (kSafe) {
        const float t[8] = {qg * mx,   qg * my,   fabsf(qg) * fabsf(mx), fabsf(qg) * fabsf(my),
                            qg * dxdx, qdy * dx,  qdy * dy,              qg};
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] += geo ? t[i] : 0.0f;
      } else {
        // the terms linear in qg are summed as sum(qg) and sum(qg dy) here
        // (v[7], v[5]) and formed from them once per splat below; the
        // magnitudes and the dy^2 term need each strip's own factor
        const float mxs = __builtin_fmaf(h.y, dy, hxdx);
        const float mys = __builtin_fmaf(h.z, dy, hwdx);
        v[2] = __builtin_fmaf(fabsf(qg), fabsf(mxs), v[2]);
        v[3] = __builtin_fmaf(fabsf(qg), fabsf(mys), v[3]);
        v[5] += qdy;
        v[6] = __builtin_fmaf(qdy, dy, v[6]);
        v[7] += qg;
      }
    }
  }
  if (!kSafe && any) {  // wave-uniform
    const float sq = v[7], sqdy = v[5];
    v[0] = __builtin_fmaf(h.y, sqdy, hxdx * sq);  // sum qg (h.x dx + h.y dy)
    v[1] = __builtin_fmaf(h.z, sqdy, hwdx * sq);  // sum qg (h.z dy + h.w dx)
    v[4] = dxdx * sq;                             // sum qg dx^2
    v[5] = dx * sqdy;                             // sum qg dx dy
  }
  return any;
}

// Splats lo+cnt-1 .. lo of the staged batch, back to front: per splat the
// gradient terms of the lane's pixels, then (when any pixel blends it) the
// wave reduction into the splat's LDS record.  The accumulators live for one
// splat and start at -0.0 (-0 + x == x exactly, so the first add folds away
// and nothing is carried or cleared between splats).
template <int NCH, bool kSafe>
__device__ __forceinline__ void bwd_batch(const float4* s_a, const float4* s_b, const float4* s_h,
                                          const float4* s_cull, float* s_rec, const int lo,
                                          const int cnt, const int l, const float pxf,
                                          const float pyf0, const int (&nc)[4],
                                          const int (&nc_max)[4], float (&T)[4], float (&SdL)[4],
                                          const float (&dL)[4][3]) {
  for (int j = cnt - 1; j >= 0; --j) {
    const float4 a = s_a[j];
    const float4 b = s_b[j];
    const float4 hh = s_h[j];
    const float4 cu = s_cull[j];
    // strips inside the splat's row extent, one bit each (the same for every
    // lane: moved to a scalar register so the strip tests are scalar)
    const uint32_t reach = __builtin_amdgcn_readfirstlane(__float_as_uint(cu.x));
    float v[kGradTerms];
#pragma unroll
    for (int k = 0; k < kGradTerms; ++k) v[k] = -0.0f;
    if (bwd_splat_terms<NCH, kSafe>(a, b, cu, hh, lo + j, pxf, pyf0, reach, nc, nc_max, T, SdL, dL,
                                    v))
      wave_reduce_terms(v, s_rec + j * kRec, l);
  }
}

// One wavefront per 16x16 tile; lane l owns the pixels (col l&15, row 4k +
// l/16), k = 0..3, one in each 16x4 strip.
template <int NCH>
__global__ void __launch_bounds__(64, 5)
raster_bwd_kernel(const fgs_raster_params prm, const fgs_raster_bwd_io io, RasterShape sh) {
  __shared__ float4 s_a[kBwdBatch];
  __shared__ float4 s_b[kBwdBatch];
  __shared__ float4 s_h[kBwdBatch];     // conic scaled by (W/2, H/2)
  __shared__ float4 s_cull[kBwdBatch];  // (strips reached as bits, -, -opacity/2, colour 3)
  __shared__ uint32_t s_g[kBwdBatch];
  __shared__ float s_rec[kBwdBatch * kRec];
  const int tile = io.tile_order ? (int)io.tile_order[blockIdx.x] : (int)blockIdx.x;
  if (tile < 0 || tile >= sh.gx * sh.gy) return;  // uniform; a permutation never takes it
  const int tx = tile % sh.gx, ty = tile / sh.gx;
  const int l = (int)threadIdx.x;
  const int px = tx * kTile + (l & 15);
  const int row0 = ty * kTile + (l >> 4);
  const size_t HW = (size_t)sh.W * (size_t)sh.H;
  uint32_t end = io.ranges[2 * tile + 1];
  if ((int64_t)end > prm.list_len) end = (uint32_t)prm.list_len;
  uint32_t start = io.ranges[2 * tile];
  if (start > end) start = end;
  int last = (int)io.max_contrib[tile];
  if (last > (int)(end - start)) last = (int)(end - start);
  if (last <= 0) return;  // uniform per workgroup
  const int P = prm.num_points;
  int nc[4];
  float T[4], SdL[4], dL[4][3];
  bool lane_finite = true;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int py = row0 + 4 * k;
    const bool inside = px < sh.W && py < sh.H;
    const size_t pix = inside ? (size_t)py * sh.W + px : 0;
    nc[k] = inside ? (int)io.n_contrib[pix] : 0;
    T[k] = inside ? io.final_t[pix] : 0.0f;
    float bgd = 0.0f;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      dL[k][c] = (inside && c < NCH) ? io.dL_dout_color[(size_t)c * HW + pix] : 0.0f;
      lane_finite = lane_finite && __builtin_isfinite(dL[k][c]);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) bgd += io.background[c] * dL[k][c];
    SdL[k] = T[k] * bgd;
    lane_finite = lane_finite && __builtin_isfinite(SdL[k]) && __builtin_isfinite(T[k]);
  }
  const bool tile_finite = __ballot(!lane_finite) == 0ull;
  // per strip, the largest contributor count of its pixels: splats at or
  // beyond it reach no pixel of the strip (wave-uniform)
  int nc_max[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    nc_max[k] = __builtin_amdgcn_readfirstlane((int)wave_max_u32((uint32_t)nc[k]));
  const float pxf = (float)px;
  const float pyf0 = (float)row0;
  const float ty0 = (float)(ty * kTile);
  const float hx = 0.5f * (float)sh.W;
  const float hy = 0.5f * (float)sh.H;
  const int rounds = (last + kBwdBatch - 1) / kBwdBatch;
  for (int r = 0; r < rounds; ++r) {
    const int hi = last - r * kBwdBatch;
    const int lo = hi > kBwdBatch ? hi - kBwdBatch : 0;
    const int cnt = hi - lo;
    bool fin = true;
    if (l < cnt) {
      const uint32_t g = io.point_list[start + lo + l];
      float4 a, b;
      float c;
      stage_splat<NCH>(g, (uint32_t)P, io.means2d, io.colors, prm.num_channels, io.conic_opacity,
                       a, b, c);
      const float4 hh = make_float4(a.z * hx, a.w * hx, b.x * hy, a.w * hy);
      // the exponent's base-2 coefficients, as the forward stages them
      const float3 k2 = splat_log2_coeffs(a.z, a.w, b.x);
      s_a[l] = make_float4(a.x, a.y, k2.x, k2.y);
      s_b[l] = make_float4(k2.z, b.y, b.z, b.w);
      s_h[l] = hh;
      s_g[l] = g;
      const float2 cu = splat_rows(a.y, a.z, a.w, b.x, b.y);
      fin = __builtin_isfinite(a.x) && __builtin_isfinite(a.y) &&
                       __builtin_isfinite(hh.x) && __builtin_isfinite(hh.y) &&
                       __builtin_isfinite(hh.z) && __builtin_isfinite(hh.w) &&
                       __builtin_isfinite(k2.x) && __builtin_isfinite(k2.y) &&
                       __builtin_isfinite(k2.z) && __builtin_isfinite(b.y) &&
                       __builtin_isfinite(b.z) && __builtin_isfinite(b.w) && __builtin_isfinite(c);
      // the strips k (rows ty0 + 4k .. + 3) the row extent reaches
      uint32_t reach = 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float strip_lo = ty0 + (float)(4 * k);
        if (cu.y >= strip_lo && cu.x <= strip_lo + 3.0f) reach |= 1u << k;
      }
      s_cull[l] = make_float4(__uint_as_float(reach), 0.0f, -0.5f * b.y, c);
    }
#pragma unroll
    for (int i = 0; i < kRec; ++i) s_rec[i * kBwdBatch + l] = 0.0f;
    // The fast form needs finite operands: the tile's loss gradients, every
    // splat record of the batch and the carried pixel state (an infinite
    // colour makes SdL infinite for the splats in front of it).
    bool ok = fin;
#pragma unroll
    for (int k = 0; k < 4; ++k) ok = ok && __builtin_isfinite(T[k]) && __builtin_isfinite(SdL[k]);
    const bool fast = tile_finite && __ballot(!ok) == 0ull;
    __syncthreads();
    if (fast)
      bwd_batch<NCH, false>(s_a, s_b, s_h, s_cull, s_rec, lo, cnt, l, pxf, pyf0, nc, nc_max,
                            T, SdL, dL);
    else
      bwd_batch<NCH, true>(s_a, s_b, s_h, s_cull, s_rec, lo, cnt, l, pxf, pyf0, nc, nc_max,
                           T, SdL, dL);
    __syncthreads();
    // Flush: lane l takes term ft = l & 15 of splats 4i + (l >> 4), so every
    // lane keeps one term (its array, row stride, column and factor) for the
    // whole flush, and one atomic instruction covers the rows of four splats.
    // Terms 0..3 are viewspace, 4..7 conic and opacity, 8.. colour (rows of
    // 4, 4 and num_channels floats).
    const int ft = l & 15, fs0 = l >> 4;
    const bool ft_ok = ft < 8 + NCH;
    float* const fbase = ft < 4 ? io.dL_dviewspace : (ft < 8 ? io.dL_dconic_opacity : io.dL_dcolors);
    const uint32_t fstride = ft < 8 ? 4u : (uint32_t)prm.num_channels;
    const uint32_t fcol = (uint32_t)(ft < 4 ? ft : (ft < 8 ? ft - 4 : ft - 8));
#pragma unroll 4
    for (int i = 0; i < (cnt + 3) / 4; ++i) {
      const int s = 4 * i + fs0;
      if (s < cnt && ft_ok) {
        // the splat's factor on its geometry terms: -o for the means2d
        // terms, |o| for their magnitudes, -o/2 for the conic's
        const float hz = s_cull[s].z;  // -o/2
        const float f = ft >= 7 ? 1.0f : (ft < 4 ? (ft < 2 ? 2.0f * hz : fabsf(2.0f * hz)) : hz);
        const float w = s_rec[s * kRec + ft] * f;
        const uint32_t g = s_g[s];
        if (w != 0.0f && g < (uint32_t)P)
          unsafeAtomicAdd(fbase + ((uint64_t)g * fstride + fcol), w);
      }
    }
    __syncthreads();
  }
}

// Launch order of the backward's tiles, heaviest first: a counting sort of
// the tiles by max_contrib (the length of each tile's walk) into 1024 buckets
// between 0 and the largest value, largest bucket first.  Per-tile work varies
// several-fold, and workgroups start in index order, so in index order the
// last heavy tiles run alone at the end of the launch; heaviest first, light
// tiles fill that tail.  Tiles of one bucket leave in no fixed order (LDS
// atomics): only the schedule depends on it.
constexpr int kOrderThreads = 1024;
constexpr int kOrderBuckets = 1024;
constexpr int kOrderCached = 8;  // values kept in registers per thread (8192 tiles)

__device__ __forceinline__ void tile_order_body(const uint32_t* __restrict__ max_contrib, int T,
                                                uint32_t* __restrict__ order) {
  __shared__ uint32_t s_cnt[kOrderBuckets];
  __shared__ uint32_t s_tmp[kOrderThreads / kWave + 1];
  __shared__ uint32_t s_max;
  const int t = (int)threadIdx.x;
  uint32_t mc[kOrderCached];
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < kOrderCached; ++c) {
    const int i = t + c * kOrderThreads;
    mc[c] = i < T ? max_contrib[i] : 0u;
    m = mc[c] > m ? mc[c] : m;
  }
  for (int i = t + kOrderCached * kOrderThreads; i < T; i += kOrderThreads)
    m = max_contrib[i] > m ? max_contrib[i] : m;
  m = wave_max_u32(m);
  if (t == 0) s_max = 0u;
  s_cnt[t] = 0u;
  __syncthreads();
  if (lane_id() == 0) atomicMax(&s_max, m);
  __syncthreads();
  // bucket 0 holds the largest values; the float scale only has to be monotone
  const float sc = s_max ? (float)(kOrderBuckets - 1) / (float)s_max : 0.0f;
  auto bucket = [sc](uint32_t v) -> uint32_t {
    const uint32_t q = (uint32_t)((float)v * sc);
    return (uint32_t)(kOrderBuckets - 1) - (q < (uint32_t)(kOrderBuckets - 1) ? q : (uint32_t)(kOrderBuckets - 1));
  };
#pragma unroll
  for (int c = 0; c < kOrderCached; ++c)
    if (t + c * kOrderThreads < T) atomicAdd(&s_cnt[bucket(mc[c])], 1u);
  for (int i = t + kOrderCached * kOrderThreads; i < T; i += kOrderThreads)
    atomicAdd(&s_cnt[bucket(max_contrib[i])], 1u);
  __syncthreads();
  const uint32_t first = block_excl_scan(s_cnt[t], s_tmp, nullptr);
  s_cnt[t] = first;
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kOrderCached; ++c) {
    const int i = t + c * kOrderThreads;
    if (i < T) order[atomicAdd(&s_cnt[bucket(mc[c])], 1u)] = (uint32_t)i;
  }
  for (int i = t + kOrderCached * kOrderThreads; i < T; i += kOrderThreads)
    order[atomicAdd(&s_cnt[bucket(max_contrib[i])], 1u)] = (uint32_t)i;
}

// The backward's preparation in one launch: workgroup 0 sorts the tile order
// (when order is set) while the others clear the atomically accumulated
// gradients.
__global__ void __launch_bounds__(kOrderThreads)
bwd_prep_kernel(FillSpans f, const uint32_t* __restrict__ max_contrib, int T,
                uint32_t* __restrict__ order) {
  const int first_fill = order ? 1 : 0;
  if ((int)blockIdx.x < first_fill) {
    tile_order_body(max_contrib, T, order);
    return;
  }
  fill_spans_body(f, (int64_t)(blockIdx.x - first_fill) * blockDim.x + threadIdx.x,
                  (int64_t)(gridDim.x - first_fill) * blockDim.x);
}

// dL/dmeans2d equals the first two viewspace terms: copied after the
// accumulation instead of being accumulated twice.
__global__ void __launch_bounds__(256)
copy_means2d_grad_kernel(const float* __restrict__ vsp, float* __restrict__ dmeans2d, int P) {
  const int g = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (g >= P) return;
  const float4 v = *reinterpret_cast<const float4*>(vsp + 4 * (size_t)g);
  *reinterpret_cast<float2*>(dmeans2d + 2 * (size_t)g) = make_float2(v.x, v.y);
}

// The copy, when the caller asks for dL_dmeans2d (a NULL one is read in place
// from dL_dviewspace).
static int32_t copy_means2d_grad(const fgs_raster_bwd_io* io, int P, hipStream_t st) {
  if (!io->dL_dmeans2d || P <= 0) return check_launch("rasterize_bwd");
  hipLaunchKernelGGL(copy_means2d_grad_kernel, dim3(ceil_div_u(P, 256)), dim3(256), 0, st,
                     io->dL_dviewspace, io->dL_dmeans2d, P);
  return check_launch("copy_means2d_grad_kernel");
}

}  // namespace fgs

using namespace fgs;

template <int NCH>
static void launch_fwd(int mode, dim3 grid, dim3 block, hipStream_t st,
                       const fgs_raster_params& p, const fgs_raster_fwd_io& io, RasterShape sh) {
  switch (mode) {
    case 0: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 0>), grid, block, 0, st, p, io, sh); break;
    case 1: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 1>), grid, block, 0, st, p, io, sh); break;
    case 2: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 2>), grid, block, 0, st, p, io, sh); break;
    case 3: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 3>), grid, block, 0, st, p, io, sh); break;
    case 4: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 4>), grid, block, 0, st, p, io, sh); break;
    case 5: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 5>), grid, block, 0, st, p, io, sh); break;
    case 6: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 6>), grid, block, 0, st, p, io, sh); break;
    default: hipLaunchKernelGGL((raster_fwd_kernel<NCH, 7>), grid, block, 0, st, p, io, sh);
  }
}

static int32_t raster_check(const fgs_raster_params* p, const char* who) {
  if (!p) return set_error(FGS_ERR_INVALID_ARGUMENT, who);
  if (p->image_width <= 0 || p->image_height <= 0 || p->num_channels <= 0 || p->num_tiles < 0 ||
      p->bucket_sum < 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, who);
  return FGS_OK;
}

extern "C" int32_t fgs_rasterize_fwd(const fgs_raster_params* p, const fgs_raster_fwd_io* io,
                                     void* stream) {
  if (raster_check(p, "fgs_rasterize_fwd: bad parameters") != FGS_OK) return FGS_ERR_INVALID_ARGUMENT;
  if (!io) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_fwd: null io");
  const int W = p->image_width, H = p->image_height;
  const int gx = (W + kTile - 1) / kTile, gy = (H + kTile - 1) / kTile;
  int tiles = gx * gy;
  if (p->num_tiles < tiles) tiles = p->num_tiles;
  const int64_t HW = (int64_t)W * H;
  if (!io->ranges || !io->bucket_offsets || !io->means2d || !io->colors || !io->conic_opacity ||
      !io->background || !io->final_t || !io->n_contrib || !io->max_contrib ||
      !io->pixel_colors || !io->out_color || (p->bucket_sum > 0 && !io->bucket_to_tile) ||
      (p->get_flag && (!io->metric_map || (p->num_points > 0 && !io->metric_count))) ||
      (p->write_sampled && p->bucket_sum > 0 && (!io->sampled_t || !io->sampled_ar)))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_fwd: missing tensor");
  hipStream_t st = (hipStream_t)stream;
  const int C = p->num_channels;
  const int NCH = C < 3 ? C : 3;
  // Elements the kernel may leave unwritten are cleared first, in as few
  // fill launches as possible.
  FillSpans f{};
  auto span = [&](void* ptr, int64_t n) {
    if (n <= 0) return;
    if (f.count == kFillSpans) {
      launch_fill_spans(f, st);
      f.count = 0;
    }
    f.p[f.count] = reinterpret_cast<uint32_t*>(ptr);
    f.n[f.count] = n;
    ++f.count;
  };
  if (p->get_flag && p->num_points > 0) span(io->metric_count, p->num_points);
  if (p->write_sampled && p->bucket_sum > 0) {
    span(io->sampled_t, p->bucket_sum * 256);
    span(io->sampled_ar, p->bucket_sum * 256 * C);
  }
  if (C > 3) {
    span(io->pixel_colors + 3 * HW, (C - 3) * HW);
    span(io->out_color + 3 * HW, (C - 3) * HW);
  }
  // Every tile the kernel renders writes its own buckets (bucket_offsets
  // partitions [0, B)), so bucket_to_tile needs clearing only when some tiles
  // are not rendered; entries past B (a caller's upper bound) are its to cut.
  if (p->bucket_sum > 0 && tiles < p->num_tiles) span(io->bucket_to_tile, p->bucket_sum);
  if (tiles < gx * gy) {
    // Pixels of tiles beyond num_tiles are never rendered: clear them.
    span(io->final_t, HW);
    span(io->n_contrib, HW);
    if (io->n_iter) span(io->n_iter, HW);
    span(io->pixel_colors, C * HW);
    span(io->out_color, C * HW);
  }
  if (p->num_tiles > tiles) span(io->max_contrib + tiles, p->num_tiles - tiles);
  if (f.count) launch_fill_spans(f, st);
  if (tiles == 0) return check_launch("rasterize_fwd");
  RasterShape sh{W, H, gx, gy};
  const int mode = (p->write_sampled && p->bucket_sum > 0 ? 1 : 0) | (p->get_flag ? 2 : 0) |
                   (io->n_iter ? 4 : 0);
  const dim3 grid(tiles), block(256);
  if (const int32_t e = launch_mark(kLaunchRasterFwd, st, 0)) return e;
  if (NCH == 3) launch_fwd<3>(mode, grid, block, st, *p, *io, sh);
  else if (NCH == 2) launch_fwd<2>(mode, grid, block, st, *p, *io, sh);
  else launch_fwd<1>(mode, grid, block, st, *p, *io, sh);
  if (check_launch("raster_fwd_kernel") != FGS_OK) return FGS_ERR_LAUNCH;
  return launch_mark(kLaunchRasterFwd, st, 1);
}

// Grids above this many tiles run in index order (one workgroup sorts the
// order; at 2^16 tiles, a 4096x4096 image, that is 64 tiles per thread).
constexpr int kMaxOrderedTiles = 1 << 16;

extern "C" int32_t fgs_rasterize_bwd(const fgs_raster_params* p, const fgs_raster_bwd_io* io,
                                     void* stream) {
  if (raster_check(p, "fgs_rasterize_bwd: bad parameters") != FGS_OK) return FGS_ERR_INVALID_ARGUMENT;
  if (!io) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_bwd: null io");
  const int W = p->image_width, H = p->image_height;
  const int gx = (W + kTile - 1) / kTile, gy = (H + kTile - 1) / kTile;
  int tiles = gx * gy;
  if (p->num_tiles < tiles) tiles = p->num_tiles;
  const int P = p->num_points;
  const int C = p->num_channels;
  if (P > 0 && (!io->dL_dcolors || !io->dL_dconic_opacity || !io->dL_dviewspace))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_bwd: missing gradient tensor");
  hipStream_t st = (hipStream_t)stream;
  // the atomically accumulated gradients start at zero
  FillSpans f{};
  f.p[0] = reinterpret_cast<uint32_t*>(io->dL_dcolors);
  f.n[0] = (int64_t)C * P;
  f.p[1] = reinterpret_cast<uint32_t*>(io->dL_dconic_opacity);
  f.n[1] = 4 * (int64_t)P;
  f.p[2] = reinterpret_cast<uint32_t*>(io->dL_dviewspace);
  f.n[2] = 4 * (int64_t)P;
  f.count = P > 0 ? 3 : 0;
  f.value = 0u;
  if (P == 0) return check_launch("rasterize_bwd");
  const int64_t fill_words = (int64_t)(C + 8) * P;
  int64_t fill_blocks = (fill_words / 4 + kOrderThreads - 1) / kOrderThreads;
  if (fill_blocks < 1) fill_blocks = 1;
  if (fill_blocks > 512) fill_blocks = 512;
  if (tiles == 0) {
    hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)fill_blocks), dim3(kOrderThreads), 0, st, f,
                       nullptr, 0, nullptr);
    return copy_means2d_grad(io, P, st);
  }
  if (!io->ranges || !io->point_list || !io->means2d || !io->colors || !io->conic_opacity ||
      !io->background || !io->final_t || !io->n_contrib || !io->max_contrib || !io->dL_dout_color)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_bwd: missing tensor");
  const int NCH = C < 3 ? C : 3;
  RasterShape sh{W, H, gx, gy};
  fgs_raster_bwd_io kio = *io;
  if (!(kio.tile_order && tiles <= kMaxOrderedTiles)) kio.tile_order = nullptr;  // index order
  hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)(fill_blocks + (kio.tile_order ? 1 : 0))),
                     dim3(kOrderThreads), 0, st, f, io->max_contrib, tiles, kio.tile_order);
  if (const int32_t e = launch_mark(kLaunchRasterBwd, st, 0)) return e;
  if (NCH == 3)
    hipLaunchKernelGGL(raster_bwd_kernel<3>, dim3(tiles), dim3(64), 0, st, *p, kio, sh);
  else if (NCH == 2)
    hipLaunchKernelGGL(raster_bwd_kernel<2>, dim3(tiles), dim3(64), 0, st, *p, kio, sh);
  else
    hipLaunchKernelGGL(raster_bwd_kernel<1>, dim3(tiles), dim3(64), 0, st, *p, kio, sh);
  if (check_launch("raster_bwd_kernel") != FGS_OK) return FGS_ERR_LAUNCH;
  if (const int32_t e = launch_mark(kLaunchRasterBwd, st, 1)) return e;
  return copy_means2d_grad(io, P, st);
}
