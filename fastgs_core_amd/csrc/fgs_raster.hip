// fgs_raster.hip -- tile rasterization forward and backward (gfx950, wave64).
//
// Forward (semantics of fastgs_rasterize.metal:25-159): one 256-thread
// workgroup per 16x16 tile, one pixel per thread, wavefront w owning rows
// 4w..4w+3.  The tile's sorted splat list is streamed through LDS in batches
// of 256 (each thread stages one splat: 2D mean, conic, opacity, colour and
// opacity), then every pixel blends the batch front to back.  Pixels stop at
// T < 1e-4; a wavefront whose pixels have all stopped skips the blend loop,
// and the workgroup leaves as soon as every pixel has stopped
// (__syncthreads_count).  (Culling by row extent or by a power threshold
// measured slower here: the batch barrier makes the block wait for its
// busiest wavefront, and staging the culling data costs more than it saves.)
//
// Backward (per-(pixel, splat) semantics of
// fastgs_rasterize_backward.metal:24-278): one wavefront per tile, each lane
// owning four pixels (one per 16x4 strip); splats are walked back to front
// from the tile's max_contrib in LDS batches of 64.  Each pixel recovers
// T_j = T_{j+1} / (1 - alpha_j) starting from final_T and carries the colour
// accumulated behind the splat, so no per-bucket sampled state is needed.
// Strips a splat cannot reach (conservative alpha >= 1/255 extent) are skipped
// wave-uniformly and exp is skipped below a per-splat power threshold.  Per
// splat, the lane's four pixel terms are summed in registers and the 11
// gradient terms are reduced across the wave with DPP adds into LDS; each
// batch is flushed with one set of global float atomics per (splat, tile).
#include "fgs_common.hpp"

// Backward tuning knobs (results are identical either way): skip strips a
// splat cannot reach, and skip exp below the splat's power threshold.
#ifndef FGS_BWD_STRIP_CULL
#define FGS_BWD_STRIP_CULL 1
#endif
#ifndef FGS_BWD_POWER_CULL
#define FGS_BWD_POWER_CULL 1
#endif

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

// Power below which a splat of opacity o cannot reach alpha >= 1/255:
// o * exp(power) >= 1/255 needs power >= -ln(255 o); 0.01 of margin covers the
// rounding of exp and of the hardware log.  +inf when o < 0.999/255 (alpha <= o: never
// contributes), -inf for a NaN opacity (no culling).
__device__ __forceinline__ float splat_power_min(float o) {
  if (!(o == o)) return -__builtin_huge_valf();
  if (!(255.0f * o >= 0.999f)) return __builtin_huge_valf();
  return -__logf(255.0f * o) - 0.01f;
}

// Culling data of a splat: rows [lo, hi] outside which no
// pixel can reach alpha >= 1/255, and a power threshold below which alpha <
// 1/255 for certain.  alpha >= 1/255 needs o*exp(power) >= 1/255, i.e.
// q(d) = d^T Conic d <= tau = 2 ln(255 o).  The row extent of {q <= tau} is
// sqrt(tau * a / det); it is widened to tau' = 1.1 tau + 1 plus 2 pixels.
// Ill-conditioned or non-positive conics and NaN opacities are not culled.
__device__ __forceinline__ float4 splat_cull(float x, float y, float a, float b, float c, float o) {
  const float inf = __builtin_huge_valf();
  float4 r = make_float4(-inf, inf, -inf, 0.f);  // (row_lo, row_hi, power_min, -)
  if (!(o == o)) return r;
  if (!(255.0f * o >= 0.999f)) {  // alpha <= o < 1/255: never contributes
    r.x = inf;
    r.y = -inf;
    r.z = inf;
    return r;
  }
  const float tau = 2.0f * __logf(255.0f * o);
  r.z = splat_power_min(o);
  const float det = a * c - b * b;
  if (!(a > 0.f) || !(c > 0.f) || !(det > 1e-3f * a * c)) return r;
  const float tq = fmaxf(tau, 0.0f) * 1.1f + 1.0f;
  const float hy = __builtin_sqrtf(tq * a / det) + 2.0f;
  r.x = y - hy;
  r.y = y + hy;
  (void)x;
  return r;
}

template <int NCH>
__global__ void __launch_bounds__(256)
raster_fwd_kernel(const fgs_raster_params prm, const fgs_raster_fwd_io io, RasterShape sh) {
  __shared__ float4 s_a[256];
  __shared__ float4 s_b[256];
  __shared__ float s_c[256];
  __shared__ uint32_t s_g[256];
  __shared__ uint32_t s_max[4];
  const int tile = (int)blockIdx.x;
  const int tx = tile % sh.gx, ty = tile / sh.gx;
  const int t = (int)threadIdx.x;
  const int lx = t & 15, ly = t >> 4;
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
  const bool count_metric = prm.get_flag && inside && io.metric_map[pix] == 1;
  const float pxf = (float)px, pyf = (float)py;
  float T = 1.0f;
  uint32_t contributor = 0, last = 0;
  float acc[3] = {0.0f, 0.0f, 0.0f};
  int done = inside ? 0 : 1;
  const int rounds = (n + 255) / 256;
  for (int r = 0; r < rounds; ++r) {
    if (__syncthreads_count(done) == 256) break;
    const int base = r * 256;
    if (base + t < n) {
      const uint32_t g = io.point_list[start + base + t];
      float4 a, b;
      float c;
      stage_splat<NCH>(g, (uint32_t)prm.num_points, io.means2d, io.colors, prm.num_channels, io.conic_opacity, a, b, c);
      s_a[t] = a;
      s_b[t] = b;
      s_c[t] = c;
      s_g[t] = g;
    }
    __syncthreads();
    const int cnt = (n - base) < 256 ? (n - base) : 256;
    if (!done) {
      for (int j = 0; j < cnt; ++j) {
        const int jj = base + j;
        if (prm.write_sampled && (jj & 31) == 0) {
          const size_t bk = (size_t)bbm0 + (size_t)(jj >> 5);
          if ((int64_t)bk < prm.bucket_sum) {
            io.sampled_t[bk * 256 + t] = T;
#pragma unroll
            for (int c = 0; c < NCH; ++c)
              io.sampled_ar[bk * (size_t)prm.num_channels * 256 + (size_t)c * 256 + t] = acc[c];
          }
        }
        contributor++;
        const float4 a = s_a[j];
        const float4 b = s_b[j];
        const float dx = a.x - pxf;
        const float dy = a.y - pyf;
        const float power = -0.5f * (a.z * dx * dx + b.x * dy * dy) - a.w * dx * dy;
        if (power > 0.0f) continue;
        const float alpha = fminf(0.99f, b.y * det_expf(power));
        if (alpha < 1.0f / 255.0f) continue;
        const float test_t = T * (1.0f - alpha);
        if (test_t < 0.0001f) {
          done = 1;
          break;
        }
        acc[0] += b.z * alpha * T;
        if (NCH > 1) acc[1] += b.w * alpha * T;
        if (NCH > 2) acc[2] += s_c[j] * alpha * T;
        if (count_metric && s_g[j] < (uint32_t)prm.num_points)
          atomicAdd(&io.metric_count[s_g[j]], 1);
        T = test_t;
        last = contributor;
      }
    }
    __syncthreads();
  }
  if (inside) {
    io.final_t[pix] = T;
    io.n_contrib[pix] = last;
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
constexpr int kBwdBatch = 64;

// One wavefront per 16x16 tile; lane l owns the pixels (col l&15, row 4k +
// l/16), k = 0..3, one in each 16x4 strip.
template <int NCH>
__global__ void __launch_bounds__(64)
raster_bwd_kernel(const fgs_raster_params prm, const fgs_raster_bwd_io io, RasterShape sh) {
  __shared__ float4 s_a[kBwdBatch];
  __shared__ float4 s_b[kBwdBatch];
  __shared__ float4 s_cull[kBwdBatch];
  __shared__ float s_c[kBwdBatch];
  __shared__ uint32_t s_g[kBwdBatch];
  __shared__ float s_acc[kGradTerms][kBwdBatch];
  const int tile = (int)blockIdx.x;
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
  float T[4], Tf[4], bgd[4], dL[4][3], S[4][3];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int py = row0 + 4 * k;
    const bool inside = px < sh.W && py < sh.H;
    const size_t pix = inside ? (size_t)py * sh.W + px : 0;
    nc[k] = inside ? (int)io.n_contrib[pix] : 0;
    Tf[k] = inside ? io.final_t[pix] : 0.0f;
    T[k] = Tf[k];
    bgd[k] = 0.0f;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      dL[k][c] = (inside && c < NCH) ? io.dL_dout_color[(size_t)c * HW + pix] : 0.0f;
      S[k][c] = 0.0f;
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) bgd[k] += io.background[c] * dL[k][c];
  }
  int ncmax = imax(imax(nc[0], nc[1]), imax(nc[2], nc[3]));
  const float pxf = (float)px;
  const float ddelx_dx = 0.5f * (float)sh.W;
  const float ddely_dy = 0.5f * (float)sh.H;
  const int rounds = (last + kBwdBatch - 1) / kBwdBatch;
  for (int r = 0; r < rounds; ++r) {
    const int hi = last - r * kBwdBatch;
    const int lo = hi > kBwdBatch ? hi - kBwdBatch : 0;
    const int cnt = hi - lo;
    if (l < cnt) {
      const uint32_t g = io.point_list[start + lo + l];
      float4 a, b;
      float c;
      stage_splat<NCH>(g, (uint32_t)P, io.means2d, io.colors, prm.num_channels, io.conic_opacity,
                       a, b, c);
      s_a[l] = a;
      s_b[l] = b;
      s_c[l] = c;
      s_g[l] = g;
      s_cull[l] = splat_cull(a.x, a.y, a.z, a.w, b.x, b.y);
    }
#pragma unroll
    for (int k = 0; k < kGradTerms; ++k) s_acc[k][l] = 0.0f;
    __syncthreads();
    for (int j = cnt - 1; j >= 0; --j) {
      const int jj = lo + j;
      if (__ballot(jj < ncmax) == 0ull) continue;  // no pixel of the tile reaches splat jj
      const float4 a = s_a[j];
      const float4 b = s_b[j];
      const float4 cu = s_cull[j];
      const float cz = s_c[j];
      float v[kGradTerms];
#pragma unroll
      for (int k = 0; k < kGradTerms; ++k) v[k] = 0.0f;
      bool any = false;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float strip_lo = (float)(ty * kTile + 4 * k);
        if (FGS_BWD_STRIP_CULL && !(cu.y >= strip_lo && cu.x <= strip_lo + 3.0f)) continue;
        if (jj >= nc[k]) continue;
        const float pyf = (float)(row0 + 4 * k);
        const float dx = a.x - pxf;
        const float dy = a.y - pyf;
        const float power = -0.5f * (a.z * dx * dx + b.x * dy * dy) - a.w * dx * dy;
        if (power > 0.0f || (FGS_BWD_POWER_CULL && power < cu.z)) continue;
        const float G = det_expf(power);
        const float alpha = fminf(0.99f, b.y * G);
        if (alpha < 1.0f / 255.0f) continue;
        any = true;
        // 1/(1-alpha) by the hardware reciprocal (1 ulp): the backward takes no
        // decision from T, so IEEE division is not needed here.
        const float rci = __builtin_amdgcn_rcpf(1.0f - alpha);
        T[k] = T[k] * rci;
        const float Tj = T[k];
        const float col[3] = {b.z, b.w, cz};
        float dL_dalpha = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          v[8 + c] += alpha * Tj * dL[k][c];
          dL_dalpha += (col[c] * Tj - rci * S[k][c]) * dL[k][c];
          S[k][c] += col[c] * alpha * Tj;
        }
        dL_dalpha += (-Tf[k] * rci) * bgd[k];
        if (!(b.y * G > 0.99f)) {
          const float dL_dG = b.y * dL_dalpha;
          const float gdx = G * dx, gdy = G * dy;
          const float dG_ddelx = -gdx * a.z - gdy * a.w;
          const float dG_ddely = -gdy * b.x - gdx * a.w;
          const float tmp_x = dL_dG * dG_ddelx * ddelx_dx;
          const float tmp_y = dL_dG * dG_ddely * ddely_dy;
          v[0] += tmp_x;
          v[1] += tmp_y;
          v[2] += fabsf(tmp_x);
          v[3] += fabsf(tmp_y);
          v[4] += -0.5f * gdx * dx * dL_dG;
          v[5] += -0.5f * gdx * dy * dL_dG;
          v[6] += -0.5f * gdy * dy * dL_dG;
          v[7] += G * dL_dalpha;
        }
      }
      if (__ballot(any) != 0ull) {
#pragma unroll
        for (int k = 0; k < kGradTerms; ++k) v[k] = wave_sum_lane63(v[k]);
        if (l == kWave - 1) {
#pragma unroll
          for (int k = 0; k < kGradTerms; ++k) s_acc[k][j] = v[k];
        }
      }
    }
    __syncthreads();
    if (l < cnt) {
      float w[kGradTerms];
      bool nz = false;
#pragma unroll
      for (int k = 0; k < kGradTerms; ++k) {
        w[k] = s_acc[k][l];
        nz = nz || (w[k] != 0.0f);
      }
      if (nz && s_g[l] < (uint32_t)P) {
        const size_t g = s_g[l];
        unsafeAtomicAdd(&io.dL_dmeans2d[2 * g + 0], w[0]);
        unsafeAtomicAdd(&io.dL_dmeans2d[2 * g + 1], w[1]);
        unsafeAtomicAdd(&io.dL_dviewspace[4 * g + 0], w[0]);
        unsafeAtomicAdd(&io.dL_dviewspace[4 * g + 1], w[1]);
        unsafeAtomicAdd(&io.dL_dviewspace[4 * g + 2], w[2]);
        unsafeAtomicAdd(&io.dL_dviewspace[4 * g + 3], w[3]);
        unsafeAtomicAdd(&io.dL_dconic_opacity[4 * g + 0], w[4]);
        unsafeAtomicAdd(&io.dL_dconic_opacity[4 * g + 1], w[5]);
        unsafeAtomicAdd(&io.dL_dconic_opacity[4 * g + 2], w[6]);
        unsafeAtomicAdd(&io.dL_dconic_opacity[4 * g + 3], w[7]);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          unsafeAtomicAdd(&io.dL_dcolors[g * (size_t)prm.num_channels + c], w[8 + c]);
      }
    }
    __syncthreads();
  }
}

}  // namespace fgs

using namespace fgs;

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
  // Elements the kernel may leave unwritten are cleared first.
  if (p->get_flag && p->num_points > 0)
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->metric_count), 0u, p->num_points, stream);
  if (p->write_sampled && p->bucket_sum > 0) {
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->sampled_t), 0u, p->bucket_sum * 256, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->sampled_ar), 0u, p->bucket_sum * 256 * C, stream);
  }
  if (C > 3) {
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->pixel_colors) + 3 * HW, 0u, (C - 3) * HW, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->out_color) + 3 * HW, 0u, (C - 3) * HW, stream);
  }
  if (p->bucket_sum > 0)
    fgs_fill_u32(io->bucket_to_tile, 0u, p->bucket_sum, stream);
  if (tiles < gx * gy) {
    // Pixels of tiles beyond num_tiles are never rendered: clear them.
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->final_t), 0u, HW, stream);
    fgs_fill_u32(io->n_contrib, 0u, HW, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->pixel_colors), 0u, C * HW, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->out_color), 0u, C * HW, stream);
  }
  if (p->num_tiles > tiles)
    fgs_fill_u32(io->max_contrib + tiles, 0u, p->num_tiles - tiles, stream);
  if (tiles == 0) return check_launch("rasterize_fwd");
  RasterShape sh{W, H, gx, gy};
  if (NCH == 3)
    hipLaunchKernelGGL(raster_fwd_kernel<3>, dim3(tiles), dim3(256), 0, st, *p, *io, sh);
  else if (NCH == 2)
    hipLaunchKernelGGL(raster_fwd_kernel<2>, dim3(tiles), dim3(256), 0, st, *p, *io, sh);
  else
    hipLaunchKernelGGL(raster_fwd_kernel<1>, dim3(tiles), dim3(256), 0, st, *p, *io, sh);
  return check_launch("raster_fwd_kernel");
}

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
  if (P > 0 && (!io->dL_dmeans2d || !io->dL_dcolors || !io->dL_dconic_opacity || !io->dL_dviewspace))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_bwd: missing gradient tensor");
  hipStream_t st = (hipStream_t)stream;
  if (P > 0) {
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->dL_dmeans2d), 0u, 2 * (int64_t)P, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->dL_dcolors), 0u, (int64_t)C * P, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->dL_dconic_opacity), 0u, 4 * (int64_t)P, stream);
    fgs_fill_u32(reinterpret_cast<uint32_t*>(io->dL_dviewspace), 0u, 4 * (int64_t)P, stream);
  }
  if (tiles == 0 || P == 0) return check_launch("rasterize_bwd");
  if (!io->ranges || !io->point_list || !io->means2d || !io->colors || !io->conic_opacity ||
      !io->background || !io->final_t || !io->n_contrib || !io->max_contrib || !io->dL_dout_color)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_rasterize_bwd: missing tensor");
  const int NCH = C < 3 ? C : 3;
  RasterShape sh{W, H, gx, gy};
  if (NCH == 3)
    hipLaunchKernelGGL(raster_bwd_kernel<3>, dim3(tiles), dim3(64), 0, st, *p, *io, sh);
  else if (NCH == 2)
    hipLaunchKernelGGL(raster_bwd_kernel<2>, dim3(tiles), dim3(64), 0, st, *p, *io, sh);
  else
    hipLaunchKernelGGL(raster_bwd_kernel<1>, dim3(tiles), dim3(64), 0, st, *p, *io, sh);
  return check_launch("raster_bwd_kernel");
}
