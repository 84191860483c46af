// fgs_loss.hip -- fused photometric loss of the training step:
//   L = w_l1 * mean|x - y| + w_ssim * (1 - mean SSIM(x, y))
// over C planes of H x W, SSIM with an 11x11 separable Gaussian window
// (zero padding, per channel), C1 = 0.01^2, C2 = 0.03^2 -- the loss the
// reference's FastGS training scripts put on the rendered image
// (scripts/train_scanner_fastgs.py:911-966), which the rasterizer's
// backward consumes as dL/dout_color.
//
// Both passes use one wavefront per strip of 64 columns x 34 output rows of
// one plane, lane l owning column l.  The wavefront walks the strip's 44
// input rows (5-row halo above and below) top to bottom: each row's 74
// values (5-column halo each side) are staged in LDS (two row buffers; a
// one-wave workgroup needs no barrier between them, only its LDS ordering),
// the lane blurs its column horizontally and keeps the result for the last
// 11 rows in a register ring (rows are taken 11 at a time, so the ring is
// indexed statically); once 11 rows are in, the vertical blur of the ring
// gives one output row.  Input rows are loaded 11 rows before they are
// staged (a second register ring), so a row's load latency overlaps the work
// of the rows before it.
// Forward: the five moments x, y, x^2, y^2, xy are blurred; the SSIM value
// and its partial derivatives with respect to the three blurred moments of x
// (E[x], E[x^2], E[xy]) are written per pixel, and per-strip partial sums of
// SSIM and |x - y| (the latter from the staged centre column) go to a
// partials array that a second kernel reduces in a fixed order
// (deterministic).
//
// Backward: the three partial-derivative maps are blurred the same way
// (the zero-padded symmetric blur is self-adjoint) and combined with x, y:
//   dL/dx = g * (w_l1 sign(x-y) / N - w_ssim / N * (B1 + 2 x B2 + y B3)),
// Bk = blur(dS/dmk), g the upstream scalar gradient (read on the device).
#include "fgs_common.hpp"

namespace fgs {

constexpr int kSW = 64;                // strip width: one column per lane
constexpr int kSH = 34;                // output rows per strip (kRows = 4 x 11)
constexpr int kLR = 5;                 // window radius (11 taps)
constexpr int kRowIn = 2 * kSW;        // staged values per row: 74 used, all lanes write two
constexpr int kRows = kSH + 2 * kLR;   // 44 input rows per strip
static_assert(kRows % 11 == 0, "the row loop takes the rows 11 at a time");

struct LossArgs {
  int C, H, W;
  int strips_x, chunks_y;
  float w_l1, w_ssim;
  float win[11];
};

// Image planes are read and written through raw buffer resources: an
// offset at or past the resource's size reads 0 and drops a store.  The zero
// padding of the window and the pixels past the image edge are therefore
// offsets, not branches, and the rows' loads and stores stay in one
// straight-line stream whose outstanding counts the compiler can track (a
// load behind a lane-masked branch made it wait for every load in flight).
// Plane sizes are checked on the host: H * W * 4 < 2^31.
constexpr uint32_t kOob = 0x80000000u;
typedef __amdgpu_buffer_rsrc_t Rsrc;

__device__ __forceinline__ Rsrc plane_rsrc(const float* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float buf_load(Rsrc r, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void buf_store(Rsrc r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, (int)off, 0, 0);
}

// The lane's staged values of one input row: column c0 - 5 + l and, for
// l < 10, column c0 + 59 + l; zero outside the image.
__device__ __forceinline__ void load_row(Rsrc p, const LossArgs& a, int gr, int c0, int l,
                                         float& v0, float& v1) {
  const bool rin = gr >= 0 && gr < a.H;
  const int ca = c0 - kLR + l, cb = c0 - kLR + kSW + l;
  const int rowo = gr * a.W;
  v0 = buf_load(p, (rin && ca >= 0 && ca < a.W) ? (uint32_t)(rowo + ca) * 4u : kOob);
  v1 = buf_load(p, (rin && l < 2 * kLR && cb < a.W) ? (uint32_t)(rowo + cb) * 4u : kOob);
}

// Input rows of NM planes loaded 11 rows ahead: row i lives in slot i % 11,
// the slot the unrolled row loop stages it from, and the load of row i + 11
// refills that slot right after.  Static slots keep the in-flight registers
// from being copied (a copy would wait for the load).
template <int NM>
struct RowRing {
  float v0[NM][11], v1[NM][11];
  __device__ __forceinline__ void fill(const Rsrc (&p)[NM], const LossArgs& a, int gr0, int c0,
                                       int l) {
#pragma unroll
    for (int q = 0; q < 11; ++q)
#pragma unroll
      for (int m = 0; m < NM; ++m) load_row(p[m], a, gr0 + q, c0, l, v0[m][q], v1[m][q]);
  }
};

template <bool kMaps>
__global__ void __launch_bounds__(kSW)
l1_ssim_fwd_kernel(const LossArgs a, const float* __restrict__ img, const float* __restrict__ tgt,
                   float* __restrict__ dmaps, float* __restrict__ partials) {
  __shared__ float s_x[2][kRowIn];
  __shared__ float s_y[2][kRowIn];
  // strips in XCD-local order: a strip and its neighbours (whose halo rows
  // and columns it shares) run on one XCD
  const int nt = (int)gridDim.x;
  const int lid = xcd_local_order((int)(blockIdx.x + blockIdx.y * gridDim.x), nt * (int)gridDim.y);
  const int plane = lid / nt, idx = lid - plane * nt;
  const int strip = idx % a.strips_x, chunk = idx / a.strips_x;
  const int l = (int)threadIdx.x;
  const int c0 = strip * kSW, r0 = chunk * kSH;
  const int gc = c0 + l;
  const size_t HW = (size_t)a.H * a.W;
  const uint32_t pb = (uint32_t)HW * 4u;
  const Rsrc src[2] = {plane_rsrc(img + plane * HW, pb), plane_rsrc(tgt + plane * HW, pb)};
  const size_t CHW = (size_t)a.C * HW;
  float* const dbase = kMaps ? dmaps : (float*)img;  // no stores without maps
  const uint32_t db = kMaps ? pb : 0u;
  const Rsrc dst[3] = {plane_rsrc(dbase + plane * HW, db), plane_rsrc(dbase + CHW + plane * HW, db),
                       plane_rsrc(dbase + 2 * CHW + plane * HW, db)};
  const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
  const bool col_in = gc < a.W;
  float ring[11][5];
  float ssim_sum = 0.f, l1_sum = 0.f;
  RowRing<2> rq;
  rq.fill(src, a, r0 - kLR, c0, l);
  // input row i, staged from ring slot sl = i % 11; `first` marks the first
  // 11 rows (i == sl), whose first ten only fill the window
  auto row = [&](const int i, const int sl, const bool first) __attribute__((always_inline)) {
    float* sx = s_x[i & 1];
    float* sy = s_y[i & 1];
    // every lane writes both values (the second is zero past lane 9), so
    // the row has no lane-masked branch for the compiler to sink work into
    sx[l] = rq.v0[0][sl];
    sy[l] = rq.v0[1][sl];
    sx[kSW + l] = rq.v1[0][sl];
    sy[kSW + l] = rq.v1[1][sl];
    // row i + 11 into the freed slot; past the strip's rows, a row index
    // outside the image makes the loads read nothing
    const int pf = i + 11 < kRows ? r0 - kLR + i + 11 : -1;
#pragma unroll
    for (int m = 0; m < 2; ++m) load_row(src[m], a, pf, c0, l, rq.v0[m][sl], rq.v1[m][sl]);
    lds_barrier();
    // the window is symmetric (win[k] == win[10 - k] exactly): taps k and
    // 10 - k share one weight, so the pair's values (and products) are added
    // before the multiply-add: 73 instructions per row instead of 88
    const float xc = sx[l + kLR], yc = sy[l + kLR];
    float m0, m1, m2, m3, m4;
    {
      const float w = a.win[kLR];
      m0 = w * xc;
      m1 = w * yc;
      m2 = w * (xc * xc);
      m3 = w * (yc * yc);
      m4 = w * (xc * yc);
    }
#pragma unroll
    for (int k = 0; k < kLR; ++k) {
      const float xa = sx[l + k], xb = sx[l + 2 * kLR - k];
      const float ya = sy[l + k], yb = sy[l + 2 * kLR - k];
      const float w = a.win[k];
      m0 = __builtin_fmaf(w, xa + xb, m0);
      m1 = __builtin_fmaf(w, ya + yb, m1);
      m2 = __builtin_fmaf(w, __builtin_fmaf(xa, xa, xb * xb), m2);
      m3 = __builtin_fmaf(w, __builtin_fmaf(ya, ya, yb * yb), m3);
      m4 = __builtin_fmaf(w, __builtin_fmaf(xa, ya, xb * yb), m4);
    }
    ring[sl][0] = m0;
    ring[sl][1] = m1;
    ring[sl][2] = m2;
    ring[sl][3] = m3;
    ring[sl][4] = m4;
    // |x - y| of the strip's own pixels, from the staged centre column (zero
    // outside the image, where both values read zero)
    l1_sum += (i >= kLR && i < kLR + kSH) ? fabsf(xc - yc) : 0.f;
    if (first && i < 2 * kLR) return;  // compile-time
    const int orow = r0 + i - 2 * kLR;
    float mx = 0.f, my = 0.f, exx = 0.f, eyy = 0.f, exy = 0.f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const int q = (sl + 1 + k) % 11;  // ring slot of input row orow - 5 + k
      const float w = a.win[k];
      mx = __builtin_fmaf(w, ring[q][0], mx);
      my = __builtin_fmaf(w, ring[q][1], my);
      exx = __builtin_fmaf(w, ring[q][2], exx);
      eyy = __builtin_fmaf(w, ring[q][3], eyy);
      exy = __builtin_fmaf(w, ring[q][4], exy);
    }
    const bool out = orow < a.H && col_in;
    {
      // contracted: the SSIM terms take no decision, and fused products
      // round less (the loss stays inside the tests' bounds)
#pragma clang fp contract(fast)
      const float sxx = exx - mx * mx, syy = eyy - my * my, sxy = exy - mx * my;
      const float A = 2.f * mx * my + C1, Bv = 2.f * sxy + C2;
      const float Cv = mx * mx + my * my + C1, D = sxx + syy + C2;
      // 1/Cv = D inv, 1/D = Cv inv; the hardware reciprocal (1 ulp; Cv D >= C1 C2
      // when the variances are not negative), no decision depends on it
      const float inv = __builtin_amdgcn_rcpf(Cv * D);
      const float S = A * Bv * inv;
      ssim_sum += out ? S : 0.f;
      if (kMaps) {
        // partials w.r.t. mu_x, sigma_xx, sigma_xy, then to the raw moments
        const float dS_dmu = 2.f * my * Bv * inv - S * 2.f * mx * (D * inv);
        const float dS_dsxx = -S * (Cv * inv);
        const float dS_dsxy = 2.f * A * inv;
        const float d1 = dS_dmu + dS_dsxx * (-2.f * mx) + dS_dsxy * (-my);
        const uint32_t po = out ? (uint32_t)(orow * a.W + gc) * 4u : kOob;
        buf_store(dst[0], po, d1);
        buf_store(dst[1], po, dS_dsxx);
        buf_store(dst[2], po, dS_dsxy);
      }
    }
  };
  // rows are kept apart in the schedule: interleaving them lengthens
  // register live ranges past three waves per SIMD
#pragma unroll
  for (int sl = 0; sl < 11; ++sl) {
    row(sl, sl, true);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int base = 11; base < kRows; base += 11) {
#pragma unroll
    for (int sl = 0; sl < 11; ++sl) {
      row(base + sl, sl, false);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // strip partial sums (fixed order)
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    ssim_sum += __shfl_xor(ssim_sum, o, kWave);
    l1_sum += __shfl_xor(l1_sum, o, kWave);
  }
  if (l == 0) {
    const size_t b = (size_t)lid;  // plane * nt + idx
    partials[2 * b + 0] = ssim_sum;
    partials[2 * b + 1] = l1_sum;
  }
}

// Reduces the per-strip partials in a fixed order into the loss scalar.
__global__ void __launch_bounds__(256)
l1_ssim_reduce_kernel(const float* __restrict__ partials, int nblocks, float w_l1, float w_ssim,
                      double inv_n, float* __restrict__ loss) {
  __shared__ double s_s[256];
  __shared__ double s_l[256];
  const int t = (int)threadIdx.x;
  double ss = 0.0, sl = 0.0;
  for (int b = t; b < nblocks; b += 256) {
    ss += (double)partials[2 * b + 0];
    sl += (double)partials[2 * b + 1];
  }
  s_s[t] = ss;
  s_l[t] = sl;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) {
      s_s[t] += s_s[t + o];
      s_l[t] += s_l[t + o];
    }
    __syncthreads();
  }
  if (t == 0) {
    const double l1 = s_l[0] * inv_n, ssim = s_s[0] * inv_n;
    loss[0] = (float)((double)w_l1 * l1 + (double)w_ssim * (1.0 - ssim));
  }
}

__global__ void __launch_bounds__(kSW)
l1_ssim_bwd_kernel(const LossArgs a, const float* __restrict__ img, const float* __restrict__ tgt,
                   const float* __restrict__ dmaps, const float* __restrict__ grad_out,
                   float* __restrict__ dimg) {
  __shared__ float s_d[2][3][kRowIn];
  const int nt = (int)gridDim.x;
  const int lid = xcd_local_order((int)(blockIdx.x + blockIdx.y * gridDim.x), nt * (int)gridDim.y);
  const int plane = lid / nt, idx = lid - plane * nt;
  const int strip = idx % a.strips_x, chunk = idx / a.strips_x;
  const int l = (int)threadIdx.x;
  const int c0 = strip * kSW, r0 = chunk * kSH;
  const int gc = c0 + l;
  const size_t HW = (size_t)a.H * a.W;
  const size_t CHW = (size_t)a.C * HW;
  const uint32_t pb = (uint32_t)HW * 4u;
  const Rsrc dp[3] = {plane_rsrc(dmaps + plane * HW, pb), plane_rsrc(dmaps + CHW + plane * HW, pb),
                      plane_rsrc(dmaps + 2 * CHW + plane * HW, pb)};
  const Rsrc xp = plane_rsrc(img + plane * HW, pb), yp = plane_rsrc(tgt + plane * HW, pb);
  const Rsrc gp = plane_rsrc(dimg + plane * HW, pb);
  const float g = grad_out ? grad_out[0] : 1.0f;
  const float inv_n = (float)(1.0 / (double)CHW);
  const bool col_in = gc < a.W;
  float ring[11][3];
  RowRing<3> rq;
  rq.fill(dp, a, r0 - kLR, c0, l);
  auto row = [&](const int i, const int sl, const bool first) __attribute__((always_inline)) {
    float (*sd)[kRowIn] = s_d[i & 1];
    // x, y of this row's output pixel, issued before the row's prefetch so
    // that their use waits for them alone, not for the prefetch
    const int orow0 = r0 + i - 2 * kLR;
    const bool has_out = !(first && i < 2 * kLR);
    const uint32_t ox = (has_out && orow0 < a.H && col_in) ? (uint32_t)(orow0 * a.W + gc) * 4u : kOob;
    const float x = buf_load(xp, ox), y = buf_load(yp, ox);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      sd[m][l] = rq.v0[m][sl];
      sd[m][kSW + l] = rq.v1[m][sl];  // zero past lane 9
    }
    const int pf = i + 11 < kRows ? r0 - kLR + i + 11 : -1;  // -1: reads nothing
#pragma unroll
    for (int m = 0; m < 3; ++m) load_row(dp[m], a, pf, c0, l, rq.v0[m][sl], rq.v1[m][sl]);
    lds_barrier();
#pragma unroll
    for (int m = 0; m < 3; ++m) {
      float h = 0.f;
#pragma unroll
      for (int k = 0; k < 11; ++k) h = __builtin_fmaf(a.win[k], sd[m][l + k], h);
      ring[sl][m] = h;
    }
    if (first && i < 2 * kLR) return;  // compile-time
    float B[3] = {0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const int q = (sl + 1 + k) % 11;
#pragma unroll
      for (int m = 0; m < 3; ++m) B[m] = __builtin_fmaf(a.win[k], ring[q][m], B[m]);
    }
    // x, y are loaded in the row that uses them: kept five rows ahead in a
    // register ring they took 29 VGPRs, two waves per SIMD instead of three
    // (39 against 42 us at 1080p)
    const uint32_t o = ox;
    const float d = x - y;
    const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
    const float dssim = B[0] + 2.f * x * B[1] + y * B[2];
    buf_store(gp, o, g * inv_n * (a.w_l1 * sgn - a.w_ssim * dssim));
  };
  // rows are kept apart in the schedule: interleaving them lengthens
  // register live ranges past three waves per SIMD
#pragma unroll
  for (int sl = 0; sl < 11; ++sl) {
    row(sl, sl, true);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int base = 11; base < kRows; base += 11) {
#pragma unroll
    for (int sl = 0; sl < 11; ++sl) {
      row(base + sl, sl, false);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

static LossArgs make_args(int C, int H, int W, float w_l1, float w_ssim) {
  LossArgs a;
  a.C = C;
  a.H = H;
  a.W = W;
  a.strips_x = (W + kSW - 1) / kSW;
  a.chunks_y = (H + kSH - 1) / kSH;
  a.w_l1 = w_l1;
  a.w_ssim = w_ssim;
  double g[11], s = 0.0;
  for (int k = 0; k < 11; ++k) {
    const double x = (double)(k - 5);
    g[k] = std::exp(-(x * x) / (2.0 * 1.5 * 1.5));
    s += g[k];
  }
  for (int k = 0; k < 11; ++k) a.win[k] = (float)(g[k] / s);
  return a;
}

// Pointwise photometric losses of the training script's loss_fn
// (scripts/train_scanner_fastgs.py:911-966): mean |x - y| (mode 0) or mean
// (x - y)^2 (mode 1).  Each term is formed in float and summed in double:
// per-block partials, then one block reduces them in a fixed order.
constexpr int kPwItems = 8;  // elements per thread, 256 threads per block
constexpr int64_t kPwBlock = 256 * kPwItems;

__device__ __forceinline__ float pw_term(float x, float y, int mode) {
  const float d = x - y;
  return mode ? d * d : fabsf(d);
}

__global__ void __launch_bounds__(256)
pointwise_loss_partials_kernel(const float* __restrict__ x, const float* __restrict__ y, int64_t n,
                               int mode, double* __restrict__ partials) {
  __shared__ double s_w[256 / kWave];
  const int64_t base = (int64_t)blockIdx.x * kPwBlock + threadIdx.x;
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < kPwItems; ++k) {
    const int64_t i = base + (int64_t)k * 256;
    if (i < n) acc += (double)pw_term(x[i], y[i], mode);
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o, kWave);
  if (lane_id() == 0) s_w[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double b = 0.0;
    for (int w = 0; w < 256 / kWave; ++w) b += s_w[w];
    partials[blockIdx.x] = b;
  }
}

__global__ void __launch_bounds__(256)
pointwise_loss_reduce_kernel(const double* __restrict__ partials, int64_t nb, double inv_n,
                             float* __restrict__ loss) {
  __shared__ double s[256];
  const int t = (int)threadIdx.x;
  double acc = 0.0;
  for (int64_t b = t; b < nb; b += 256) acc += partials[b];
  s[t] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) s[t] += s[t + o];
    __syncthreads();
  }
  if (t == 0) loss[0] = (float)(s[0] * inv_n);
}

// dL/dx = g * sign(x - y) / n (mode 0; 0 where x == y) or g * 2 (x - y) / n.
__global__ void __launch_bounds__(256)
pointwise_loss_bwd_kernel(const float* __restrict__ x, const float* __restrict__ y, int64_t n,
                          int mode, const float* __restrict__ grad_out, float inv_n,
                          float* __restrict__ dx) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = (grad_out ? grad_out[0] : 1.0f) * inv_n;
  const float d = x[i] - y[i];
  const float s = mode ? 2.0f * d : (d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f));
  dx[i] = g * s;
}

}  // namespace fgs

using namespace fgs;

extern "C" size_t fgs_l1_ssim_workspace_bytes(int32_t C, int32_t H, int32_t W) {
  if (C <= 0 || H <= 0 || W <= 0) return 256;
  const size_t blocks = (size_t)C * ((W + kSW - 1) / kSW) * ((H + kSH - 1) / kSH);
  return (blocks * 2 * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" int32_t fgs_l1_ssim_fwd(const float* img, const float* tgt, int32_t C, int32_t H,
                                   int32_t W, float w_l1, float w_ssim, float* loss, float* dmaps,
                                   void* workspace, void* stream) {
  if (C <= 0 || H <= 0 || W <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_fwd: bad image shape");
  if ((size_t)H * (size_t)W >= ((size_t)1 << 29))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_fwd: image plane of 2^29 pixels or more");
  if (!img || !tgt || !loss || !workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_fwd: null pointer");
  const LossArgs a = make_args(C, H, W, w_l1, w_ssim);
  const int nt = a.strips_x * a.chunks_y;
  hipStream_t st = (hipStream_t)stream;
  if (const int32_t e = launch_mark(kLaunchLossFwd, st, 0)) return e;
  if (dmaps)
    hipLaunchKernelGGL(l1_ssim_fwd_kernel<true>, dim3(nt, C), dim3(kSW), 0, st, a, img, tgt, dmaps,
                       (float*)workspace);
  else
    hipLaunchKernelGGL(l1_ssim_fwd_kernel<false>, dim3(nt, C), dim3(kSW), 0, st, a, img, tgt,
                       dmaps, (float*)workspace);
  if (check_launch("l1_ssim_fwd") != FGS_OK) return FGS_ERR_LAUNCH;
  if (const int32_t e = launch_mark(kLaunchLossFwd, st, 1)) return e;
  hipLaunchKernelGGL(l1_ssim_reduce_kernel, dim3(1), dim3(256), 0, st, (const float*)workspace,
                     nt * C, w_l1, w_ssim, 1.0 / ((double)C * H * W), loss);
  return check_launch("l1_ssim_fwd");
}

extern "C" int32_t fgs_l1_ssim_bwd(const float* img, const float* tgt, const float* dmaps,
                                   const float* grad_out, int32_t C, int32_t H, int32_t W,
                                   float w_l1, float w_ssim, float* dimg, void* stream) {
  if (C <= 0 || H <= 0 || W <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_bwd: bad image shape");
  if ((size_t)H * (size_t)W >= ((size_t)1 << 29))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_bwd: image plane of 2^29 pixels or more");
  if (!img || !tgt || !dmaps || !dimg)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_bwd: null pointer");
  const LossArgs a = make_args(C, H, W, w_l1, w_ssim);
  const int nt = a.strips_x * a.chunks_y;
  hipStream_t st = (hipStream_t)stream;
  if (const int32_t e = launch_mark(kLaunchLossBwd, st, 0)) return e;
  hipLaunchKernelGGL(l1_ssim_bwd_kernel, dim3(nt, C), dim3(kSW), 0, st, a, img, tgt, dmaps,
                     grad_out, dimg);
  if (check_launch("l1_ssim_bwd") != FGS_OK) return FGS_ERR_LAUNCH;
  return launch_mark(kLaunchLossBwd, st, 1);
}

extern "C" size_t fgs_pointwise_loss_workspace_bytes(int64_t n) {
  const int64_t nb = (n + kPwBlock - 1) / kPwBlock;
  return (size_t)((nb < 1 ? 1 : nb) * 8);
}

extern "C" int32_t fgs_pointwise_loss_fwd(const float* x, const float* y, int64_t n, int32_t mode,
                                          void* workspace, float* loss, void* stream) {
  if (n <= 0 || (mode != 0 && mode != 1))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_pointwise_loss_fwd: bad arguments");
  if (!x || !y || !workspace || !loss)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_pointwise_loss_fwd: null pointer");
  const int64_t nb = (n + kPwBlock - 1) / kPwBlock;
  if (nb > 0x7FFFFFFF) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_pointwise_loss_fwd: too large");
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(pointwise_loss_partials_kernel, dim3((unsigned)nb), dim3(256), 0, st, x, y, n,
                     mode, (double*)workspace);
  hipLaunchKernelGGL(pointwise_loss_reduce_kernel, dim3(1), dim3(256), 0, st,
                     (const double*)workspace, nb, 1.0 / (double)n, loss);
  return check_launch("pointwise_loss_fwd");
}

extern "C" int32_t fgs_pointwise_loss_bwd(const float* x, const float* y, int64_t n, int32_t mode,
                                          const float* grad_out, float* dx, void* stream) {
  if (n <= 0 || (mode != 0 && mode != 1))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_pointwise_loss_bwd: bad arguments");
  if (!x || !y || !dx)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_pointwise_loss_bwd: null pointer");
  hipLaunchKernelGGL(pointwise_loss_bwd_kernel, dim3(ceil_div_u(n, 256)), dim3(256), 0,
                     (hipStream_t)stream, x, y, n, mode, grad_out, (float)(1.0 / (double)n), dx);
  return check_launch("pointwise_loss_bwd_kernel");
}
