// fgs_loss.hip -- fused photometric loss of the training step:
//   L = w_l1 * mean|x - y| + w_ssim * (1 - mean SSIM(x, y))
// over C planes of H x W, SSIM with an 11x11 separable Gaussian window
// (zero padding, per channel), C1 = 0.01^2, C2 = 0.03^2 -- the loss the
// reference's FastGS training scripts put on the rendered image
// (scripts/train_scanner_fastgs.py:911-966), which the rasterizer's
// backward consumes as dL/dout_color.
//
// Forward: one 256-thread workgroup per 32x32 output tile of one plane.  x
// and y are staged with a 5-pixel halo in LDS, blurred horizontally into five
// LDS maps (x, y, x^2, y^2, xy) and vertically per output pixel; the SSIM
// value and its partial derivatives with respect to the three blurred
// moments of x (E[x], E[x^2], E[xy]) are written per pixel, and per-block
// partial sums of SSIM and |x - y| go to a partials array that a second
// kernel reduces in a fixed order (deterministic).
//
// Backward: the three partial-derivative maps are blurred the same way
// (the zero-padded symmetric blur is self-adjoint) and combined with x, y:
//   dL/dx = g * (w_l1 sign(x-y) / N - w_ssim / N * (B1 + 2 x B2 + y B3)),
// Bk = blur(dS/dmk), g the upstream scalar gradient (read on the device).
#include "fgs_common.hpp"

namespace fgs {

constexpr int kLT = 32;            // output tile edge
constexpr int kLR = 5;             // window radius (11 taps)
constexpr int kLIn = kLT + 2 * kLR;  // 42: staged edge with halo

struct LossArgs {
  int C, H, W;
  int tiles_x, tiles_y;
  float w_l1, w_ssim;
  float win[11];
};

__device__ __forceinline__ float load_or_zero(const float* __restrict__ p, int H, int W, int r,
                                              int c) {
  return (r >= 0 && r < H && c >= 0 && c < W) ? p[(size_t)r * W + c] : 0.0f;
}

__global__ void __launch_bounds__(256)
l1_ssim_fwd_kernel(const LossArgs a, const float* __restrict__ img, const float* __restrict__ tgt,
                   float* __restrict__ dmaps, float* __restrict__ partials) {
  __shared__ float s_x[kLIn][kLIn + 1];
  __shared__ float s_y[kLIn][kLIn + 1];
  __shared__ float s_h[5][kLIn][kLT + 1];
  __shared__ float s_red[2][4];
  const int tile = (int)blockIdx.x;
  const int plane = (int)blockIdx.y;
  const int t = (int)threadIdx.x;
  const int ty0 = (tile / a.tiles_x) * kLT;
  const int tx0 = (tile % a.tiles_x) * kLT;
  const size_t HW = (size_t)a.H * a.W;
  const float* __restrict__ xp = img + plane * HW;
  const float* __restrict__ yp = tgt + plane * HW;
  for (int i = t; i < kLIn * kLIn; i += 256) {
    const int r = i / kLIn, c = i % kLIn;
    s_x[r][c] = load_or_zero(xp, a.H, a.W, ty0 - kLR + r, tx0 - kLR + c);
    s_y[r][c] = load_or_zero(yp, a.H, a.W, ty0 - kLR + r, tx0 - kLR + c);
  }
  __syncthreads();
  for (int i = t; i < kLIn * kLT; i += 256) {
    const int r = i / kLT, c = i % kLT;
    float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f, m4 = 0.f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const float x = s_x[r][c + k], y = s_y[r][c + k], w = a.win[k];
      m0 += w * x;
      m1 += w * y;
      m2 += w * (x * x);
      m3 += w * (y * y);
      m4 += w * (x * y);
    }
    s_h[0][r][c] = m0;
    s_h[1][r][c] = m1;
    s_h[2][r][c] = m2;
    s_h[3][r][c] = m3;
    s_h[4][r][c] = m4;
  }
  __syncthreads();
  const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
  float ssim_sum = 0.f, l1_sum = 0.f;
  for (int i = t; i < kLT * kLT; i += 256) {
    const int r = i / kLT, c = i % kLT;
    const int gr = ty0 + r, gc = tx0 + c;
    if (gr >= a.H || gc >= a.W) continue;
    float mx = 0.f, my = 0.f, exx = 0.f, eyy = 0.f, exy = 0.f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const float w = a.win[k];
      mx += w * s_h[0][r + k][c];
      my += w * s_h[1][r + k][c];
      exx += w * s_h[2][r + k][c];
      eyy += w * s_h[3][r + k][c];
      exy += w * s_h[4][r + k][c];
    }
    const float sxx = exx - mx * mx, syy = eyy - my * my, sxy = exy - mx * my;
    const float A = 2.f * mx * my + C1, Bv = 2.f * sxy + C2;
    const float Cv = mx * mx + my * my + C1, D = sxx + syy + C2;
    const float inv = 1.0f / (Cv * D);
    const float S = A * Bv * inv;
    ssim_sum += S;
    const float x = s_x[r + kLR][c + kLR], y = s_y[r + kLR][c + kLR];
    l1_sum += fabsf(x - y);
    if (dmaps) {
      // partials w.r.t. mu_x, sigma_xx, sigma_xy, then to the raw moments
      const float dS_dmu = 2.f * my * Bv * inv - S * 2.f * mx / Cv;
      const float dS_dsxx = -S / D;
      const float dS_dsxy = 2.f * A * inv;
      const float d1 = dS_dmu + dS_dsxx * (-2.f * mx) + dS_dsxy * (-my);
      const size_t o = (size_t)plane * HW + (size_t)gr * a.W + gc;
      dmaps[o] = d1;
      dmaps[(size_t)a.C * HW + o] = dS_dsxx;
      dmaps[(size_t)2 * a.C * HW + o] = dS_dsxy;
    }
  }
  // block partial sums (fixed order)
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    ssim_sum += __shfl_xor(ssim_sum, o, kWave);
    l1_sum += __shfl_xor(l1_sum, o, kWave);
  }
  if (lane_id() == 0) {
    s_red[0][t / kWave] = ssim_sum;
    s_red[1][t / kWave] = l1_sum;
  }
  __syncthreads();
  if (t == 0) {
    const size_t b = (size_t)plane * gridDim.x + tile;
    partials[2 * b + 0] = (s_red[0][0] + s_red[0][1]) + (s_red[0][2] + s_red[0][3]);
    partials[2 * b + 1] = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);
  }
}

// Reduces the per-block partials in a fixed order into the loss scalar.
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

__global__ void __launch_bounds__(256)
l1_ssim_bwd_kernel(const LossArgs a, const float* __restrict__ img, const float* __restrict__ tgt,
                   const float* __restrict__ dmaps, const float* __restrict__ grad_out,
                   float* __restrict__ dimg) {
  __shared__ float s_d[3][kLIn][kLIn + 1];
  __shared__ float s_h[3][kLIn][kLT + 1];
  const int tile = (int)blockIdx.x;
  const int plane = (int)blockIdx.y;
  const int t = (int)threadIdx.x;
  const int ty0 = (tile / a.tiles_x) * kLT;
  const int tx0 = (tile % a.tiles_x) * kLT;
  const size_t HW = (size_t)a.H * a.W;
  const size_t CHW = (size_t)a.C * HW;
  for (int i = t; i < kLIn * kLIn; i += 256) {
    const int r = i / kLIn, c = i % kLIn;
    const int gr = ty0 - kLR + r, gc = tx0 - kLR + c;
    const bool in = gr >= 0 && gr < a.H && gc >= 0 && gc < a.W;
    const size_t o = plane * HW + (in ? (size_t)gr * a.W + gc : 0);
    s_d[0][r][c] = in ? dmaps[o] : 0.f;
    s_d[1][r][c] = in ? dmaps[CHW + o] : 0.f;
    s_d[2][r][c] = in ? dmaps[2 * CHW + o] : 0.f;
  }
  __syncthreads();
  for (int i = t; i < kLIn * kLT; i += 256) {
    const int r = i / kLT, c = i % kLT;
    float b0 = 0.f, b1 = 0.f, b2 = 0.f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const float w = a.win[k];
      b0 += w * s_d[0][r][c + k];
      b1 += w * s_d[1][r][c + k];
      b2 += w * s_d[2][r][c + k];
    }
    s_h[0][r][c] = b0;
    s_h[1][r][c] = b1;
    s_h[2][r][c] = b2;
  }
  __syncthreads();
  const float g = grad_out ? grad_out[0] : 1.0f;
  const float inv_n = (float)(1.0 / (double)CHW);
  for (int i = t; i < kLT * kLT; i += 256) {
    const int r = i / kLT, c = i % kLT;
    const int gr = ty0 + r, gc = tx0 + c;
    if (gr >= a.H || gc >= a.W) continue;
    float B1 = 0.f, B2 = 0.f, B3 = 0.f;
#pragma unroll
    for (int k = 0; k < 11; ++k) {
      const float w = a.win[k];
      B1 += w * s_h[0][r + k][c];
      B2 += w * s_h[1][r + k][c];
      B3 += w * s_h[2][r + k][c];
    }
    const size_t o = plane * HW + (size_t)gr * a.W + gc;
    const float x = img[o], y = tgt[o];
    const float d = x - y;
    const float sgn = d > 0.f ? 1.f : (d < 0.f ? -1.f : 0.f);
    const float dssim = B1 + 2.f * x * B2 + y * B3;
    dimg[o] = g * inv_n * (a.w_l1 * sgn - a.w_ssim * dssim);
  }
}

static LossArgs make_args(int C, int H, int W, float w_l1, float w_ssim) {
  LossArgs a;
  a.C = C;
  a.H = H;
  a.W = W;
  a.tiles_x = (W + kLT - 1) / kLT;
  a.tiles_y = (H + kLT - 1) / kLT;
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

}  // namespace fgs

using namespace fgs;

extern "C" size_t fgs_l1_ssim_workspace_bytes(int32_t C, int32_t H, int32_t W) {
  if (C <= 0 || H <= 0 || W <= 0) return 256;
  const size_t blocks = (size_t)C * ((W + kLT - 1) / kLT) * ((H + kLT - 1) / kLT);
  return (blocks * 2 * sizeof(float) + 255) & ~(size_t)255;
}

extern "C" int32_t fgs_l1_ssim_fwd(const float* img, const float* tgt, int32_t C, int32_t H,
                                   int32_t W, float w_l1, float w_ssim, float* loss, float* dmaps,
                                   void* workspace, void* stream) {
  if (C <= 0 || H <= 0 || W <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_fwd: bad image shape");
  if (!img || !tgt || !loss || !workspace)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_fwd: null pointer");
  const LossArgs a = make_args(C, H, W, w_l1, w_ssim);
  const int nt = a.tiles_x * a.tiles_y;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(l1_ssim_fwd_kernel, dim3(nt, C), dim3(256), 0, st, a, img, tgt, dmaps,
                     (float*)workspace);
  hipLaunchKernelGGL(l1_ssim_reduce_kernel, dim3(1), dim3(256), 0, st, (const float*)workspace,
                     nt * C, w_l1, w_ssim, 1.0 / ((double)C * H * W), loss);
  return check_launch("l1_ssim_fwd");
}

extern "C" int32_t fgs_l1_ssim_bwd(const float* img, const float* tgt, const float* dmaps,
                                   const float* grad_out, int32_t C, int32_t H, int32_t W,
                                   float w_l1, float w_ssim, float* dimg, void* stream) {
  if (C <= 0 || H <= 0 || W <= 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_bwd: bad image shape");
  if (!img || !tgt || !dmaps || !dimg)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_l1_ssim_bwd: null pointer");
  const LossArgs a = make_args(C, H, W, w_l1, w_ssim);
  const int nt = a.tiles_x * a.tiles_y;
  hipLaunchKernelGGL(l1_ssim_bwd_kernel, dim3(nt, C), dim3(256), 0, (hipStream_t)stream, a, img,
                     tgt, dmaps, grad_out, dimg);
  return check_launch("l1_ssim_bwd");
}
