// fgs_train.hip -- training-step glue on either side of the rasterizer.
//
// Parameter activations (the caller contract of the reference training
// scripts, scripts/train_scanner_fixed.py:523-536, train_square.py:181-191):
//   opacity  = sigmoid(opacity_logit) = 1 / (1 + exp(-x))
//   scale    = exp(log_scale)
//   rotation = q / (|q| + 1e-8)
// and their backward, one thread per Gaussian, AoS rows read and written as
// vectors where the row is 16 bytes.
//
// Adam (the optimizer of scripts/train_scanner_fastgs.py:77-182, MLX's
// mlx.optimizers.Adam, whose default has no bias correction):
//   m = b1 m + (1 - b1) g,  v = b2 v + (1 - b2) g^2,
//   p = p - lr m / (sqrt(v) + eps)                       (bias_correction = 0)
//   p = p - (lr / (1 - b1^t)) m / (sqrt(v) / sqrt(1 - b2^t) + eps)   (= 1)
// over any number of elements, in place.
#include "fgs_common.hpp"

namespace fgs {

__global__ void __launch_bounds__(256)
activations_fwd_kernel(int32_t P, const float* __restrict__ log_scales,
                       const float* __restrict__ quats, const float* __restrict__ logits,
                       float* __restrict__ scales, float* __restrict__ rotations,
                       float* __restrict__ opacities) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  if (log_scales) {
#pragma unroll
    for (int k = 0; k < 3; ++k) scales[3 * (size_t)i + k] = act_scale(log_scales[3 * (size_t)i + k]);
  }
  if (quats)
    *reinterpret_cast<float4*>(rotations + 4 * (size_t)i) =
        act_rotation(*reinterpret_cast<const float4*>(quats + 4 * (size_t)i));
  if (logits) opacities[i] = act_opacity(logits[i]);
}

// Gradients w.r.t. the raw parameters from the gradients of the activated
// ones (absent gradients are zero):
//   d log_scale = d scale * scale
//   d logit     = d opacity * (1 - opacity) * opacity
//   d q         = d r / d - q (q . d r) / (d^2 |q|),  d = |q| + 1e-8
//                 (the second term is 0 at q = 0)
__global__ void __launch_bounds__(256)
activations_bwd_kernel(int32_t P, const float* __restrict__ quats,
                       const float* __restrict__ scales, const float* __restrict__ opacities,
                       const float* __restrict__ d_scales, const float* __restrict__ d_rotations,
                       const float* __restrict__ d_opacities, float* __restrict__ d_log_scales,
                       float* __restrict__ d_quats, float* __restrict__ d_logits) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  if (d_log_scales) {
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const float g = d_scales ? d_scales[3 * (size_t)i + k] : 0.0f;
      d_log_scales[3 * (size_t)i + k] = g * scales[3 * (size_t)i + k];
    }
  }
  if (d_quats) {
    const float4 q = *reinterpret_cast<const float4*>(quats + 4 * (size_t)i);
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
    if (d_rotations) g = *reinterpret_cast<const float4*>(d_rotations + 4 * (size_t)i);
    *reinterpret_cast<float4*>(d_quats + 4 * (size_t)i) = quat_normalize_grad(q, g);
  }
  if (d_logits) {
    const float o = opacities[i];
    const float g = d_opacities ? d_opacities[i] : 0.0f;
    d_logits[i] = g * (1.0f - o) * o;
  }
}

struct AdamArgs {
  float b1, b2, one_minus_b1, one_minus_b2, step_size, bc2_sqrt, eps;
  int bias_correction;
};

// In-place Adam on n elements; four elements per thread when aligned.
__global__ void __launch_bounds__(256)
adam_kernel(int64_t n, AdamArgs a, float* __restrict__ p, const float* __restrict__ g,
            float* __restrict__ m, float* __restrict__ v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = g[i];
  const float mi = a.b1 * m[i] + a.one_minus_b1 * gi;
  const float vi = a.b2 * v[i] + a.one_minus_b2 * (gi * gi);
  m[i] = mi;
  v[i] = vi;
  if (a.bias_correction)
    p[i] = p[i] - (a.step_size * mi) / (sqrtf(vi) / a.bc2_sqrt + a.eps);
  else
    p[i] = p[i] - (a.step_size * mi) / (sqrtf(vi) + a.eps);
}

// Several tensors in one launch: the blocks of group k are [block_end[k-1],
// block_end[k]); per-group step size and bias correction, the same update.
constexpr int kAdamGroups = 8;
struct AdamGroupDev {
  float* p;
  const float* g;
  float* m;
  float* v;
  int64_t n;
  float step_size, bc2_sqrt;
};
struct AdamMulti {
  AdamGroupDev grp[kAdamGroups];
  int64_t block_end[kAdamGroups];
  int count;
  float b1, b2, one_minus_b1, one_minus_b2, eps;
  int bias_correction;
};

__global__ void __launch_bounds__(256) adam_multi_kernel(const AdamMulti a) {
  int k = 0;
  while (k < a.count - 1 && (int64_t)blockIdx.x >= a.block_end[k]) ++k;  // uniform
  const int64_t b0 = k ? a.block_end[k - 1] : 0;
  const AdamGroupDev& G = a.grp[k];
  const int64_t i = ((int64_t)blockIdx.x - b0) * blockDim.x + threadIdx.x;
  if (i >= G.n) return;
  const float gi = G.g[i];
  const float mi = a.b1 * G.m[i] + a.one_minus_b1 * gi;
  const float vi = a.b2 * G.v[i] + a.one_minus_b2 * (gi * gi);
  G.m[i] = mi;
  G.v[i] = vi;
  if (a.bias_correction)
    G.p[i] = G.p[i] - (G.step_size * mi) / (sqrtf(vi) / G.bc2_sqrt + a.eps);
  else
    G.p[i] = G.p[i] - (G.step_size * mi) / (sqrtf(vi) + a.eps);
}

// Step size and sqrt of the second bias correction of one Adam step (bias
// corrections in double, as a host optimizer computes them).
static void adam_scales(float lr, float beta1, float beta2, int32_t step, int32_t bias_correction,
                        float* step_size, float* bc2_sqrt) {
  if (bias_correction) {
    const double bc1 = 1.0 - __builtin_pow((double)beta1, (double)step);
    const double bc2 = 1.0 - __builtin_pow((double)beta2, (double)step);
    *step_size = (float)((double)lr / bc1);
    *bc2_sqrt = (float)__builtin_sqrt(bc2);
  } else {
    *step_size = lr;
    *bc2_sqrt = 1.0f;
  }
}

}  // namespace fgs

using namespace fgs;

extern "C" int32_t fgs_activations_fwd(int32_t P, const float* log_scales, const float* quats,
                                       const float* opacity_logits, float* scales,
                                       float* rotations, float* opacities, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_activations_fwd: P < 0");
  if ((log_scales && !scales) || (quats && !rotations) || (opacity_logits && !opacities))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_activations_fwd: missing output");
  if (P == 0) return FGS_OK;
  hipLaunchKernelGGL(activations_fwd_kernel, dim3(ceil_div_u(P, 256)), dim3(256), 0,
                     (hipStream_t)stream, P, log_scales, quats, opacity_logits, scales, rotations,
                     opacities);
  return check_launch("activations_fwd_kernel");
}

extern "C" int32_t fgs_activations_bwd(int32_t P, const float* quats, const float* scales,
                                       const float* opacities, const float* d_scales,
                                       const float* d_rotations, const float* d_opacities,
                                       float* d_log_scales, float* d_quats, float* d_logits,
                                       void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_activations_bwd: P < 0");
  if ((d_log_scales && !scales) || (d_quats && !quats) || (d_logits && !opacities))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_activations_bwd: missing forward tensor");
  if (P == 0) return FGS_OK;
  hipLaunchKernelGGL(activations_bwd_kernel, dim3(ceil_div_u(P, 256)), dim3(256), 0,
                     (hipStream_t)stream, P, quats, scales, opacities, d_scales, d_rotations,
                     d_opacities, d_log_scales, d_quats, d_logits);
  return check_launch("activations_bwd_kernel");
}

extern "C" int32_t fgs_adam_step(float* param, const float* grad, float* exp_avg,
                                 float* exp_avg_sq, int64_t n, float lr, float beta1, float beta2,
                                 float eps, int32_t step, int32_t bias_correction, void* stream) {
  if (n < 0 || step < 1 || !(beta1 >= 0.0f && beta1 < 1.0f) || !(beta2 >= 0.0f && beta2 < 1.0f))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step: bad arguments");
  if (n == 0) return FGS_OK;
  if (!param || !grad || !exp_avg || !exp_avg_sq)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step: null pointer");
  AdamArgs a;
  a.b1 = beta1;
  a.b2 = beta2;
  a.one_minus_b1 = 1.0f - beta1;
  a.one_minus_b2 = 1.0f - beta2;
  a.eps = eps;
  a.bias_correction = bias_correction ? 1 : 0;
  adam_scales(lr, beta1, beta2, step, bias_correction, &a.step_size, &a.bc2_sqrt);
  hipLaunchKernelGGL(adam_kernel, dim3(ceil_div_u(n, 256)), dim3(256), 0, (hipStream_t)stream, n,
                     a, param, grad, exp_avg, exp_avg_sq);
  return check_launch("adam_kernel");
}

extern "C" int32_t fgs_adam_step_multi(const fgs_adam_group* groups, int32_t count, float beta1,
                                       float beta2, float eps, int32_t bias_correction,
                                       void* stream) {
  if (count < 0 || count > kAdamGroups || (count > 0 && !groups) ||
      !(beta1 >= 0.0f && beta1 < 1.0f) || !(beta2 >= 0.0f && beta2 < 1.0f))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step_multi: bad arguments");
  AdamMulti a{};
  a.b1 = beta1;
  a.b2 = beta2;
  a.one_minus_b1 = 1.0f - beta1;
  a.one_minus_b2 = 1.0f - beta2;
  a.eps = eps;
  a.bias_correction = bias_correction ? 1 : 0;
  int64_t blocks = 0;
  for (int k = 0; k < count; ++k) {
    const fgs_adam_group& g = groups[k];
    if (g.n < 0 || g.step < 1)
      return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step_multi: bad group");
    if (g.n > 0 && (!g.param || !g.grad || !g.exp_avg || !g.exp_avg_sq))
      return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step_multi: null pointer");
    if (g.n == 0) continue;
    AdamGroupDev& d = a.grp[a.count];
    d.p = g.param;
    d.g = g.grad;
    d.m = g.exp_avg;
    d.v = g.exp_avg_sq;
    d.n = g.n;
    adam_scales(g.lr, beta1, beta2, g.step, bias_correction, &d.step_size, &d.bc2_sqrt);
    blocks += (g.n + 255) / 256;
    a.block_end[a.count] = blocks;
    ++a.count;
  }
  if (a.count == 0) return FGS_OK;
  if (blocks > 0x7FFFFFFF) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_adam_step_multi: too large");
  hipLaunchKernelGGL(adam_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     a);
  return check_launch("adam_multi_kernel");
}
