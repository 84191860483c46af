// fgs_densify.hip -- FastGS densification and pruning on the GPU.
//
// The reference (scripts/train_scanner_fastgs.py) keeps the Gaussians and the
// Adam moments in MLX arrays and densifies on the host with numpy: gradient
// statistics (:391-405), scores from a metric render (:279-340), clone /
// split / prune (:470-616, :661-742), final pruning (:745-793) and opacity
// capping (:619-658).  Here every per-Gaussian step is a kernel over
// device-resident rows:
//
//   stats      max_radii2d / |grad xy| / |grad abs| / denom accumulation
//   classify   clone and split flags of the current rows
//   layout     the pre-prune rows: kept originals, clones, split children
//   keys       prune candidates and their weighted-sampling keys
//   select     the k smallest keys removed, the rest compacted
//   build      every parameter, Adam-moment and statistics row of the new
//              set gathered from its source in one pass, split children
//              computed, opacity capped
//
// Numbers follow the reference's float32 expressions with contraction off;
// exp/log are the library's deterministic det_expf / det_logf, so the CPU
// oracle reproduces every decision bit for bit.  Random numbers (split
// offsets, prune sampling) are inputs, drawn by the caller.
#include "fgs_common.hpp"

namespace fgs {

__device__ __forceinline__ float sigmoid_det(float x) { return 1.0f / (1.0f + det_expf(-x)); }

// numpy logit of train_scanner_fixed.py:157-159: clip to [1e-6, 1 - 1e-6].
__device__ __forceinline__ float logit_det(float p) {
  const float lo = 1.0e-6f, hi = 0.999999f;  // float32(1 - 1e-6)
  p = fminf(fmaxf(p, lo), hi);
  return det_logf(p / (1.0f - p));
}

__device__ __forceinline__ float max_scale3(const float* ls) {
  return fmaxf(fmaxf(det_expf(ls[0]), det_expf(ls[1])), det_expf(ls[2]));
}

// Split child: log scale log(exp(ls) / (0.8 * factor)) per axis.
__device__ __forceinline__ float child_log_scale(float ls, float div) {
  return det_logf(det_expf(ls) / div);
}

__global__ void __launch_bounds__(256)
densify_stats_kernel(int32_t P, const int32_t* __restrict__ radii,
                     const float* __restrict__ dvs, float* __restrict__ max_radii2d,
                     float* __restrict__ acc, float* __restrict__ acc_abs,
                     float* __restrict__ denom, int32_t* __restrict__ tmp_radii) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const int32_t r = radii[i];
  tmp_radii[i] = r;
  if (r <= 0) return;
  const float4 g = *reinterpret_cast<const float4*>(dvs + 4 * (size_t)i);
  max_radii2d[i] = fmaxf(max_radii2d[i], (float)r);
  acc[i] = acc[i] + __builtin_sqrtf(g.x * g.x + g.y * g.y);
  acc_abs[i] = acc_abs[i] + __builtin_sqrtf(g.z * g.z + g.w * g.w);
  denom[i] = denom[i] + 1.0f;
}

__global__ void __launch_bounds__(256)
densify_classify_kernel(int32_t P, fgs_densify_params prm, const float* __restrict__ acc,
                        const float* __restrict__ acc_abs, const float* __restrict__ denom,
                        const float* __restrict__ log_scales, const float* __restrict__ importance,
                        uint32_t* __restrict__ clone_flag, uint32_t* __restrict__ split_flag) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const float d = fmaxf(denom[i], 1.0f);
  const float gv = acc[i] / d, ga = acc_abs[i] / d;
  const bool grad_q = fabsf(gv) >= prm.grad_thresh;
  const bool grad_q_abs = fabsf(ga) >= prm.grad_abs_thresh;
  const float ms = max_scale3(log_scales + 3 * (size_t)i);
  const bool clone_q = ms <= prm.clone_max_scale;
  const bool metric = importance[i] > prm.importance_threshold;
  clone_flag[i] = (metric && clone_q && grad_q) ? 1u : 0u;
  split_flag[i] = (metric && !clone_q && grad_q_abs) ? 1u : 0u;
}

// Pre-prune rows: original rows that are not split sources keep their order,
// then the clones (source order), then split_factor children per source
// (source order, children consecutive).  kind: 0 kept, 1 clone, 2 child;
// child: the child's index into the normals array.
__global__ void __launch_bounds__(256)
densify_layout_kernel(int32_t P, int32_t factor, const uint32_t* __restrict__ clone_incl,
                      const uint32_t* __restrict__ split_incl, int32_t* __restrict__ l2_src,
                      int32_t* __restrict__ l2_kind, int32_t* __restrict__ l2_child) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const uint32_t nc = clone_incl[P - 1], ns = split_incl[P - 1];
  const uint32_t cs = clone_incl[i], ss = split_incl[i];
  const uint32_t c_ex = cs - (i ? clone_incl[i - 1] : 0u);
  const uint32_t s_ex = ss - (i ? split_incl[i - 1] : 0u);
  const uint32_t s_before = ss - s_ex;
  const uint32_t base = (uint32_t)P - ns;  // kept originals
  if (!s_ex) {
    const uint32_t r = (uint32_t)i - s_before;
    l2_src[r] = i;
    l2_kind[r] = 0;
    l2_child[r] = -1;
  } else {
    for (int k = 0; k < factor; ++k) {
      const uint32_t ch = s_before * (uint32_t)factor + (uint32_t)k;
      const uint32_t r = base + nc + ch;
      l2_src[r] = i;
      l2_kind[r] = 2;
      l2_child[r] = (int32_t)ch;
    }
  }
  if (c_ex) {
    const uint32_t r = base + (cs - 1u);
    l2_src[r] = i;
    l2_kind[r] = 1;
    l2_child[r] = -1;
  }
}

// Prune candidates among the pre-prune rows (opacity, screen and world
// tests of :698-708) and their keys for the budgeted weighted removal: the
// k smallest of (-log u) * (1e-6 + (1 - score)) are a sample without
// replacement with probabilities proportional to 1 / (1e-6 + (1 - score))
// (Efraimidis-Spirakis); other rows get key 0xFFFFFFFF.
__global__ void __launch_bounds__(256)
densify_prune_keys_kernel(int32_t P2, fgs_densify_params prm, int32_t any_appended,
                          const int32_t* __restrict__ l2_src, const int32_t* __restrict__ l2_kind,
                          const float* __restrict__ logits, const float* __restrict__ log_scales,
                          const float* __restrict__ max_radii2d,
                          const float* __restrict__ pruning, const float* __restrict__ uniforms,
                          uint64_t* __restrict__ keys, uint32_t* __restrict__ cand) {
  const int r = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= P2) return;
  const int32_t s = l2_src ? l2_src[r] : r;
  const int32_t kind = l2_kind ? l2_kind[r] : 0;
  const float o = sigmoid_det(logits[s]);
  const float* ls = log_scales + 3 * (size_t)s;
  float ms;
  if (kind == 2) {
    const float div = 0.8f * (float)prm.split_factor;
    ms = fmaxf(fmaxf(det_expf(child_log_scale(ls[0], div)), det_expf(child_log_scale(ls[1], div))),
               det_expf(child_log_scale(ls[2], div)));
  } else {
    ms = max_scale3(ls);
  }
  bool c = o < prm.min_opacity;
  // max_radii2d restarts at zero whenever rows are appended (:470-480)
  if (prm.max_screen_size > 0.0f && !any_appended) c = c || max_radii2d[s] > prm.max_screen_size;
  if (prm.world_max_scale > 0.0f) c = c || ms > prm.world_max_scale;
  cand[r] = c ? 1u : 0u;
  uint64_t key = 0xFFFFFFFFull;
  if (c && pruning) {
    const float u = 1.0f - uniforms[r];  // (0, 1]
    const float inv_w = 1.0e-6f + (1.0f - pruning[s]);
    const float k = (-det_logf(u)) * inv_w;
    key = (uint64_t)__float_as_uint(fmaxf(k, 0.0f));
  }
  keys[r] = key;
}

// keep[r] = 0 for the first k rows of the sorted order, 1 otherwise.
__global__ void __launch_bounds__(256)
densify_select_kernel(int32_t P2, int64_t k, const uint32_t* __restrict__ sorted_rows,
                      uint32_t* __restrict__ keep) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= P2) return;
  const uint32_t r = sorted_rows[j];
  if (r < (uint32_t)P2) keep[r] = j < k ? 0u : 1u;
}

__global__ void __launch_bounds__(256)
densify_compact_kernel(int32_t P2, const uint32_t* __restrict__ keep,
                       const uint32_t* __restrict__ keep_incl, int32_t* __restrict__ rows) {
  const int r = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (r >= P2 || !keep[r]) return;
  // rows holds keep_incl[P2 - 1] entries; a scan whose wait gave up can leave
  // other prefixes above it, which are dropped
  const uint32_t at = keep_incl[r] - 1u;
  if (at < keep_incl[P2 - 1]) rows[at] = r;
}

// Final rows: row f comes from pre-prune row rows[f] (identity when NULL),
// which comes from source l2_src (identity when NULL) as kind l2_kind.
// One thread per (row, array) element group: the arrays are walked by
// blockIdx.y.
struct BuildArray {
  const float* src;
  float* dst;
  int32_t width;   // floats per row
  int32_t policy;  // 0 copy, 1 zero for appended rows, 2 zero, 3 zero if reset else copy
};
constexpr int kMaxBuildArrays = 24;
struct BuildArrays {
  BuildArray a[kMaxBuildArrays];
  int32_t n;
};

__global__ void __launch_bounds__(256)
densify_gather_kernel(int32_t P_new, BuildArrays arrs, int32_t reset_stats,
                      const int32_t* __restrict__ rows, const int32_t* __restrict__ l2_src,
                      const int32_t* __restrict__ l2_kind) {
  const BuildArray A = arrs.a[blockIdx.y];
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)P_new * A.width;
  if (e >= total) return;
  const int64_t f = e / A.width;
  const int c = (int)(e - f * A.width);
  const int32_t r = rows ? rows[f] : (int32_t)f;
  const int32_t s = l2_src ? l2_src[r] : r;
  const int32_t kind = l2_kind ? l2_kind[r] : 0;
  bool zero = false;
  if (A.policy == 1) zero = kind != 0;
  else if (A.policy == 2) zero = true;
  else if (A.policy == 3) zero = reset_stats != 0;
  A.dst[e] = zero ? 0.0f : A.src[(size_t)s * A.width + c];
}

__global__ void __launch_bounds__(256)
densify_tmp_radii_kernel(int32_t P_new, const int32_t* __restrict__ rows,
                         const int32_t* __restrict__ l2_src, const int32_t* __restrict__ src,
                         int32_t* __restrict__ dst) {
  const int f = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (f >= P_new) return;
  const int32_t r = rows ? rows[f] : f;
  dst[f] = src[l2_src ? l2_src[r] : r];
}

// Means, log scales and opacity logits of the new rows: split children get
// mean + R(q) (s * z) and log(exp(ls) / (0.8 factor)) (:571-583); every
// row's opacity goes through logit(min(sigmoid(x), cap)) when cap > 0
// (:619-637).  R(q) as quat_to_rotmat_np (:189-203).
__global__ void __launch_bounds__(256)
densify_geometry_kernel(int32_t P_new, int32_t factor, float cap, const int32_t* __restrict__ rows,
                        const int32_t* __restrict__ l2_src, const int32_t* __restrict__ l2_kind,
                        const int32_t* __restrict__ l2_child, const float* __restrict__ means,
                        const float* __restrict__ log_scales, const float* __restrict__ rotations,
                        const float* __restrict__ logits, const float* __restrict__ normals,
                        float* __restrict__ d_means, float* __restrict__ d_log_scales,
                        float* __restrict__ d_logits) {
  const int f = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (f >= P_new) return;
  const int32_t r = rows ? rows[f] : f;
  const int32_t s = l2_src ? l2_src[r] : r;
  const int32_t kind = l2_kind ? l2_kind[r] : 0;
  const float* m = means + 3 * (size_t)s;
  const float* ls = log_scales + 3 * (size_t)s;
  float nm[3] = {m[0], m[1], m[2]};
  float nls[3] = {ls[0], ls[1], ls[2]};
  if (kind == 2) {
    const float* q = rotations + 4 * (size_t)s;
    const float nrm = __builtin_sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    const float dn = fmaxf(nrm, 1.0e-8f);
    const float w = q[0] / dn, x = q[1] / dn, y = q[2] / dn, z = q[3] / dn;
    float R[3][3];
    R[0][0] = 1.0f - 2.0f * (y * y + z * z);
    R[0][1] = 2.0f * (x * y - z * w);
    R[0][2] = 2.0f * (x * z + y * w);
    R[1][0] = 2.0f * (x * y + z * w);
    R[1][1] = 1.0f - 2.0f * (x * x + z * z);
    R[1][2] = 2.0f * (y * z - x * w);
    R[2][0] = 2.0f * (x * z - y * w);
    R[2][1] = 2.0f * (y * z + x * w);
    R[2][2] = 1.0f - 2.0f * (x * x + y * y);
    const float* zc = normals + 3 * (size_t)l2_child[r];
    float l[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) l[j] = det_expf(ls[j]) * zc[j];
    const float div = 0.8f * (float)factor;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      nm[i] = m[i] + (R[i][0] * l[0] + R[i][1] * l[1] + R[i][2] * l[2]);
      nls[i] = child_log_scale(ls[i], div);
    }
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    d_means[3 * (size_t)f + i] = nm[i];
    d_log_scales[3 * (size_t)f + i] = nls[i];
  }
  float lg = logits[s];
  if (cap > 0.0f) lg = logit_det(fminf(sigmoid_det(lg), cap));
  d_logits[f] = lg;
}

__global__ void __launch_bounds__(256)
opacity_cap_kernel(int32_t P, float cap, float* __restrict__ logits, float* __restrict__ m,
                   float* __restrict__ v) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  logits[i] = logit_det(fminf(sigmoid_det(logits[i]), cap));
  if (m) m[i] = 0.0f;
  if (v) v[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Scores (:279-340).
// ---------------------------------------------------------------------------
// Ordered-int encodings for float min/max by integer atomics.
__device__ __forceinline__ uint32_t ord_f(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unord_f(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// Wave-wide float min / max / double sum (butterfly; every lane ends with the
// result).  fminf / fmaxf drop NaN operands, as the restatement's scan does.
__device__ __forceinline__ void wave_min_max(float& mn, float& mx) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  }
}
__device__ __forceinline__ double wave_sum_f64(double x) {
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
  return x;
}

// Metric-map workspace: the per-pixel L1 map, then one (sum, min, max)
// partial per block, then the reduced (min, max).
constexpr int kMetricT = 256;
constexpr int kMetricPix = 4;  // pixels per thread, kMetricT apart
constexpr int64_t kMetricBlockPix = (int64_t)kMetricT * kMetricPix;
struct MetricWs {
  float* map;
  double* bsum;
  float* bmin;
  float* bmax;
  float* stat;  // [0] min, [1] max
};

__host__ __device__ inline int64_t metric_blocks(int64_t HW) {
  return (HW + kMetricBlockPix - 1) / kMetricBlockPix;
}

// l = (|p0 - t0| + |p1 - t1| + ...) / C per pixel (l1_map_chw, :262-270),
// and per block: the sum of every |pred - target| (double), min l, max l.
template <int kC>
__global__ void __launch_bounds__(kMetricT)
metric_l1_kernel(int32_t C_rt, int64_t HW, const float* __restrict__ pred,
                 const float* __restrict__ target, MetricWs ws) {
  __shared__ double s_sum[kMetricT / kWave];
  __shared__ float s_mn[kMetricT / kWave], s_mx[kMetricT / kWave];
  const int C = kC > 0 ? kC : C_rt;
  const int64_t base = (int64_t)blockIdx.x * kMetricBlockPix + threadIdx.x;
  double part = 0.0;
  float mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMetricPix; ++k) {
    const int64_t p = base + (int64_t)k * kMetricT;
    if (p < HW) {
      float acc = 0.0f;
      for (int c = 0; c < C; ++c) {
        const float d = fabsf(pred[(size_t)c * HW + p] - target[(size_t)c * HW + p]);
        acc = acc + d;
        part += (double)d;
      }
      const float l = acc / (float)C;
      ws.map[p] = l;
      mn = fminf(mn, l);
      mx = fmaxf(mx, l);
    }
  }
  part = wave_sum_f64(part);
  wave_min_max(mn, mx);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_sum[w] = part;
    s_mn[w] = mn;
    s_mx[w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double b = s_sum[0];
    float bmn = s_mn[0], bmx = s_mx[0];
    for (int i = 1; i < kMetricT / kWave; ++i) {
      b += s_sum[i];
      bmn = fminf(bmn, s_mn[i]);
      bmx = fmaxf(bmx, s_mx[i]);
    }
    ws.bsum[blockIdx.x] = b;
    ws.bmin[blockIdx.x] = bmn;
    ws.bmax[blockIdx.x] = bmx;
  }
}

// One block: the block partials reduced in a fixed order (so the loss is the
// same on every run), min / max to ws.stat, loss = sum / (C * HW).
__global__ void __launch_bounds__(kMetricT)
metric_reduce_kernel(int64_t nb, int64_t count, MetricWs ws, float* __restrict__ loss) {
  __shared__ double s_sum[kMetricT / kWave];
  __shared__ float s_mn[kMetricT / kWave], s_mx[kMetricT / kWave];
  double part = 0.0;
  float mn = INFINITY, mx = -INFINITY;
  for (int64_t b = threadIdx.x; b < nb; b += kMetricT) {
    part += ws.bsum[b];
    mn = fminf(mn, ws.bmin[b]);
    mx = fmaxf(mx, ws.bmax[b]);
  }
  part = wave_sum_f64(part);
  wave_min_max(mn, mx);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_sum[w] = part;
    s_mn[w] = mn;
    s_mx[w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = s_sum[0];
    float bmn = s_mn[0], bmx = s_mx[0];
    for (int i = 1; i < kMetricT / kWave; ++i) {
      s += s_sum[i];
      bmn = fminf(bmn, s_mn[i]);
      bmx = fmaxf(bmx, s_mx[i]);
    }
    ws.stat[0] = bmn;
    ws.stat[1] = bmx;
    *loss = (float)(s / (double)count);
  }
}

// metric_map = (l - min) / max(max - min, 1e-6) > loss_thresh
// (normalized_positive_map, :262-270).
__global__ void __launch_bounds__(kMetricT)
metric_map_kernel(int64_t HW, float loss_thresh, MetricWs ws, int32_t* __restrict__ metric_map) {
  const float mn = ws.stat[0], mx = ws.stat[1];
  const float dn = fmaxf(mx - mn, 1.0e-6f);
  const int64_t base = (int64_t)blockIdx.x * kMetricBlockPix + threadIdx.x;
#pragma unroll
  for (int k = 0; k < kMetricPix; ++k) {
    const int64_t p = base + (int64_t)k * kMetricT;
    if (p < HW) metric_map[p] = ((ws.map[p] - mn) / dn > loss_thresh) ? 1 : 0;
  }
}

// counts += metric_count; score += loss * metric_count (float32).
__global__ void __launch_bounds__(256)
score_accumulate_kernel(int32_t P, const int32_t* __restrict__ metric_count,
                        const float* __restrict__ loss, float* __restrict__ counts,
                        float* __restrict__ score) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const float mc = (float)metric_count[i];
  counts[i] = counts[i] + mc;
  score[i] = score[i] + (*loss) * mc;
}

// min / max of x[0..P) into mm (ordered-int atomics, one pair per block; the
// result does not depend on the order).
__global__ void __launch_bounds__(kMetricT)
minmax_kernel(int32_t P, const float* __restrict__ x, uint32_t* __restrict__ mm) {
  __shared__ float s_mn[kMetricT / kWave], s_mx[kMetricT / kWave];
  const int64_t base = (int64_t)blockIdx.x * kMetricBlockPix + threadIdx.x;
  float mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMetricPix; ++k) {
    const int64_t i = base + (int64_t)k * kMetricT;
    if (i < P) {
      mn = fminf(mn, x[i]);
      mx = fmaxf(mx, x[i]);
    }
  }
  wave_min_max(mn, mx);
  const int w = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_mn[w] = mn;
    s_mx[w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bmn = s_mn[0], bmx = s_mx[0];
    for (int i = 1; i < kMetricT / kWave; ++i) {
      bmn = fminf(bmn, s_mn[i]);
      bmx = fmaxf(bmx, s_mx[i]);
    }
    atomicMin(&mm[0], ord_f(bmn));
    atomicMax(&mm[1], ord_f(bmx));
  }
}

// pruning = (score - min) / max(max - min, 1e-6); importance =
// floor(counts / max(n, 1)).
__global__ void __launch_bounds__(256)
score_finalize_kernel(int32_t P, int32_t n_cams, const uint32_t* __restrict__ mm,
                      const float* __restrict__ counts, const float* __restrict__ score,
                      float* __restrict__ importance, float* __restrict__ pruning) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const float mn = unord_f(mm[0]), mx = unord_f(mm[1]);
  pruning[i] = (score[i] - mn) / fmaxf(mx - mn, 1.0e-6f);
  if (importance) importance[i] = floorf(counts[i] / (float)(n_cams > 1 ? n_cams : 1));
}

// Final prune (:745-793): prune = opacity < min_opacity || score > thresh;
// priority keys sort ascending in order of descending opacity - score (ties
// by row).
__global__ void __launch_bounds__(256)
final_prune_kernel(int32_t P, float min_opacity, float score_thresh,
                   const float* __restrict__ logits, const float* __restrict__ pruning,
                   uint32_t* __restrict__ prune, uint64_t* __restrict__ keys) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= P) return;
  const float o = sigmoid_det(logits[i]);
  const float s = pruning[i];
  prune[i] = (o < min_opacity || s > score_thresh) ? 1u : 0u;
  keys[i] = (uint64_t)(~ord_f(o - s));
}

__global__ void __launch_bounds__(256)
keep_first_kernel(int32_t P, int64_t k, const uint32_t* __restrict__ sorted_rows,
                  uint32_t* __restrict__ keep) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= P) return;
  const uint32_t r = sorted_rows[j];
  if (r < (uint32_t)P) keep[r] = j < k ? 1u : 0u;
}

__global__ void __launch_bounds__(256)
invert_flags_kernel(int32_t n, const uint32_t* __restrict__ in, uint32_t* __restrict__ out) {
  const int i = (int)(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) out[i] = in[i] ? 0u : 1u;
}

}  // namespace fgs

using namespace fgs;

static unsigned blocks_for(int64_t n) { return ceil_div_u(n, 256); }

extern "C" int32_t fgs_densify_stats(int32_t P, const int32_t* radii, const float* d_viewspace,
                                     float* max_radii2d, float* grad_accum, float* grad_accum_abs,
                                     float* denom, int32_t* tmp_radii, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_stats: P < 0");
  if (P == 0) return FGS_OK;
  if (!radii || !d_viewspace || !max_radii2d || !grad_accum || !grad_accum_abs || !denom ||
      !tmp_radii)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_stats: null pointer");
  hipLaunchKernelGGL(densify_stats_kernel, dim3(blocks_for(P)), dim3(256), 0, (hipStream_t)stream,
                     P, radii, d_viewspace, max_radii2d, grad_accum, grad_accum_abs, denom,
                     tmp_radii);
  return check_launch("densify_stats_kernel");
}

extern "C" int32_t fgs_densify_classify(int32_t P, const fgs_densify_params* prm,
                                        const float* grad_accum, const float* grad_accum_abs,
                                        const float* denom, const float* log_scales,
                                        const float* importance, uint32_t* clone_flag,
                                        uint32_t* split_flag, void* stream) {
  if (P < 0 || !prm) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_classify: bad arguments");
  if (P == 0) return FGS_OK;
  if (!grad_accum || !grad_accum_abs || !denom || !log_scales || !importance || !clone_flag ||
      !split_flag)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_classify: null pointer");
  hipLaunchKernelGGL(densify_classify_kernel, dim3(blocks_for(P)), dim3(256), 0,
                     (hipStream_t)stream, P, *prm, grad_accum, grad_accum_abs, denom, log_scales,
                     importance, clone_flag, split_flag);
  return check_launch("densify_classify_kernel");
}

extern "C" int32_t fgs_densify_layout(int32_t P, int32_t split_factor, const uint32_t* clone_incl,
                                      const uint32_t* split_incl, int32_t* l2_src,
                                      int32_t* l2_kind, int32_t* l2_child, void* stream) {
  if (P < 0 || split_factor < 1)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_layout: bad arguments");
  if (P == 0) return FGS_OK;
  if (!clone_incl || !split_incl || !l2_src || !l2_kind || !l2_child)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_layout: null pointer");
  hipLaunchKernelGGL(densify_layout_kernel, dim3(blocks_for(P)), dim3(256), 0, (hipStream_t)stream,
                     P, split_factor, clone_incl, split_incl, l2_src, l2_kind, l2_child);
  return check_launch("densify_layout_kernel");
}

extern "C" int32_t fgs_densify_prune_keys(int32_t P2, const fgs_densify_params* prm,
                                          int32_t any_appended, const int32_t* l2_src,
                                          const int32_t* l2_kind, const float* opacity_logits,
                                          const float* log_scales, const float* max_radii2d,
                                          const float* pruning_score, const float* uniforms,
                                          uint64_t* keys, uint32_t* candidate, void* stream) {
  if (P2 < 0 || !prm) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_prune_keys: bad arguments");
  if (P2 == 0) return FGS_OK;
  if (!opacity_logits || !log_scales || !keys || !candidate || (pruning_score && !uniforms) ||
      (prm->max_screen_size > 0.0f && !any_appended && !max_radii2d) || (!l2_src != !l2_kind))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_prune_keys: null pointer");
  hipLaunchKernelGGL(densify_prune_keys_kernel, dim3(blocks_for(P2)), dim3(256), 0,
                     (hipStream_t)stream, P2, *prm, any_appended, l2_src, l2_kind, opacity_logits,
                     log_scales, max_radii2d, pruning_score, uniforms, keys, candidate);
  return check_launch("densify_prune_keys_kernel");
}

extern "C" int32_t fgs_densify_select(int32_t P2, int64_t k, const uint32_t* sorted_rows,
                                      uint32_t* keep, void* stream) {
  if (P2 < 0 || k < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_select: bad arguments");
  if (P2 == 0) return FGS_OK;
  if (!sorted_rows || !keep) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_select: null pointer");
  hipLaunchKernelGGL(densify_select_kernel, dim3(blocks_for(P2)), dim3(256), 0, (hipStream_t)stream,
                     P2, k, sorted_rows, keep);
  return check_launch("densify_select_kernel");
}

extern "C" int32_t fgs_densify_keep_first(int32_t P, int64_t k, const uint32_t* sorted_rows,
                                          uint32_t* keep, void* stream) {
  if (P < 0 || k < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_keep_first: bad arguments");
  if (P == 0) return FGS_OK;
  if (!sorted_rows || !keep) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_keep_first: null pointer");
  hipLaunchKernelGGL(keep_first_kernel, dim3(blocks_for(P)), dim3(256), 0, (hipStream_t)stream, P, k,
                     sorted_rows, keep);
  return check_launch("keep_first_kernel");
}

extern "C" int32_t fgs_invert_flags(int32_t n, const uint32_t* in, uint32_t* out, void* stream) {
  if (n < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_invert_flags: n < 0");
  if (n == 0) return FGS_OK;
  if (!in || !out) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_invert_flags: null pointer");
  hipLaunchKernelGGL(invert_flags_kernel, dim3(blocks_for(n)), dim3(256), 0, (hipStream_t)stream, n,
                     in, out);
  return check_launch("invert_flags_kernel");
}

extern "C" int32_t fgs_densify_compact(int32_t P2, const uint32_t* keep, const uint32_t* keep_incl,
                                       int32_t* rows, void* stream) {
  if (P2 < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_compact: P2 < 0");
  if (P2 == 0) return FGS_OK;
  if (!keep || !keep_incl || !rows)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_compact: null pointer");
  hipLaunchKernelGGL(densify_compact_kernel, dim3(blocks_for(P2)), dim3(256), 0, (hipStream_t)stream,
                     P2, keep, keep_incl, rows);
  return check_launch("densify_compact_kernel");
}

extern "C" int32_t fgs_densify_build(const fgs_densify_build_io* io, void* stream) {
  if (!io || io->P_new < 0 || io->split_factor < 1 || io->sh_row < 0)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_build: bad arguments");
  if (io->P_new == 0) return FGS_OK;
  if (!io->means3d || !io->features_dc || !io->opacity_logits || !io->log_scales ||
      !io->rotations || !io->d_means3d || !io->d_features_dc || !io->d_opacity_logits ||
      !io->d_log_scales || !io->d_rotations || (io->sh_row > 0 && (!io->features_rest ||
                                                                    !io->d_features_rest)))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_build: null parameter pointer");
  if (!io->l2_src != !io->l2_kind || (io->l2_src && (!io->l2_child || !io->normals)))
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_densify_build: inconsistent row map");
  hipStream_t st = (hipStream_t)stream;
  // parameter order of the Adam moments: means3d, features_dc, features_rest,
  // opacity_logits, log_scales, rotations
  const int32_t widths[6] = {3, 3, io->sh_row, 1, 3, 4};
  BuildArrays arrs{};
  int n = 0;
  auto add = [&](const float* s, float* d, int32_t w, int32_t pol) {
    if (w <= 0 || !s || !d) return;
    arrs.a[n++] = BuildArray{s, d, w, pol};
  };
  add(io->features_dc, io->d_features_dc, 3, 0);
  add(io->features_rest, io->d_features_rest, io->sh_row, 0);
  add(io->rotations, io->d_rotations, 4, 0);
  for (int k = 0; k < 6; ++k) {
    // opacity moments restart at zero when the opacities are capped
    const int32_t pol = (k == 3 && io->opacity_cap > 0.0f) ? 2 : 1;
    add(io->exp_avg[k], io->d_exp_avg[k], widths[k], pol);
    add(io->exp_avg_sq[k], io->d_exp_avg_sq[k], widths[k], pol);
  }
  add(io->max_radii2d, io->d_max_radii2d, 1, 3);
  add(io->grad_accum, io->d_grad_accum, 1, 3);
  add(io->grad_accum_abs, io->d_grad_accum_abs, 1, 3);
  add(io->denom, io->d_denom, 1, 3);
  arrs.n = n;
  int32_t maxw = 1;
  for (int k = 0; k < n; ++k) maxw = arrs.a[k].width > maxw ? arrs.a[k].width : maxw;
  if (n > 0)
    hipLaunchKernelGGL(densify_gather_kernel,
                       dim3(ceil_div_u((int64_t)io->P_new * maxw, 256), (unsigned)n), dim3(256), 0,
                       st, io->P_new, arrs, io->reset_stats, io->rows, io->l2_src, io->l2_kind);
  if (io->tmp_radii && io->d_tmp_radii)
    hipLaunchKernelGGL(densify_tmp_radii_kernel, dim3(blocks_for(io->P_new)), dim3(256), 0, st,
                       io->P_new, io->rows, io->l2_src, io->tmp_radii, io->d_tmp_radii);
  hipLaunchKernelGGL(densify_geometry_kernel, dim3(blocks_for(io->P_new)), dim3(256), 0, st,
                     io->P_new, io->split_factor, io->opacity_cap, io->rows, io->l2_src,
                     io->l2_kind, io->l2_child, io->means3d, io->log_scales, io->rotations,
                     io->opacity_logits, io->normals, io->d_means3d, io->d_log_scales,
                     io->d_opacity_logits);
  return check_launch("densify_build");
}

extern "C" int32_t fgs_opacity_cap(int32_t P, float cap, float* opacity_logits, float* exp_avg,
                                   float* exp_avg_sq, void* stream) {
  if (P < 0 || !(cap > 0.0f)) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_opacity_cap: bad arguments");
  if (P == 0) return FGS_OK;
  if (!opacity_logits) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_opacity_cap: null pointer");
  hipLaunchKernelGGL(opacity_cap_kernel, dim3(blocks_for(P)), dim3(256), 0, (hipStream_t)stream, P,
                     cap, opacity_logits, exp_avg, exp_avg_sq);
  return check_launch("opacity_cap_kernel");
}

static size_t metric_ws_layout(int64_t HW, MetricWs* ws, char* w) {
  const int64_t nb = metric_blocks(HW);
  size_t off = (size_t)((HW * 4 + 255) & ~255);
  const size_t o_sum = off;
  off += (size_t)((nb * 8 + 255) & ~255);
  const size_t o_min = off;
  off += (size_t)((nb * 4 + 255) & ~255);
  const size_t o_max = off;
  off += (size_t)((nb * 4 + 255) & ~255);
  const size_t o_stat = off;
  off += 256;
  if (ws) {
    ws->map = (float*)w;
    ws->bsum = (double*)(w + o_sum);
    ws->bmin = (float*)(w + o_min);
    ws->bmax = (float*)(w + o_max);
    ws->stat = (float*)(w + o_stat);
  }
  return off;
}

extern "C" size_t fgs_metric_map_workspace_bytes(int64_t HW) {
  return HW > 0 ? metric_ws_layout(HW, nullptr, nullptr) : 0;
}

extern "C" int32_t fgs_metric_map(int32_t C, int64_t HW, const float* pred, const float* target,
                                  float loss_thresh, void* workspace, int32_t* metric_map,
                                  float* photometric_loss, void* stream) {
  if (C <= 0 || HW <= 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_metric_map: bad sizes");
  if (!pred || !target || !workspace || !metric_map || !photometric_loss)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_metric_map: null pointer");
  hipStream_t st = (hipStream_t)stream;
  MetricWs ws;
  metric_ws_layout(HW, &ws, (char*)workspace);
  const int64_t nb = metric_blocks(HW);
  if (nb > 0x7FFFFFFF) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_metric_map: HW too large");
  if (C == 3)
    hipLaunchKernelGGL(metric_l1_kernel<3>, dim3((unsigned)nb), dim3(kMetricT), 0, st, C, HW,
                       pred, target, ws);
  else
    hipLaunchKernelGGL(metric_l1_kernel<0>, dim3((unsigned)nb), dim3(kMetricT), 0, st, C, HW,
                       pred, target, ws);
  hipLaunchKernelGGL(metric_reduce_kernel, dim3(1), dim3(kMetricT), 0, st, nb, (int64_t)C * HW,
                     ws, photometric_loss);
  hipLaunchKernelGGL(metric_map_kernel, dim3((unsigned)nb), dim3(kMetricT), 0, st, HW,
                     loss_thresh, ws, metric_map);
  return check_launch("metric_map");
}

extern "C" int32_t fgs_score_accumulate(int32_t P, const int32_t* metric_count,
                                        const float* photometric_loss, float* counts,
                                        float* score, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_score_accumulate: P < 0");
  if (P == 0) return FGS_OK;
  if (!metric_count || !photometric_loss || !counts || !score)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_score_accumulate: null pointer");
  hipLaunchKernelGGL(score_accumulate_kernel, dim3(blocks_for(P)), dim3(256), 0,
                     (hipStream_t)stream, P, metric_count, photometric_loss, counts, score);
  return check_launch("score_accumulate_kernel");
}

extern "C" int32_t fgs_score_finalize(int32_t P, int32_t n_cams, const float* counts,
                                      const float* score, float* importance, float* pruning,
                                      uint32_t* minmax_ws, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_score_finalize: P < 0");
  if (P == 0) return FGS_OK;
  if (!counts || !score || !pruning || !minmax_ws)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_score_finalize: null pointer");
  hipStream_t st = (hipStream_t)stream;
  fgs_fill_u32(minmax_ws, 0xFFFFFFFFu, 1, stream);
  fgs_fill_u32(minmax_ws + 1, 0u, 1, stream);
  hipLaunchKernelGGL(minmax_kernel, dim3((unsigned)metric_blocks(P)), dim3(kMetricT), 0, st, P,
                     score, minmax_ws);
  hipLaunchKernelGGL(score_finalize_kernel, dim3(blocks_for(P)), dim3(256), 0, st, P, n_cams,
                     minmax_ws, counts, score, importance, pruning);
  return check_launch("score_finalize");
}

extern "C" int32_t fgs_final_prune_mask(int32_t P, float min_opacity, float score_thresh,
                                        const float* opacity_logits, const float* pruning_score,
                                        uint32_t* prune, uint64_t* priority_keys, void* stream) {
  if (P < 0) return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_final_prune_mask: P < 0");
  if (P == 0) return FGS_OK;
  if (!opacity_logits || !pruning_score || !prune || !priority_keys)
    return set_error(FGS_ERR_INVALID_ARGUMENT, "fgs_final_prune_mask: null pointer");
  hipLaunchKernelGGL(final_prune_kernel, dim3(blocks_for(P)), dim3(256), 0, (hipStream_t)stream, P,
                     min_opacity, score_thresh, opacity_logits, pruning_score, prune,
                     priority_keys);
  return check_launch("final_prune_kernel");
}
