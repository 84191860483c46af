/* fgs_densify_oracle.c -- CPU restatement of the densification kernels
 * (TEST INFRASTRUCTURE ONLY; only tests/ load it, through oracle/densify.py).
 *
 * It follows the reference's numpy code of scripts/train_scanner_fastgs.py
 * expression by expression in float32 (no contraction), with the library's
 * deterministic exp/log (orc_expf / orc_logf of fgs_oracle.c), so the GPU
 * kernels must agree bit for bit:
 *   orc_densify_stats      update_densification_stats          :391-405
 *   orc_densify_classify   the qualifiers of densify_and_prune  :670-683
 *   orc_densify_keys       the prune tests of :697-708 and the weighted
 *                          removal keys (Efraimidis-Spirakis form of
 *                          rng.choice(p=...), :712-723)
 *   orc_densify_geometry   split children (:560-583) and cap_opacity_logits
 *                          (:619-637)
 *   orc_opacity_cap        cap/reset_opacity_logits              :619-658
 *   orc_metric_l1          l1_map_chw + normalized_positive_map  :262-270
 *   orc_score_finalize     the score normalisation                :334-339
 *   orc_final_prune_mask   final_prune_fastgs masks/priority     :754-776
 * Always float: the file is compiled into both oracle builds unchanged. */
#include <math.h>
#include <stdint.h>
#include <string.h>

float orc_expf(float x);
float orc_logf(float x);

static float sigmoid_o(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

static float logit_o(float p) {
  const float lo = 1.0e-6f, hi = 0.999999f;
  p = fminf(fmaxf(p, lo), hi);
  return orc_logf(p / (1.0f - p));
}

static float max_scale3_o(const float* ls) {
  return fmaxf(fmaxf(orc_expf(ls[0]), orc_expf(ls[1])), orc_expf(ls[2]));
}

static float child_log_scale_o(float ls, float div) { return orc_logf(orc_expf(ls) / div); }

void orc_densify_stats(int32_t P, const int32_t* radii, const float* dvs, float* max_radii2d,
                       float* acc, float* acc_abs, float* denom, int32_t* tmp_radii) {
  for (int32_t i = 0; i < P; ++i) {
    const int32_t r = radii[i];
    tmp_radii[i] = r;
    if (r <= 0) continue;
    const float* g = dvs + 4 * (size_t)i;
    max_radii2d[i] = fmaxf(max_radii2d[i], (float)r);
    acc[i] = acc[i] + sqrtf(g[0] * g[0] + g[1] * g[1]);
    acc_abs[i] = acc_abs[i] + sqrtf(g[2] * g[2] + g[3] * g[3]);
    denom[i] = denom[i] + 1.0f;
  }
}

/* prm: grad_thresh, grad_abs_thresh, clone_max_scale, importance_threshold */
void orc_densify_classify(int32_t P, const float* prm, const float* acc, const float* acc_abs,
                          const float* denom, const float* log_scales, const float* importance,
                          uint32_t* clone_flag, uint32_t* split_flag) {
  for (int32_t i = 0; i < P; ++i) {
    const float d = fmaxf(denom[i], 1.0f);
    const float gv = acc[i] / d, ga = acc_abs[i] / d;
    const int grad_q = fabsf(gv) >= prm[0];
    const int grad_q_abs = fabsf(ga) >= prm[1];
    const float ms = max_scale3_o(log_scales + 3 * (size_t)i);
    const int clone_q = ms <= prm[2];
    const int metric = importance[i] > prm[3];
    clone_flag[i] = (metric && clone_q && grad_q) ? 1u : 0u;
    split_flag[i] = (metric && !clone_q && grad_q_abs) ? 1u : 0u;
  }
}

/* prm: min_opacity, max_screen_size, world_max_scale, split_factor */
void orc_densify_keys(int32_t P2, const float* prm, int32_t any_appended, const int32_t* l2_src,
                      const int32_t* l2_kind, const float* logits, const float* log_scales,
                      const float* max_radii2d, const float* pruning, const float* uniforms,
                      uint64_t* keys, uint32_t* cand) {
  for (int32_t r = 0; r < P2; ++r) {
    const int32_t s = l2_src[r];
    const int32_t kind = l2_kind[r];
    const float o = sigmoid_o(logits[s]);
    const float* ls = log_scales + 3 * (size_t)s;
    float ms;
    if (kind == 2) {
      const float div = 0.8f * prm[3];
      ms = fmaxf(fmaxf(orc_expf(child_log_scale_o(ls[0], div)),
                       orc_expf(child_log_scale_o(ls[1], div))),
                 orc_expf(child_log_scale_o(ls[2], div)));
    } else {
      ms = max_scale3_o(ls);
    }
    int c = o < prm[0];
    if (prm[1] > 0.0f && !any_appended) c = c || max_radii2d[s] > prm[1];
    if (prm[2] > 0.0f) c = c || ms > prm[2];
    cand[r] = c ? 1u : 0u;
    uint64_t key = 0xFFFFFFFFull;
    if (c && pruning) {
      const float u = 1.0f - uniforms[r];
      const float inv_w = 1.0e-6f + (1.0f - pruning[s]);
      float k = (-orc_logf(u)) * inv_w;
      k = fmaxf(k, 0.0f);
      uint32_t bits;
      memcpy(&bits, &k, 4);
      key = bits;
    }
    keys[r] = key;
  }
}

/* New means3d / log_scales / opacity logits of the rows (src, kind, child). */
void orc_densify_geometry(int32_t n, int32_t factor, float cap, const int32_t* src,
                          const int32_t* kind, const int32_t* child, const float* means,
                          const float* log_scales, const float* rotations, const float* logits,
                          const float* normals, float* d_means, float* d_log_scales,
                          float* d_logits) {
  for (int32_t f = 0; f < n; ++f) {
    const int32_t s = src[f];
    const float* m = means + 3 * (size_t)s;
    const float* ls = log_scales + 3 * (size_t)s;
    float nm[3] = {m[0], m[1], m[2]};
    float nls[3] = {ls[0], ls[1], ls[2]};
    if (kind[f] == 2) {
      const float* q = rotations + 4 * (size_t)s;
      const float nrm = sqrtf(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
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
      const float* zc = normals + 3 * (size_t)child[f];
      float l[3];
      for (int j = 0; j < 3; ++j) l[j] = orc_expf(ls[j]) * zc[j];
      const float div = 0.8f * (float)factor;
      for (int i = 0; i < 3; ++i) {
        nm[i] = m[i] + (R[i][0] * l[0] + R[i][1] * l[1] + R[i][2] * l[2]);
        nls[i] = child_log_scale_o(ls[i], div);
      }
    }
    for (int i = 0; i < 3; ++i) {
      d_means[3 * (size_t)f + i] = nm[i];
      d_log_scales[3 * (size_t)f + i] = nls[i];
    }
    float lg = logits[s];
    if (cap > 0.0f) lg = logit_o(fminf(sigmoid_o(lg), cap));
    d_logits[f] = lg;
  }
}

void orc_opacity_cap(int32_t P, float cap, float* logits) {
  for (int32_t i = 0; i < P; ++i) logits[i] = logit_o(fminf(sigmoid_o(logits[i]), cap));
}

/* Per-pixel l (float) and the metric map; loss = mean |pred - target| summed
 * in double in pixel order (the GPU sums the same terms in another order, so
 * tests compare it to a tolerance). */
void orc_metric_l1(int32_t C, int64_t HW, const float* pred, const float* target,
                   float loss_thresh, int32_t* metric_map, float* loss) {
  float mn = INFINITY, mx = -INFINITY;
  double sum = 0.0;
  for (int64_t p = 0; p < HW; ++p) {
    float acc = 0.0f;
    for (int c = 0; c < C; ++c) {
      const float d = fabsf(pred[(size_t)c * HW + p] - target[(size_t)c * HW + p]);
      acc = acc + d;
      sum += (double)d;
    }
    const float l = acc / (float)C;
    mn = fminf(mn, l);
    mx = fmaxf(mx, l);
  }
  const float dn = fmaxf(mx - mn, 1.0e-6f);
  for (int64_t p = 0; p < HW; ++p) {
    float acc = 0.0f;
    for (int c = 0; c < C; ++c)
      acc = acc + fabsf(pred[(size_t)c * HW + p] - target[(size_t)c * HW + p]);
    const float l = acc / (float)C;
    metric_map[p] = ((l - mn) / dn > loss_thresh) ? 1 : 0;
  }
  *loss = (float)(sum / (double)((int64_t)C * HW));
}

void orc_score_accumulate(int32_t P, const int32_t* metric_count, float loss, float* counts,
                          float* score) {
  for (int32_t i = 0; i < P; ++i) {
    const float mc = (float)metric_count[i];
    counts[i] = counts[i] + mc;
    score[i] = score[i] + loss * mc;
  }
}

void orc_score_finalize(int32_t P, int32_t n_cams, const float* counts, const float* score,
                        float* importance, float* pruning) {
  float mn = INFINITY, mx = -INFINITY;
  for (int32_t i = 0; i < P; ++i) {
    mn = fminf(mn, score[i]);
    mx = fmaxf(mx, score[i]);
  }
  const float dn = fmaxf(mx - mn, 1.0e-6f);
  for (int32_t i = 0; i < P; ++i) {
    pruning[i] = (score[i] - mn) / dn;
    if (importance) importance[i] = floorf(counts[i] / (float)(n_cams > 1 ? n_cams : 1));
  }
}

/* prune flags and the keep priority opacity - score */
void orc_final_prune_mask(int32_t P, float min_opacity, float score_thresh, const float* logits,
                          const float* pruning, uint32_t* prune, float* priority) {
  for (int32_t i = 0; i < P; ++i) {
    const float o = sigmoid_o(logits[i]);
    const float s = pruning[i];
    prune[i] = (o < min_opacity || s > score_thresh) ? 1u : 0u;
    priority[i] = o - s;
  }
}
