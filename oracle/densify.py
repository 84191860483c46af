"""CPU restatement of FastGS densification and pruning (TEST INFRASTRUCTURE ONLY).

Only ``tests/`` import this module.  It follows the reference's numpy code of
scripts/train_scanner_fastgs.py step by step -- ``append_new_points`` /
``prune_points`` as concatenations and boolean takes (:470-511),
``densify_and_clone_fastgs`` / ``densify_and_split_fastgs`` (:514-587),
``densify_and_prune_fastgs`` (:661-742), ``final_prune_fastgs`` (:745-793),
``cap_opacity_logits`` (:619-637), the score helpers (:262-340) -- with every
float decision taken by the C restatement in ``fgs_densify_oracle.c`` (the
library's deterministic exp/log, float32, no contraction).

The reference's inconsistencies are resolved as the GPU does (documented in
``fastgs_core_amd/densify.py``): split sources are chosen among the pre-clone
rows, appended rows inherit their source's pruning score, ``tmp_radii``
follows its row.  The random draws are inputs: ``normals`` (standard normals
of the split children, scaled by the source's scales as
``rng.normal(0, scales)``) and ``uniforms`` (one per pre-prune row, the
Efraimidis-Spirakis keys that replace ``rng.choice(p=...)``).

Parity status: pinned by tests/test_densify_oracle.py (closed forms for the
statistics, the split geometry and the opacity cap; the exact inclusion
probabilities of successive weighted sampling for the removal keys; brute
force numpy for the metric map and the scores).
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_int64, c_void_p

import numpy as np

from .oracle import Oracle

PARAMS = ("means3d", "features_dc", "features_rest", "opacity_logits", "log_scales", "rotations")
STATS = ("max_radii2d", "grad_accum", "grad_accum_abs", "denom")


def _f(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return a.ctypes.data_as(c_void_p)


class DensifyOracle:
    def __init__(self):
        self.lib = Oracle(double=False).lib
        L = self.lib
        L.orc_densify_stats.argtypes = [c_int32] + [c_void_p] * 7
        L.orc_densify_classify.argtypes = [c_int32] + [c_void_p] * 8
        L.orc_densify_keys.argtypes = [c_int32, c_void_p, c_int32] + [c_void_p] * 9
        L.orc_densify_geometry.argtypes = [c_int32, c_int32, c_float] + [c_void_p] * 11
        L.orc_opacity_cap.argtypes = [c_int32, c_float, c_void_p]
        L.orc_metric_l1.argtypes = [c_int32, c_int64, c_void_p, c_void_p, c_float, c_void_p,
                                    c_void_p]
        L.orc_score_accumulate.argtypes = [c_int32, c_void_p, c_float, c_void_p, c_void_p]
        L.orc_score_finalize.argtypes = [c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]
        L.orc_final_prune_mask.argtypes = [c_int32, c_float, c_float, c_void_p, c_void_p, c_void_p,
                                           c_void_p]

    # ------------------------------------------------------------- statistics
    def update_stats(self, state, radii, d_viewspace):
        P = len(radii)
        r = np.ascontiguousarray(radii, dtype=np.int32)
        g = _f(d_viewspace)
        for n in STATS:
            state[n] = _f(state[n]).copy()
        state["tmp_radii"] = np.zeros(P, np.int32)
        self.lib.orc_densify_stats(P, _ptr(r), _ptr(g), _ptr(state["max_radii2d"]),
                                   _ptr(state["grad_accum"]), _ptr(state["grad_accum_abs"]),
                                   _ptr(state["denom"]), _ptr(state["tmp_radii"]))
        return state

    # -------------------------------------------------------------- densify
    def classify(self, cfg, scene_extent, state, log_scales, importance):
        P = len(importance)
        prm = np.array([cfg.grad_thresh, cfg.grad_abs_thresh, np.float32(cfg.dense * scene_extent),
                        cfg.importance_score_threshold], np.float32)
        cf = np.zeros(P, np.uint32)
        sf = np.zeros(P, np.uint32)
        self.lib.orc_densify_classify(P, _ptr(prm), _ptr(_f(state["grad_accum"])),
                                      _ptr(_f(state["grad_accum_abs"])), _ptr(_f(state["denom"])),
                                      _ptr(_f(log_scales)), _ptr(_f(importance)), _ptr(cf),
                                      _ptr(sf))
        return cf.astype(bool), sf.astype(bool)

    def densify_and_prune(self, cfg, scene_extent, model, adam, state, importance, pruning,
                          normals, uniforms):
        """model: name -> rows; adam: name -> (m, v); state: statistics and
        tmp_radii.  Returns the new (model, adam, state, info)."""
        P0 = len(model["means3d"])
        f = int(cfg.split_factor)
        clone, split = self.classify(cfg, scene_extent, state, model["log_scales"], importance)
        cl = np.flatnonzero(clone)
        sp = np.flatnonzero(split)
        nc, ns = len(cl), len(sp)
        # append clones, then split children; drop the split sources
        # (append_new_points + prune_points of :514-587 with the masks padded)
        keep0 = np.flatnonzero(~split)
        l2_src = np.concatenate([keep0, cl, np.repeat(sp, f)]).astype(np.int32)
        l2_kind = np.concatenate([np.zeros(len(keep0)), np.ones(nc), np.full(ns * f, 2)]).astype(np.int32)
        l2_child = np.concatenate([np.full(len(keep0) + nc, -1), np.arange(ns * f)]).astype(np.int32)
        P2 = len(l2_src)
        appended = (nc + ns) > 0
        prm = np.array([cfg.min_opacity, cfg.max_screen_size,
                        np.float32(cfg.max_world_scale_factor * scene_extent)
                        if cfg.max_world_scale_factor > 0 else 0.0, f], np.float32)
        keys = np.zeros(P2, np.uint64)
        cand = np.zeros(P2, np.uint32)
        use_scores = pruning is not None and np.size(pruning) > 0
        pr = _f(pruning) if use_scores else None
        un = _f(uniforms) if use_scores else None
        self.lib.orc_densify_keys(P2, _ptr(prm), int(appended), _ptr(l2_src), _ptr(l2_kind),
                                  _ptr(_f(model["opacity_logits"]).reshape(-1)),
                                  _ptr(_f(model["log_scales"])), _ptr(_f(state["max_radii2d"])),
                                  _ptr(pr) if use_scores else None,
                                  _ptr(un) if use_scores else None, _ptr(keys), _ptr(cand))
        to_remove = int(cand.sum())
        budget = int(cfg.prune_budget_factor * to_remove)
        k = min(budget, to_remove) if use_scores else 0
        keep = np.ones(P2, bool)
        if k > 0:
            order = np.argsort(keys, kind="stable")
            keep[order[:k]] = False
        rows = np.flatnonzero(keep)
        src, kind, child = l2_src[rows], l2_kind[rows], l2_child[rows]
        new = self._gather(model, adam, state, src, kind, child, f, normals, appended,
                           float(cfg.opacity_cap_after_densify))
        info = {"cloned": nc, "split_sources": ns, "split_children": ns * f,
                "total_prune_candidates": to_remove, "prune_budget": budget,
                "actual_removed": k, "points": len(rows)}
        return new + (info,)

    def _gather(self, model, adam, state, src, kind, child, f, normals, reset_stats, cap):
        n = len(src)
        nm = {}
        for p in ("features_dc", "features_rest", "rotations"):
            nm[p] = _f(model[p])[src]
        d_means = np.zeros((n, 3), np.float32)
        d_ls = np.zeros((n, 3), np.float32)
        d_lg = np.zeros(n, np.float32)
        lg = _f(model["opacity_logits"]).reshape(-1)
        nz = _f(normals).reshape(-1, 3) if normals is not None and np.size(normals) else \
            np.zeros((1, 3), np.float32)
        if n:
            self.lib.orc_densify_geometry(n, f, cap, _ptr(np.ascontiguousarray(src, np.int32)),
                                          _ptr(np.ascontiguousarray(kind, np.int32)),
                                          _ptr(np.ascontiguousarray(child, np.int32)),
                                          _ptr(_f(model["means3d"])), _ptr(_f(model["log_scales"])),
                                          _ptr(_f(model["rotations"])), _ptr(lg), _ptr(nz),
                                          _ptr(d_means), _ptr(d_ls), _ptr(d_lg))
        nm["means3d"] = d_means
        nm["log_scales"] = d_ls
        nm["opacity_logits"] = d_lg.reshape(-1, 1)
        na = {}
        for p in PARAMS:
            m, v = adam[p]
            m = _f(m)[src].copy()
            v = _f(v)[src].copy()
            m[kind != 0] = 0.0
            v[kind != 0] = 0.0
            if p == "opacity_logits" and cap > 0.0:
                m[:] = 0.0
                v[:] = 0.0
            na[p] = (m, v)
        ns_ = {}
        for s in STATS:
            ns_[s] = np.zeros(n, np.float32) if reset_stats else _f(state[s])[src]
        ns_["tmp_radii"] = np.asarray(state["tmp_radii"], np.int32)[src]
        return nm, na, ns_

    def final_prune(self, model, adam, state, min_opacity, pruning, score_thresh, min_gaussians):
        P = len(model["means3d"])
        prune = np.zeros(P, np.uint32)
        prio = np.zeros(P, np.float32)
        self.lib.orc_final_prune_mask(P, min_opacity, score_thresh,
                                      _ptr(_f(model["opacity_logits"]).reshape(-1)),
                                      _ptr(_f(pruning)), _ptr(prune), _ptr(prio))
        requested = int(prune.sum())
        min_keep = min(max(int(min_gaussians), 0), P)
        if P - requested < min_keep:
            order = np.lexsort((np.arange(P), -prio))  # descending priority, ties by row
            keep = np.zeros(P, bool)
            keep[order[:min_keep]] = True
        else:
            keep = prune == 0
        rows = np.flatnonzero(keep)
        zeros = np.zeros(len(rows), np.int32)
        new = self._gather(model, adam, state, rows, zeros, zeros - 1, 1, None, False, 0.0)
        return new + ({"requested_remove": requested, "kept": len(rows)},)

    def opacity_cap(self, logits, cap):
        x = _f(logits).reshape(-1).copy()
        self.lib.orc_opacity_cap(len(x), cap, _ptr(x))
        return x

    # ---------------------------------------------------------------- scores
    def metric_map(self, pred, target, loss_thresh):
        pred = _f(pred)
        target = _f(target)
        C, HW = pred.shape
        mm = np.zeros(HW, np.int32)
        loss = np.zeros(1, np.float32)
        self.lib.orc_metric_l1(C, HW, _ptr(pred), _ptr(target), loss_thresh, _ptr(mm), _ptr(loss))
        return mm, float(loss[0])

    def score_accumulate(self, counts, score, metric_count, loss):
        counts = _f(counts).copy()
        score = _f(score).copy()
        mc = np.ascontiguousarray(metric_count, np.int32)
        self.lib.orc_score_accumulate(len(counts), _ptr(mc), loss, _ptr(counts), _ptr(score))
        return counts, score

    def score_finalize(self, counts, score, n_cams):
        P = len(counts)
        imp = np.zeros(P, np.float32)
        prn = np.zeros(P, np.float32)
        self.lib.orc_score_finalize(P, n_cams, _ptr(_f(counts)), _ptr(_f(score)), _ptr(imp),
                                    _ptr(prn))
        return imp, prn
