"""Pins the densification oracle (oracle/fgs_densify_oracle.c, oracle/densify.py)
against closed forms, brute force and the reference's own numpy flow
(scripts/train_scanner_fastgs.py:391-405, 470-793)."""
import itertools
import math
from types import SimpleNamespace

import numpy as np
import pytest

from fastgs_core_amd.densify import DensifyConfig


@pytest.fixture(scope="module")
def dor():
    from oracle.densify import DensifyOracle

    return DensifyOracle()


def _model(rng, P, M=3):
    q = rng.normal(0, 1, (P, 4)).astype(np.float32)
    return {
        "means3d": rng.normal(0, 1, (P, 3)).astype(np.float32),
        "features_dc": rng.uniform(0, 1, (P, 3)).astype(np.float32),
        "features_rest": rng.normal(0, 0.05, (P, M, 3)).astype(np.float32),
        "opacity_logits": rng.normal(-1, 2.5, (P, 1)).astype(np.float32),
        "log_scales": rng.normal(-3.5, 1.0, (P, 3)).astype(np.float32),
        "rotations": q,
    }


def _adam(rng, model):
    return {k: (rng.normal(0, 1, v.shape).astype(np.float32),
                rng.uniform(0, 1, v.shape).astype(np.float32)) for k, v in model.items()}


def _state(rng, P):
    return {"max_radii2d": rng.uniform(0, 40, P).astype(np.float32),
            "grad_accum": rng.uniform(0, 4e-3, P).astype(np.float32),
            "grad_accum_abs": rng.uniform(0, 2e-2, P).astype(np.float32),
            "denom": rng.integers(0, 8, P).astype(np.float32),
            "tmp_radii": rng.integers(0, 30, P).astype(np.int32)}


def test_stats_closed_form(dor):
    radii = np.array([0, 3, 7, -1], np.int32)
    g = np.array([[9, 9, 9, 9], [3, 4, 6, 8], [0.5, 0, 0, 0.25], [1, 1, 1, 1]], np.float32)
    st = {"max_radii2d": np.array([5, 1, 9, 2], np.float32),
          "grad_accum": np.array([1, 1, 1, 1], np.float32),
          "grad_accum_abs": np.zeros(4, np.float32), "denom": np.array([2, 2, 2, 2], np.float32)}
    st = dor.update_stats(st, radii, g)
    np.testing.assert_array_equal(st["max_radii2d"], [5, 3, 9, 2])
    np.testing.assert_array_equal(st["grad_accum"], np.float32([1, 1 + 5, 1 + 0.5, 1]))
    np.testing.assert_array_equal(st["grad_accum_abs"], np.float32([0, 10, 0.25, 0]))
    np.testing.assert_array_equal(st["denom"], [2, 3, 3, 2])
    np.testing.assert_array_equal(st["tmp_radii"], radii)


def test_classify_thresholds(dor):
    cfg = DensifyConfig()
    ext = 2.0  # clone if max scale <= 0.02
    ls = np.log(np.array([[0.01, 0.015, 0.005], [0.05, 0.01, 0.01],
                          [0.01, 0.01, 0.01], [0.1, 0.1, 0.1], [0.019, 0.01, 0.01]], np.float64))
    st = {"grad_accum": np.float32([4e-4, 0, 2e-4, 0, 1e-4]),
          "grad_accum_abs": np.float32([0, 5e-3, 0, 1e-3, 0]),
          "denom": np.float32([1, 2, 0.5, 0, 1])}
    imp = np.float32([6, 6, 6, 6, 5])
    clone, split = dor.classify(cfg, ext, st, ls.astype(np.float32), imp)
    # row 0: small, grad 4e-4 >= 2e-4 -> clone; row 1: large, abs 2.5e-3 >= 1.2e-3 -> split;
    # row 2: denom clamps to 1, grad 2e-4 -> clone; row 3: abs 1e-3 < 1.2e-3 -> none;
    # row 4: importance 5 is not > 5 -> none
    np.testing.assert_array_equal(clone, [1, 0, 1, 0, 0])
    np.testing.assert_array_equal(split, [0, 1, 0, 0, 0])


def _rotmat64(q):
    q = np.asarray(q, np.float64)
    q = q / max(np.linalg.norm(q), 1e-8)
    w, x, y, z = q
    return np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - z * w), 2 * (x * z + y * w)],
                     [2 * (x * y + z * w), 1 - 2 * (x * x + z * z), 2 * (y * z - x * w)],
                     [2 * (x * z - y * w), 2 * (y * z + x * w), 1 - 2 * (x * x + y * y)]])


def test_split_children_and_cap_closed_form(dor):
    rng = np.random.default_rng(1)
    P = 40
    model = _model(rng, P)
    src = np.arange(P, dtype=np.int32)
    kind = np.full(P, 2, np.int32)
    child = np.arange(P, dtype=np.int32)
    normals = rng.normal(0, 1, (P, 3)).astype(np.float32)
    adam = _adam(rng, model)
    st = _state(rng, P)
    nm, na, ns = dor._gather(model, adam, st, src, kind, child, 2, normals, True, 0.82)
    for i in range(P):
        s = np.exp(model["log_scales"][i].astype(np.float64))
        want = model["means3d"][i] + _rotmat64(model["rotations"][i]) @ (s * normals[i])
        np.testing.assert_allclose(nm["means3d"][i], want, rtol=2e-6, atol=2e-6)
        np.testing.assert_allclose(nm["log_scales"][i], np.log(s / 1.6), rtol=1e-6, atol=1e-6)
        o = 1 / (1 + np.exp(-np.float64(model["opacity_logits"][i, 0])))
        p = min(max(min(o, np.float64(np.float32(0.82))), 1e-6), 1 - 1e-6)
        np.testing.assert_allclose(nm["opacity_logits"][i, 0], np.log(p / (1 - p)), rtol=2e-5,
                                   atol=2e-5)
    for k in ("means3d", "features_dc", "features_rest", "log_scales", "rotations"):
        assert not na[k][0].any() and not na[k][1].any()  # appended rows: zero moments
    assert not ns["grad_accum"].any()


def _successive_inclusion(w, k):
    """Exact inclusion probabilities of sampling k of len(w) without
    replacement, each draw proportional to the remaining weights."""
    n = len(w)
    inc = np.zeros(n)
    for perm in itertools.permutations(range(n), k):
        p, rem = 1.0, float(sum(w))
        for i in perm:
            p *= w[i] / rem
            rem -= w[i]
        for i in perm:
            inc[i] += p
    return inc


def test_removal_keys_sample_like_successive_weighted_choice(dor):
    """The k smallest keys select like rng.choice(size=k, replace=False, p=w/sum w)."""
    cfg = DensifyConfig(min_opacity=1.1, max_screen_size=0.0, max_world_scale_factor=0.0)
    score = np.float32([0.0, 0.5, 0.9, 0.99, 0.3])
    w = 1.0 / (1e-6 + (1.0 - score.astype(np.float64)))
    n, k, trials = len(score), 2, 20000
    P2 = n
    src = np.arange(n, dtype=np.int32)
    kind = np.zeros(n, np.int32)
    rng = np.random.default_rng(7)
    hits = np.zeros(n)
    from oracle.densify import _f, _ptr

    prm = np.array([cfg.min_opacity, 0, 0, 2], np.float32)
    logits = np.zeros(n, np.float32)
    ls = np.full((n, 3), -3, np.float32)
    mr = np.zeros(n, np.float32)
    for _ in range(trials):
        u = rng.random(n).astype(np.float32)
        keys = np.zeros(P2, np.uint64)
        cand = np.zeros(P2, np.uint32)
        dor.lib.orc_densify_keys(P2, _ptr(prm), 0, _ptr(src), _ptr(kind), _ptr(logits), _ptr(ls),
                                 _ptr(mr), _ptr(_f(score)), _ptr(u), _ptr(keys), _ptr(cand))
        assert cand.all()
        hits[np.argsort(keys, kind="stable")[:k]] += 1
    np.testing.assert_allclose(hits / trials, _successive_inclusion(w, k), atol=0.015)


def _reference_flow(cfg, ext, model, state, importance, normals):
    """The reference's clone -> split -> drop-sources flow (:514-587) in plain
    numpy float64, masks padded for the appended rows."""
    P0 = len(model["means3d"])
    d = np.maximum(state["denom"].astype(np.float64), 1.0)
    gv = state["grad_accum"] / d
    ga = state["grad_accum_abs"] / d
    ms = np.exp(model["log_scales"].astype(np.float64)).max(axis=1)
    metric = importance > cfg.importance_score_threshold
    cl = metric & (ms <= cfg.dense * ext) & (np.abs(gv) >= cfg.grad_thresh)
    sp = metric & (ms > cfg.dense * ext) & (np.abs(ga) >= cfg.grad_abs_thresh)
    means = np.concatenate([model["means3d"], model["means3d"][cl]])
    sel = np.concatenate([sp, np.zeros(cl.sum(), bool)])
    f = cfg.split_factor
    rs = np.repeat(np.exp(model["log_scales"][sp].astype(np.float64)), f, axis=0)
    rm = np.repeat([_rotmat64(q) for q in model["rotations"][sp]], f, axis=0) \
        if sp.any() else np.zeros((0, 3, 3))
    off = np.einsum("nij,nj->ni", rm, rs * normals)
    means = np.concatenate([means, np.repeat(model["means3d"][sp], f, axis=0) + off])
    keep = ~np.concatenate([sel, np.zeros(sp.sum() * f, bool)])
    return means[keep], int(cl.sum()), int(sp.sum())


def test_densify_layout_matches_reference_flow(dor):
    rng = np.random.default_rng(3)
    P = 300
    model = _model(rng, P)
    adam = _adam(rng, model)
    st = _state(rng, P)
    imp = rng.integers(0, 12, P).astype(np.float32)
    cfg = DensifyConfig(min_opacity=0.0, max_screen_size=0.0, max_world_scale_factor=0.0)
    ext = 3.0
    # draw the normals once the split count is known
    cf, sf = dor.classify(cfg, ext, st, model["log_scales"], imp)
    n_split = int(sf.sum())
    normals = rng.normal(0, 1, (n_split * cfg.split_factor, 3)).astype(np.float32)
    nm, na, ns, info = dor.densify_and_prune(cfg, ext, model, adam, st, imp, None, normals, None)
    want_means, nc, nsp = _reference_flow(cfg, ext, model, st, imp, normals)
    assert info["cloned"] == nc and info["split_sources"] == nsp and nc > 0 and nsp > 0
    np.testing.assert_allclose(nm["means3d"], want_means, rtol=2e-6, atol=2e-6)
    assert len(nm["features_rest"]) == P - nsp + nc + 2 * nsp


def test_metric_map_brute_force(dor):
    rng = np.random.default_rng(5)
    C, HW = 3, 4000
    pred = rng.uniform(0, 1, (C, HW)).astype(np.float32)
    tgt = rng.uniform(0, 1, (C, HW)).astype(np.float32)
    mm, loss = dor.metric_map(pred, tgt, 0.06)
    l = np.abs(pred.astype(np.float64) - tgt).mean(axis=0)
    nrm = (l - l.min()) / max(l.max() - l.min(), 1e-6)
    far = np.abs(nrm - 0.06) > 1e-5
    np.testing.assert_array_equal(mm[far], (nrm > 0.06)[far])
    assert abs(loss - np.abs(pred.astype(np.float64) - tgt).mean()) < 1e-6


def test_scores_closed_form(dor):
    counts = np.zeros(4, np.float32)
    score = np.zeros(4, np.float32)
    counts, score = dor.score_accumulate(counts, score, [0, 2, 4, 6], 0.5)
    counts, score = dor.score_accumulate(counts, score, [1, 0, 2, 2], 0.25)
    imp, prn = dor.score_finalize(counts, score, 2)
    np.testing.assert_array_equal(counts, [1, 2, 6, 8])
    np.testing.assert_array_equal(imp, [0, 1, 3, 4])  # floor(counts / 2)
    s = np.array([0.25, 1.0, 2.5, 3.5])
    np.testing.assert_allclose(prn, (s - s.min()) / (s.max() - s.min()), rtol=1e-7)


def test_final_prune_min_keep_branch(dor):
    rng = np.random.default_rng(9)
    P = 50
    model = _model(rng, P)
    adam = _adam(rng, model)
    st = _state(rng, P)
    prn = rng.uniform(0, 1, P).astype(np.float32)
    nm, na, ns, info = dor.final_prune(model, adam, st, 0.99, prn, 0.0, 10)
    # every row qualifies for pruning; the 10 of highest opacity - score stay
    o = 1 / (1 + np.exp(-model["opacity_logits"][:, 0].astype(np.float64)))
    top = np.sort(np.argsort(-(o - prn), kind="stable")[:10])
    assert info["kept"] == 10
    np.testing.assert_array_equal(nm["features_dc"], model["features_dc"][top])
    np.testing.assert_array_equal(na["means3d"][0], adam["means3d"][0][top])
    nm2, _, _, info2 = dor.final_prune(model, adam, st, 0.0, prn, 0.5, 10)
    np.testing.assert_array_equal(nm2["rotations"], model["rotations"][prn <= 0.5])
