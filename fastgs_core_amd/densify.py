"""FastGS densification and pruning on the GPU (HIP kernels of csrc/fgs_densify.hip).

The reference trains with ``scripts/train_scanner_fastgs.py``: the Gaussians
and their Adam moments live in MLX arrays, and every densification interval
the host copies them to numpy, clones / splits / prunes, and rebuilds every
array (``append_new_points`` / ``prune_points``, :470-511).  Here the rows
stay on the device:

* ``GaussianTrainState`` keeps the six parameter tensors, their Adam moments
  and the densification statistics in capacity-sized buffers (two sets).  A
  densify or prune step computes the new row map on the GPU and writes the new
  set into the other buffers in one gather pass; capacity grows by 1.5x only
  when the new count exceeds it, so the number of reallocations is
  logarithmic in the growth.
* ``GaussianTrainState.step`` is the FastGS optimizer policy (the cadence of
  :159-171, MLX Adam without bias correction) on the fused Adam kernel.
* The densification operations mirror ``ScannerGaussianOps`` (:383-467):
  ``update_densification_stats``, ``compute_gaussian_scores_fastgs``,
  ``densify_and_prune_fastgs``, ``final_prune_fastgs``,
  ``reset_opacity_logits`` / ``cap_opacity_logits``.

Defined where the reference is inconsistent (it indexes arrays of the
pre-clone size with masks of the grown size): split sources are chosen among
the rows that existed before cloning, the rows appended in a step inherit
their source's pruning score, and ``tmp_radii`` follows its row.  Random
numbers are tensors drawn on the device with a ``torch.Generator``: split
offsets are standard normals scaled by the source's scales (as
``rng.normal(0, scales)``), and the budgeted pruning draw is the
Efraimidis-Spirakis form of ``rng.choice(p=...)`` without replacement (same
distribution, a different random stream).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Sequence

import torch

from . import _lib
from .rasterizer import _p, _stream, check_wait
from .train import FastGSOptimizerPolicy, expon_lr_func

PARAM_NAMES = ("means3d", "features_dc", "features_rest", "opacity_logits", "log_scales",
               "rotations")
STAT_NAMES = ("max_radii2d", "grad_accum", "grad_accum_abs", "denom")


@dataclass
class DensifyConfig:
    """Densification arguments and defaults of train_scanner_fastgs.py:827-850."""
    grad_thresh: float = 2.0e-4
    grad_abs_thresh: float = 1.2e-3
    dense: float = 0.01
    loss_thresh: float = 0.06
    importance_score_threshold: float = 5.0
    densify_camera_sample: int = 10
    split_factor: int = 2
    min_opacity: float = 0.005
    max_screen_size: float = 20.0
    max_world_scale_factor: float = 0.1
    prune_budget_factor: float = 0.5
    opacity_cap_after_densify: float = 0.82
    opacity_reset_value: float = 0.82
    final_prune_min_opacity: float = 0.1
    final_prune_score_thresh: float = 0.9
    final_prune_min_gaussians: int = 64


@dataclass
class OptimConfig:
    """Learning rates of train_scanner_fastgs.py:813-820 (MLX Adam, betas 0.9 / 0.99)."""
    means_lr: float = 3e-3
    dc_lr: float = 1e-3
    sh_lr: float = 1e-3
    opacity_lr: float = 1e-3
    scaling_lr: float = 1e-3
    rotation_lr: float = 1e-3
    sh_lr_divisor: float = 20.0
    betas: tuple = (0.9, 0.99)
    eps: float = 1e-8
    position_lr_init: Optional[float] = None
    position_lr_final: float = 1.6e-6
    position_lr_delay_mult: float = 0.01
    position_lr_max_steps: int = 30000
    spatial_lr_scale: float = 1.0


def compute_scene_extent(points: torch.Tensor) -> float:
    """train_scanner_fastgs.py:206-209: diagonal of the bounding box."""
    lo = points.min(dim=0).values
    hi = points.max(dim=0).values
    return max(float(torch.linalg.norm((hi - lo).double())), 1.0e-6)


def _check(rc):
    _lib.check(rc)


def _u32(n, dev):
    return torch.empty(max(int(n), 0), dtype=torch.int32, device=dev)


class _Scanner:
    """Inclusive u32 scans and last-element reads on one device.  Each scan's
    output is the head of an (n + 1)-word buffer whose last word receives the
    scan's wait status, read back together with the total by ``last``."""

    def __init__(self, dev):
        self.dev = dev
        self.lib = _lib.load()

    def incl(self, flags: torch.Tensor) -> torch.Tensor:
        n = flags.numel()
        buf = torch.empty(n + 1, dtype=torch.int32, device=self.dev)
        ws = torch.empty(int(self.lib.fgs_scan_workspace_bytes(max(n, 1))), dtype=torch.uint8,
                         device=self.dev)
        _check(self.lib.fgs_inclusive_scan_u32(_p(flags), _p(buf[:n]) if n else None, n, _p(ws),
                                               _p(buf[n:]), _stream(self.dev)))
        return buf[:n]

    @staticmethod
    def last(t: torch.Tensor) -> int:
        """The total (last element) of an ``incl`` result, after checking the
        scan's wait status stored in the word that follows it."""
        n = t.numel()
        pair = torch.as_strided(t, (2,), (1,), t.storage_offset() + n - 1) if n else \
            torch.as_strided(t, (1,), (1,), t.storage_offset())
        a = pair.cpu().numpy()
        check_wait(int(a[-1]) & 0xFFFFFFFF, "densification scan")
        return int(a[0]) & 0xFFFFFFFF if n else 0


def _sort_rows_by_key(lib, keys, P, dev, st):
    """Rows in ascending order of their 32-bit keys (stable), through
    fgs_sort_pairs_u64, with its wait status checked."""
    skeys = torch.empty(P, dtype=torch.int64, device=dev)
    srows = _u32(P, dev)
    ws = torch.empty(int(lib.fgs_sort_workspace_bytes(P)), dtype=torch.uint8, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    _check(lib.fgs_sort_pairs_u64(_p(keys), None, _p(skeys), _p(srows), P, 0, 32, _p(ws),
                                  _p(status), st))
    check_wait(int(status.item()) & 0xFFFFFFFF, "densification sort")
    return srows


class GaussianTrainState:
    """Device-resident Gaussians (reference parameter names and shapes), their
    Adam moments and the FastGS densification statistics.

    ``params`` holds ``means3d [P,3]``, ``features_dc [P,3]``, ``features_rest
    [P,M,3]``, ``opacity_logits [P,1]``, ``log_scales [P,3]``, ``rotations
    [P,4]`` (w,x,y,z).  ``param(name)`` returns the leaf tensor of the current
    rows (``requires_grad``); it is replaced after a densify/prune step.
    """

    def __init__(self, params: Dict[str, torch.Tensor], optim: Optional[OptimConfig] = None,
                 capacity: Optional[int] = None):
        if not torch.cuda.is_available():
            raise RuntimeError("fastgs_core_amd requires a ROCm GPU; there is no CPU fallback")
        self.lib = _lib.load()
        self.dev = params["means3d"].device
        if self.dev.type != "cuda":
            raise RuntimeError("GaussianTrainState needs GPU tensors (no CPU fallback)")
        self.P = int(params["means3d"].shape[0])
        rest = params["features_rest"]
        self.M = int(rest.shape[1]) if rest.dim() == 3 else 0
        self.widths = {"means3d": 3, "features_dc": 3, "features_rest": 3 * self.M,
                       "opacity_logits": 1, "log_scales": 3, "rotations": 4}
        self.optim = optim or OptimConfig()
        cap = max(int(capacity or 0), self.P, 1)
        self._bufs = [self._alloc(cap), None]
        self._cur = 0
        b = self._bufs[0]
        for n in PARAM_NAMES:
            b[n][: self.P * self.widths[n]].copy_(
                params[n].detach().to(self.dev, torch.float32).reshape(-1))
            for k in ("m", "v"):
                b[k + n].zero_()
        for n in STAT_NAMES:
            b[n].zero_()
        b["tmp_radii"].zero_()
        self.step_count = {n: 0 for n in PARAM_NAMES}
        lr_init = self.optim.position_lr_init if self.optim.position_lr_init is not None \
            else self.optim.means_lr
        self.xyz_scheduler = expon_lr_func(
            lr_init * self.optim.spatial_lr_scale,
            self.optim.position_lr_final * self.optim.spatial_lr_scale,
            lr_delay_mult=self.optim.position_lr_delay_mult,
            max_steps=self.optim.position_lr_max_steps)
        self.lrs = {"means3d": self.optim.means_lr, "features_dc": self.optim.dc_lr,
                    "features_rest": self.optim.sh_lr / self.optim.sh_lr_divisor,
                    "opacity_logits": self.optim.opacity_lr, "log_scales": self.optim.scaling_lr,
                    "rotations": self.optim.rotation_lr}
        self.reallocations = 0
        self._make_leaves()

    # ------------------------------------------------------------------ storage
    def _alloc(self, cap: int) -> Dict[str, torch.Tensor]:
        f32 = dict(dtype=torch.float32, device=self.dev)
        b = {"capacity": cap}
        for n in PARAM_NAMES:
            w = self.widths[n]
            b[n] = torch.empty(cap * w, **f32)
            b["m" + n] = torch.empty(cap * w, **f32)
            b["v" + n] = torch.empty(cap * w, **f32)
        for n in STAT_NAMES:
            b[n] = torch.empty(cap, **f32)
        b["tmp_radii"] = torch.empty(cap, dtype=torch.int32, device=self.dev)
        return b

    def _shape(self, name: str, P: int):
        return {"means3d": (P, 3), "features_dc": (P, 3), "features_rest": (P, self.M, 3),
                "opacity_logits": (P, 1), "log_scales": (P, 3), "rotations": (P, 4)}[name]

    def _make_leaves(self):
        b = self._bufs[self._cur]
        self._leaves = {}
        for n in PARAM_NAMES:
            v = b[n][: self.P * self.widths[n]].view(self._shape(n, self.P))
            self._leaves[n] = v.detach().requires_grad_(True)

    def param(self, name: str) -> torch.Tensor:
        return self._leaves[name]

    def moments(self, name: str):
        b = self._bufs[self._cur]
        w = self.widths[name] * self.P
        return b["m" + name][:w], b["v" + name][:w]

    def stat(self, name: str) -> torch.Tensor:
        return self._bufs[self._cur][name][: self.P]

    def tmp_radii(self) -> torch.Tensor:
        return self._bufs[self._cur]["tmp_radii"][: self.P]

    @property
    def capacity(self) -> int:
        return self._bufs[self._cur]["capacity"]

    def _target(self, P_new: int) -> Dict[str, torch.Tensor]:
        o = 1 - self._cur
        if self._bufs[o] is None or self._bufs[o]["capacity"] < P_new:
            self._bufs[o] = None
            self._bufs[o] = self._alloc(max(P_new, int(1.5 * max(P_new, self.capacity)), 1))
            self.reallocations += 1
        return self._bufs[o]

    # -------------------------------------------------------------- optimizer
    def update_learning_rate(self, iteration: int) -> float:
        lr = self.xyz_scheduler(iteration)
        self.lrs["means3d"] = lr
        return lr

    @torch.no_grad()
    def step(self, iteration: int) -> None:
        """Adam on the parameters whose cadence fires (FastGSOptimizerPolicy)."""
        main = FastGSOptimizerPolicy.should_step_main(iteration)
        sh = FastGSOptimizerPolicy.should_step_sh(iteration)
        b1, b2 = self.optim.betas
        groups, keep = [], []
        for n in PARAM_NAMES:
            if (n == "features_rest" and not sh) or (n != "features_rest" and not main):
                continue
            leaf = self._leaves[n]
            if leaf.grad is None or leaf.numel() == 0:
                continue
            g = leaf.grad.to(torch.float32).contiguous()
            keep.append(g)
            m, v = self.moments(n)
            self.step_count[n] += 1
            groups.append(_lib.AdamGroup(_p(leaf), _p(g), _p(m), _p(v), leaf.numel(),
                                         float(self.lrs[n]), self.step_count[n]))
        if groups:  # the six tensors in one launch
            arr = (_lib.AdamGroup * len(groups))(*groups)
            _check(self.lib.fgs_adam_step_multi(arr, len(groups), float(b1), float(b2),
                                                float(self.optim.eps), 0, _stream(self.dev)))

    def zero_grad(self) -> None:
        for t in self._leaves.values():
            t.grad = None

    # ------------------------------------------------------------ densification
    @torch.no_grad()
    def update_densification_stats(self, radii: torch.Tensor, d_viewspace: torch.Tensor) -> None:
        """update_densification_stats (:391-405) from one step's radii and
        viewspace gradient."""
        b = self._bufs[self._cur]
        r = radii.to(self.dev, torch.int32).contiguous()
        g = d_viewspace.to(self.dev, torch.float32).contiguous()
        if r.numel() != self.P or g.shape != (self.P, 4):
            raise ValueError(f"update_densification_stats: radii [{self.P}] and d_viewspace "
                             f"[{self.P},4] expected")
        _check(self.lib.fgs_densify_stats(self.P, _p(r), _p(g), _p(b["max_radii2d"]),
                                          _p(b["grad_accum"]), _p(b["grad_accum_abs"]),
                                          _p(b["denom"]), _p(b["tmp_radii"]), _stream(self.dev)))

    def reset_densification_buffers(self) -> None:
        for n in STAT_NAMES:
            self._bufs[self._cur][n][: self.P].zero_()

    @torch.no_grad()
    def cap_opacity_logits(self, cap: float) -> None:
        """cap_opacity_logits / reset_opacity_logits (:619-658): opacity
        logits to logit(min(sigmoid(x), cap)); their Adam moments restart."""
        m, v = self.moments("opacity_logits")
        _check(self.lib.fgs_opacity_cap(self.P, float(cap), _p(self._leaves["opacity_logits"]),
                                        _p(m), _p(v), _stream(self.dev)))

    reset_opacity_logits = cap_opacity_logits

    def _build(self, P_new: int, rows, l2_src, l2_kind, l2_child, normals, reset_stats: bool,
               opacity_cap: float) -> None:
        src = self._bufs[self._cur]
        dst = self._target(P_new)
        io = _lib.DensifyBuildIO()
        io.P_new = P_new
        io.sh_row = 3 * self.M
        io.split_factor = 1 if l2_src is None else self._split_factor
        io.reset_stats = int(bool(reset_stats))
        io.opacity_cap = float(opacity_cap)
        io.rows, io.l2_src, io.l2_kind, io.l2_child, io.normals = (
            _p(rows), _p(l2_src), _p(l2_kind), _p(l2_child), _p(normals))
        for n in PARAM_NAMES:
            setattr(io, n, _p(src[n]) if self.widths[n] else None)
            setattr(io, "d_" + n, _p(dst[n]) if self.widths[n] else None)
        for k, n in enumerate(PARAM_NAMES):
            if self.widths[n]:
                io.exp_avg[k], io.exp_avg_sq[k] = _p(src["m" + n]), _p(src["v" + n])
                io.d_exp_avg[k], io.d_exp_avg_sq[k] = _p(dst["m" + n]), _p(dst["v" + n])
        for n in STAT_NAMES:
            setattr(io, n, _p(src[n]))
            setattr(io, "d_" + n, _p(dst[n]))
        io.tmp_radii, io.d_tmp_radii = _p(src["tmp_radii"]), _p(dst["tmp_radii"])
        if P_new > 0:
            _check(self.lib.fgs_densify_build(ctypes.byref(io), _stream(self.dev)))
        self._cur = 1 - self._cur
        self.P = P_new
        self._make_leaves()

    @torch.no_grad()
    def densify_and_prune_fastgs(self, cfg: DensifyConfig, scene_extent: float,
                                 importance_score: torch.Tensor, pruning_score: torch.Tensor,
                                 generator: Optional[torch.Generator] = None,
                                 normals: Optional[torch.Tensor] = None,
                                 uniforms: Optional[torch.Tensor] = None) -> Dict[str, int]:
        """densify_and_prune_fastgs (:661-742): clone and split the rows the
        metric and gradient tests select, prune by opacity / screen size /
        world scale within the budget, cap the opacities.  ``normals`` /
        ``uniforms`` override the draws (tests)."""
        lib, dev, st = self.lib, self.dev, _stream(self.dev)
        P0 = self.P
        f = int(cfg.split_factor)
        if f < 1:
            raise ValueError("split_factor must be >= 1")
        self._split_factor = f
        prm = _lib.DensifyParams(
            float(cfg.grad_thresh), float(cfg.grad_abs_thresh),
            float(cfg.dense * scene_extent), float(cfg.importance_score_threshold),
            float(cfg.min_opacity), float(cfg.max_screen_size),
            float(cfg.max_world_scale_factor * scene_extent) if cfg.max_world_scale_factor > 0 else 0.0,
            f)
        b = self._bufs[self._cur]
        imp = importance_score.to(dev, torch.float32).contiguous()
        prn = pruning_score.to(dev, torch.float32).contiguous() if pruning_score is not None else None
        if imp.numel() != P0 or (prn is not None and prn.numel() not in (0, P0)):
            raise ValueError("importance_score / pruning_score must have one entry per Gaussian")
        sc = _Scanner(dev)
        cflag, sflag = _u32(P0, dev), _u32(P0, dev)
        if P0:
            _check(lib.fgs_densify_classify(P0, ctypes.byref(prm), _p(b["grad_accum"]),
                                            _p(b["grad_accum_abs"]), _p(b["denom"]),
                                            _p(b["log_scales"]), _p(imp), _p(cflag), _p(sflag), st))
        metric_hits = int((imp > cfg.importance_score_threshold).sum())
        cincl, sincl = sc.incl(cflag), sc.incl(sflag)
        nc, ns = sc.last(cincl), sc.last(sincl)
        P2 = P0 - ns + nc + ns * f
        l2_src, l2_kind, l2_child = _u32(P2, dev), _u32(P2, dev), _u32(P2, dev)
        if P0:
            _check(lib.fgs_densify_layout(P0, f, _p(cincl), _p(sincl), _p(l2_src), _p(l2_kind),
                                          _p(l2_child), st))
        if normals is None:
            normals = torch.randn((ns * f, 3), generator=generator, device=dev)
        normals = normals.to(dev, torch.float32).contiguous()
        if normals.shape != (ns * f, 3):
            raise ValueError(f"normals must be [{ns * f}, 3]")
        appended = (nc + ns) > 0
        if uniforms is None:
            uniforms = torch.rand((P2,), generator=generator, device=dev)
        uniforms = uniforms.to(dev, torch.float32).contiguous()
        keys = torch.empty(P2, dtype=torch.int64, device=dev)
        cand = _u32(P2, dev)
        use_scores = prn is not None and prn.numel() > 0
        if P2:
            _check(lib.fgs_densify_prune_keys(P2, ctypes.byref(prm), int(appended), _p(l2_src),
                                              _p(l2_kind), _p(b["opacity_logits"]),
                                              _p(b["log_scales"]), _p(b["max_radii2d"]),
                                              _p(prn) if use_scores else None,
                                              _p(uniforms) if use_scores else None, _p(keys),
                                              _p(cand), st))
        to_remove = sc.last(sc.incl(cand))
        budget = int(cfg.prune_budget_factor * to_remove)
        k = min(budget, to_remove) if use_scores else 0
        rows = None
        P_new = P2
        if k > 0:
            srows = _sort_rows_by_key(lib, keys, P2, dev, st)
            keep = _u32(P2, dev)
            _check(lib.fgs_densify_select(P2, k, _p(srows), _p(keep), st))
            kincl = sc.incl(keep)
            P_new = P2 - k
            rows = _u32(P_new, dev)
            _check(lib.fgs_densify_compact(P2, _p(keep), _p(kincl), _p(rows), st))
        if normals.numel() == 0:  # no split child reads it; the build wants a pointer
            normals = torch.zeros((1, 3), dtype=torch.float32, device=dev)
        self._build(P_new, rows, l2_src, l2_kind, l2_child, normals, appended,
                    float(cfg.opacity_cap_after_densify))
        return {"metric_hits": metric_hits, "cloned": nc, "split_sources": ns,
                "split_children": ns * f, "total_prune_candidates": to_remove,
                "prune_budget": budget, "actual_removed": k, "points": P_new}

    @torch.no_grad()
    def final_prune_fastgs(self, min_opacity: float, pruning_score: torch.Tensor,
                           score_thresh: float, min_gaussians: int) -> Dict[str, int]:
        """final_prune_fastgs (:745-793)."""
        lib, dev, st = self.lib, self.dev, _stream(self.dev)
        P = self.P
        if P == 0:
            return {"total": 0, "requested_remove": 0, "actual_remove": 0, "kept": 0}
        prn = pruning_score.to(dev, torch.float32).contiguous()
        prune = _u32(P, dev)
        keys = torch.empty(P, dtype=torch.int64, device=dev)
        _check(lib.fgs_final_prune_mask(P, float(min_opacity), float(score_thresh),
                                        _p(self._leaves["opacity_logits"]), _p(prn), _p(prune),
                                        _p(keys), st))
        sc = _Scanner(dev)
        requested = sc.last(sc.incl(prune))
        min_keep = min(max(int(min_gaussians), 0), P)
        keep = _u32(P, dev)
        if P - requested < min_keep:
            srows = _sort_rows_by_key(lib, keys, P, dev, st)
            _check(lib.fgs_densify_keep_first(P, min_keep, _p(srows), _p(keep), st))
        else:
            _check(lib.fgs_invert_flags(P, _p(prune), _p(keep), st))
        kincl = sc.incl(keep)
        P_new = sc.last(kincl)
        rows = _u32(P_new, dev)
        _check(lib.fgs_densify_compact(P, _p(keep), _p(kincl), _p(rows), st))
        self._split_factor = 1
        self._build(P_new, rows, None, None, None, None, False, 0.0)
        return {"total": P, "requested_remove": requested, "actual_remove": P - P_new,
                "kept": P_new}

    # ------------------------------------------------------------------ scores
    @torch.no_grad()
    def compute_gaussian_scores_fastgs(self, render: Callable, targets: Sequence[torch.Tensor],
                                       camera_indices: Sequence[int], loss_thresh: float,
                                       densify: bool):
        """compute_gaussian_scores_fastgs (:279-340).  ``render(idx,
        metric_map=None)`` renders camera ``idx`` with this state's rows and
        returns the ``rasterize_gaussians`` output dict (with ``metric_count``
        when a metric map is given); ``targets[idx]`` is ``[C, H*W]``."""
        lib, dev, st = self.lib, self.dev, _stream(self.dev)
        P = self.P
        counts = torch.zeros(P, dtype=torch.float32, device=dev)
        score = torch.zeros(P, dtype=torch.float32, device=dev)
        loss = torch.zeros(1, dtype=torch.float32, device=dev)
        n = 0
        for idx in camera_indices:
            out = render(idx, None)
            pred = out["out_color"].contiguous()
            tgt = targets[idx].to(dev, torch.float32).contiguous()
            C, HW = pred.shape
            ws = torch.empty(int(lib.fgs_metric_map_workspace_bytes(HW)), dtype=torch.uint8,
                             device=dev)
            mm = torch.empty(HW, dtype=torch.int32, device=dev)
            _check(lib.fgs_metric_map(C, HW, _p(pred), _p(tgt), float(loss_thresh), _p(ws),
                                      _p(mm), _p(loss), st))
            second = render(idx, mm)
            mc = second["metric_count"].to(torch.int32).contiguous()
            _check(lib.fgs_score_accumulate(P, _p(mc), _p(loss), _p(counts), _p(score), st))
            n += 1
        importance = torch.zeros(P, dtype=torch.float32, device=dev) if densify else None
        pruning = torch.zeros(P, dtype=torch.float32, device=dev)
        if n and P:
            mm_ws = torch.empty(2, dtype=torch.int32, device=dev)
            _check(lib.fgs_score_finalize(P, n, _p(counts), _p(score), _p(importance),
                                          _p(pruning), _p(mm_ws), st))
        return importance, pruning

    # ----------------------------------------------------------------- render
    @torch.no_grad()
    def preprocess_radii(self, camera_inputs: Dict[str, torch.Tensor], width: int, height: int,
                         tan_fovx: float, tan_fovy: float) -> torch.Tensor:
        """The current rows' radii for one camera from the preprocess alone
        (``preprocess_forward``, binding.cpp:397-508): the radii a full render
        of the same camera returns, without its binning and blend."""
        from .rasterizer import preprocess_forward

        d = self.render_inputs(camera_inputs)
        pf = {"means3d": d["means3d"], "opacities": d["opacities"],
              "viewmat": d["viewmatrix"], "projmat": d["projmatrix"], "cam_pos": d["campos"],
              "viewspace_points": torch.zeros((self.P, 4), dtype=torch.float32, device=self.dev),
              "scales": d["scales"], "quats": d["rotations"], "dc": d["dc"], "sh": d["sh"]}
        return preprocess_forward(pf, width, height, 16, 16, tan_fovx, tan_fovy, 0)["radii"]

    def render_inputs(self, camera_inputs: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
        """The ``rasterize_gaussians`` input dict of the current rows (the
        activations of :523-536 through ``fastgs_core_amd.activate``)."""
        from .train import activate

        s, r, o = activate(self._leaves["log_scales"], self._leaves["rotations"],
                           self._leaves["opacity_logits"])
        d = dict(camera_inputs)
        d.update(means3d=self._leaves["means3d"], dc=self._leaves["features_dc"],
                 sh=self._leaves["features_rest"], opacities=o.view(-1), scales=s, rotations=r)
        return d


# ---------------------------------------------------------------------- loop
@dataclass
class LoopConfig:
    """The schedule of the FastGS training loop (train_scanner_fastgs.py:968-1060,
    defaults of :799-849 except where a workload sets them).

    ``stats_render``: where the densification statistics take their radii.
    "post_step" is the reference's: a second forward render of the same
    camera after the optimizer step (:1014-1019).  "train" takes them from the
    training render itself (one render fewer per iteration; the radii then
    describe the pre-step parameters, so ``max_radii2d`` and the ``radii > 0``
    mask can differ from the reference's on the same draws)."""
    interval: int = 500
    densify_from: int = 500
    densify_until: int = 15000
    mse_until: int = 600
    sh_interval: int = 1000
    opacity_reset_interval: int = 3000
    final_prune_start: int = 15000
    final_prune_end: int = 30000
    final_prune_interval: int = 3000
    stats_render: str = "post_step"


class FastGSTrainLoop:
    """One iteration of the reference loop at a time on a GaussianTrainState.

    ``render(ts, idx, degree, metric_map=None, vsp=None)`` renders camera
    ``idx`` with the state's current rows and returns the
    ``rasterize_gaussians`` dict; ``targets[idx]`` is ``[3, H*W]``.
    ``radii(ts, idx)`` (optional) returns camera ``idx``'s radii for the
    post-step statistics (``GaussianTrainState.preprocess_radii`` gives them
    from the preprocess alone); without it a full render is made.  Cameras
    are popped from a seeded viewpoint stack (:974-978); the loss is MSE up to
    ``mse_until`` and L1 after (:960-963); Adam follows the FastGS cadence.
    The statistics accumulate while ``it < densify_until``; a densification
    event runs at ``it > densify_from`` and ``it % interval == 0`` (:1021):
    metric-map scores over ``densify_camera_sample`` sampled cameras, then
    densify_and_prune_fastgs.  The opacity reset (:1047-1049) and the final
    prune (:1051-1060) follow their intervals."""

    def __init__(self, ts: GaussianTrainState, render: Callable, targets: Sequence[torch.Tensor],
                 n_cameras: int, degree: int, dcfg: DensifyConfig, lcfg: LoopConfig,
                 scene_extent: float, seed: int = 42,
                 generator: Optional[torch.Generator] = None,
                 radii: Optional[Callable] = None):
        import numpy as np

        from .loss import l1_loss, mse_loss

        if lcfg.stats_render not in ("post_step", "train"):
            raise ValueError("stats_render must be 'post_step' or 'train'")
        self.ts, self.render, self.targets = ts, render, targets
        self.radii = radii
        self.n_cameras, self.degree = int(n_cameras), int(degree)
        self.dcfg, self.lcfg, self.extent = dcfg, lcfg, float(scene_extent)
        self.rng = np.random.default_rng(seed)
        self.gen = generator
        self.stack: List[int] = []
        self._losses = (mse_loss, l1_loss)
        self.last_stats = None  # (radii, d_viewspace) of the last statistics update

    def active_degree(self, it: int) -> int:
        return min(it // self.lcfg.sh_interval, self.degree)

    def train_iteration(self, it: int):
        """Forward, loss, backward, Adam step and the statistics of iteration
        ``it`` (1-based).  Returns (loss tensor, camera index)."""
        ts, lc = self.ts, self.lcfg
        ts.update_learning_rate(it)
        active = self.active_degree(it)
        if not self.stack:
            self.stack = list(range(self.n_cameras))
        idx = self.stack.pop(int(self.rng.integers(0, len(self.stack))))
        vsp = torch.zeros((ts.P, 4), device=ts.dev, requires_grad=True)
        out = self.render(ts, idx, active, vsp=vsp)
        img = out["out_color"].reshape(3, -1)
        mse_loss, l1_loss = self._losses
        loss = mse_loss(img, self.targets[idx]) if it <= lc.mse_until else \
            l1_loss(img, self.targets[idx])
        ts.zero_grad()
        loss.backward()
        ts.step(it)
        self.last_stats = None
        if it < lc.densify_until:
            if lc.stats_render == "post_step":
                with torch.no_grad():
                    radii = (self.radii(ts, idx) if self.radii is not None
                             else self.render(ts, idx, active)["radii"])
            else:
                radii = out["radii"]
            ts.update_densification_stats(radii, vsp.grad)
            self.last_stats = (radii, vsp.grad)
        return loss.detach(), idx

    def is_densify_event(self, it: int) -> bool:
        lc = self.lcfg
        return it < lc.densify_until and it > lc.densify_from and it % lc.interval == 0

    def sample_cameras(self) -> List[int]:
        """sample_camera_indices (:262-276)."""
        n = min(self.dcfg.densify_camera_sample, self.n_cameras)
        return [int(i) for i in self.rng.choice(self.n_cameras, size=n, replace=False)]

    def scores(self, it: int, ids: Sequence[int], densify: bool = True, on_render=None):
        """compute_gaussian_scores_fastgs over cameras ``ids`` at the active
        degree.  ``on_render(out)`` sees each render (tests)."""
        active = self.active_degree(it)

        def r(i, mm):
            o = self.render(self.ts, i, active, metric_map=mm)
            if on_render is not None:
                on_render(o)
            return o

        with torch.no_grad():
            return self.ts.compute_gaussian_scores_fastgs(r, self.targets, ids,
                                                          self.dcfg.loss_thresh, densify)

    def densify_event(self, it: int) -> Dict[str, int]:
        """The event of iteration ``it``: scores over the sampled cameras, then
        densify_and_prune_fastgs with draws from the loop's generator."""
        imp, prn = self.scores(it, self.sample_cameras(), True)
        return self.ts.densify_and_prune_fastgs(self.dcfg, self.extent, imp, prn,
                                                generator=self.gen)

    def after_iteration(self, it: int) -> Optional[Dict[str, int]]:
        """The opacity reset and the final prune of iteration ``it`` (run after
        any densification event of the same iteration)."""
        lc = self.lcfg
        if it < lc.densify_until and lc.opacity_reset_interval > 0 and \
                it % lc.opacity_reset_interval == 0:
            self.ts.reset_opacity_logits(self.dcfg.opacity_reset_value)
        if lc.final_prune_interval > 0 and it % lc.final_prune_interval == 0 and \
                lc.final_prune_start < it < lc.final_prune_end:
            _, prn = self.scores(it, self.sample_cameras(), False)
            return self.ts.final_prune_fastgs(self.dcfg.final_prune_min_opacity, prn,
                                              self.dcfg.final_prune_score_thresh,
                                              self.dcfg.final_prune_min_gaussians)
        return None
