"""Training-step glue on either side of the rasterizer, on the GPU.

* ``activate`` -- the parameter activations of the reference training
  scripts (scripts/train_scanner_fixed.py:523-536, train_square.py:181-191):
  ``sigmoid(opacity_logits)``, ``exp(log_scales)``, ``q / (|q| + 1e-8)``,
  forward and backward as one HIP kernel each (csrc/fgs_train.hip).
* ``FusedAdam`` -- in-place Adam with one HIP kernel per parameter tensor;
  ``bias_correction=False`` is MLX's ``mlx.optimizers.Adam`` default, the
  optimizer of scripts/train_scanner_fastgs.py:80-90.
* ``FastGSOptimizerPolicy`` -- the reference's optimizer policy
  (scripts/train_scanner_fastgs.py:77-182): one Adam per main parameter, one
  for the SH rest coefficients with ``sh_lr / sh_lr_divisor``, the stepping
  cadence of ``_should_step_main`` / ``_should_step_sh`` and the exponential
  position learning-rate schedule.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from . import _lib
from .rasterizer import _p, _stream


def _gpu_f32(x: torch.Tensor, name: str) -> torch.Tensor:
    if not torch.is_tensor(x) or not x.is_cuda:
        raise RuntimeError("fastgs_core_amd requires a ROCm GPU; there is no CPU fallback "
                           f"({name} is not a GPU tensor)")
    return x.to(torch.float32).contiguous()


class _Activate(torch.autograd.Function):
    @staticmethod
    def forward(ctx, log_scales, quats, logits):
        lib = _lib.load()
        P = quats.shape[0]
        dev = quats.device
        scales = torch.empty_like(log_scales)
        rots = torch.empty_like(quats)
        opac = torch.empty_like(logits)
        _lib.check(lib.fgs_activations_fwd(P, _p(log_scales), _p(quats), _p(logits), _p(scales),
                                           _p(rots), _p(opac), _stream(dev)))
        ctx.save_for_backward(quats, scales, opac)
        return scales, rots, opac

    @staticmethod
    def backward(ctx, d_scales, d_rots, d_opac):
        lib = _lib.load()
        quats, scales, opac = ctx.saved_tensors
        P = quats.shape[0]
        need = ctx.needs_input_grad
        d_ls = torch.empty_like(scales) if need[0] else None
        d_q = torch.empty_like(quats) if need[1] else None
        d_lg = torch.empty_like(opac) if need[2] else None
        f = lambda t: None if t is None else t.to(torch.float32).contiguous()  # noqa: E731
        _lib.check(lib.fgs_activations_bwd(P, _p(quats), _p(scales), _p(opac), _p(f(d_scales)),
                                           _p(f(d_rots)), _p(f(d_opac)), _p(d_ls), _p(d_q),
                                           _p(d_lg), _stream(quats.device)))
        return d_ls, d_q, d_lg


def activate(log_scales: torch.Tensor, quats: torch.Tensor, opacity_logits: torch.Tensor
             ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(exp(log_scales) [P,3], q/(|q|+1e-8) [P,4], sigmoid(opacity_logits)), differentiable."""
    ls = _gpu_f32(log_scales, "log_scales")
    q = _gpu_f32(quats, "quats")
    lg = _gpu_f32(opacity_logits, "opacity_logits")
    P = q.shape[0]
    if q.dim() != 2 or q.shape[1] != 4 or ls.shape != (P, 3) or lg.numel() != P:
        raise ValueError(f"activate expects log_scales [P,3], quats [P,4], opacity_logits [P] or "
                         f"[P,1]; got {tuple(ls.shape)}, {tuple(q.shape)}, {tuple(lg.shape)}")
    return _Activate.apply(ls, q, lg)


class FusedAdam(torch.optim.Optimizer):
    """Adam with one fused HIP kernel per parameter tensor (csrc/fgs_train.hip).

    ``bias_correction=False`` (default) is MLX's Adam: p -= lr m / (sqrt(v) + eps);
    ``True`` is the bias-corrected form of torch.optim.Adam.
    """

    def __init__(self, params, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, bias_correction: bool = False):
        if lr < 0.0 or not (0.0 <= betas[0] < 1.0) or not (0.0 <= betas[1] < 1.0) or eps < 0.0:
            raise ValueError("FusedAdam: invalid hyper-parameter")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps,
                                      bias_correction=bias_correction))

    @torch.no_grad()
    def step(self, closure=None):
        """One update of every parameter with a gradient: the tensors of a
        parameter group go to the GPU eight per launch (fgs_adam_step_multi)."""
        loss = closure() if closure is not None else None
        lib = _lib.load()
        for group in self.param_groups:
            b1, b2 = group["betas"]
            batch, keep = [], []
            dev = None
            for p in group["params"]:
                if p.grad is None:
                    continue
                if not p.is_cuda or p.dtype != torch.float32 or not p.is_contiguous():
                    raise RuntimeError("FusedAdam needs contiguous float32 GPU parameters")
                if dev is not None and p.device != dev:
                    raise RuntimeError("FusedAdam: the parameters of a group share one device")
                dev = p.device
                st = self.state[p]
                if not st:
                    st["step"] = 0
                    st["exp_avg"] = torch.zeros_like(p)
                    st["exp_avg_sq"] = torch.zeros_like(p)
                st["step"] += 1
                g = p.grad.to(torch.float32).contiguous()
                keep.append(g)
                batch.append(_lib.AdamGroup(_p(p), _p(g), _p(st["exp_avg"]),
                                            _p(st["exp_avg_sq"]), p.numel(), float(group["lr"]),
                                            int(st["step"])))
            for i in range(0, len(batch), 8):
                part = batch[i:i + 8]
                arr = (_lib.AdamGroup * len(part))(*part)
                _lib.check(lib.fgs_adam_step_multi(arr, len(part), float(b1), float(b2),
                                                   float(group["eps"]),
                                                   int(bool(group["bias_correction"])),
                                                   _stream(dev)))
        return loss


def expon_lr_func(lr_init: float, lr_final: float, lr_delay_steps: int = 0,
                  lr_delay_mult: float = 1.0, max_steps: int = 1_000_000):
    """Log-linear learning-rate decay with an optional sine warm-up
    (scripts/train_scanner_fastgs.py:54-74, the 3DGS position schedule)."""

    def lr_at(step: int) -> float:
        if step < 0 or (lr_init == 0.0 and lr_final == 0.0):
            return 0.0
        if lr_delay_steps > 0:
            warm = min(max(step / lr_delay_steps, 0.0), 1.0)
            delay = lr_delay_mult + (1.0 - lr_delay_mult) * math.sin(0.5 * math.pi * warm)
        else:
            delay = 1.0
        t = min(max(step / max_steps, 0.0), 1.0)
        return delay * math.exp(math.log(lr_init) * (1.0 - t) + math.log(lr_final) * t)

    return lr_at


@dataclass
class OptimizerPolicyConfig:
    """scripts/train_scanner_fastgs.py:38-51."""
    means_lr: float
    dc_lr: float
    sh_lr: float
    opacity_lr: float
    scaling_lr: float
    rotation_lr: float
    position_lr_init: Optional[float] = None
    position_lr_final: float = 1.6e-6
    position_lr_delay_mult: float = 0.01
    position_lr_max_steps: int = 30000
    spatial_lr_scale: float = 1.0
    betas: Tuple[float, float] = (0.9, 0.99)
    sh_lr_divisor: float = 20.0


MAIN_PARAMS = ("means3d", "features_dc", "opacity_logits", "log_scales", "rotations")


class FastGSOptimizerPolicy:
    """The FastGS training optimizer policy on fused Adam kernels.

    ``params`` maps the reference's parameter names (``means3d``,
    ``features_dc``, ``opacity_logits``, ``log_scales``, ``rotations``,
    ``features_rest``) to GPU tensors whose ``.grad`` the training step fills.
    """

    def __init__(self, cfg: OptimizerPolicyConfig, params: Dict[str, torch.Tensor]):
        self.cfg = cfg
        lrs = {"means3d": cfg.means_lr, "features_dc": cfg.dc_lr,
               "opacity_logits": cfg.opacity_lr, "log_scales": cfg.scaling_lr,
               "rotations": cfg.rotation_lr}
        self.main_optimizers = {n: FusedAdam([params[n]], lr=lrs[n], betas=cfg.betas)
                                for n in MAIN_PARAMS if n in params}
        self.sh_optimizer = None
        if "features_rest" in params:
            self.sh_optimizer = FusedAdam([params["features_rest"]],
                                          lr=cfg.sh_lr / cfg.sh_lr_divisor, betas=cfg.betas)
        xyz_lr_init = cfg.position_lr_init if cfg.position_lr_init is not None else cfg.means_lr
        self.xyz_scheduler = expon_lr_func(
            lr_init=xyz_lr_init * cfg.spatial_lr_scale,
            lr_final=cfg.position_lr_final * cfg.spatial_lr_scale,
            lr_delay_mult=cfg.position_lr_delay_mult, max_steps=cfg.position_lr_max_steps)

    def update_learning_rate(self, iteration: int) -> float:
        lr = self.xyz_scheduler(iteration)
        if "means3d" in self.main_optimizers:
            self.main_optimizers["means3d"].param_groups[0]["lr"] = lr
        return lr

    @staticmethod
    def should_step_main(iteration: int) -> bool:
        if iteration <= 15000:
            return True
        if iteration <= 20000:
            return iteration % 32 == 0
        return iteration % 64 == 0

    @staticmethod
    def should_step_sh(iteration: int) -> bool:
        if iteration <= 15000:
            return iteration % 16 == 0
        if iteration <= 20000:
            return iteration % 32 == 0
        return iteration % 64 == 0

    def apply_gradients(self, iteration: int) -> None:
        if self.should_step_main(iteration):
            for opt in self.main_optimizers.values():
                opt.step()
        if self.sh_optimizer is not None and self.should_step_sh(iteration):
            self.sh_optimizer.step()
