"""Fused photometric loss of the FastGS training step on the GPU.

    L = w_l1 * mean|img - target| + w_ssim * (1 - mean SSIM(img, target))

SSIM uses an 11x11 Gaussian window (sigma 1.5), zero padding, per channel,
C1 = 0.01^2, C2 = 0.03^2 -- the loss the reference training scripts apply to
``out_color`` (scripts/train_scanner_fastgs.py:911-966).  Forward and
backward are single HIP kernels each (csrc/fgs_loss.hip); the gradient is
taken w.r.t. ``img`` only.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .rasterizer import _p, _stream, _stage


class _L1SSIM(torch.autograd.Function):
    @staticmethod
    def forward(ctx, img, tgt, w_l1, w_ssim):
        lib = _lib.load()
        C, H, W = img.shape
        dev = img.device
        loss = torch.empty((), dtype=torch.float32, device=dev)
        need = img.requires_grad
        dmaps = torch.empty((3, C, H, W), dtype=torch.float32, device=dev) if need else None
        ws = torch.empty(int(lib.fgs_l1_ssim_workspace_bytes(C, H, W)), dtype=torch.uint8,
                         device=dev)
        with _stage("loss_fwd"):
            _lib.check(lib.fgs_l1_ssim_fwd(_p(img), _p(tgt), C, H, W, float(w_l1), float(w_ssim),
                                           _p(loss), _p(dmaps), _p(ws), _stream(dev)))
        ctx.save_for_backward(img, tgt, dmaps)
        ctx.w = (float(w_l1), float(w_ssim))
        return loss

    @staticmethod
    def backward(ctx, g):
        lib = _lib.load()
        img, tgt, dmaps = ctx.saved_tensors
        C, H, W = img.shape
        g = g.to(torch.float32).contiguous()
        dimg = torch.empty_like(img)
        with _stage("loss_bwd"):
            _lib.check(lib.fgs_l1_ssim_bwd(_p(img), _p(tgt), _p(dmaps), _p(g), C, H, W, ctx.w[0],
                                           ctx.w[1], _p(dimg), _stream(img.device)))
        return dimg, None, None, None


def l1_ssim_loss(img: torch.Tensor, target: torch.Tensor, w_l1: float = 1.0,
                 w_ssim: float = 0.2) -> torch.Tensor:
    """Scalar loss of [C,H,W] float32 images on the GPU (differentiable in ``img``)."""
    if img.dim() != 3 or img.shape != target.shape:
        raise ValueError(f"l1_ssim_loss expects two [C,H,W] images of the same shape, got "
                         f"{tuple(img.shape)} and {tuple(target.shape)}")
    if not img.is_cuda:
        raise RuntimeError("fastgs_core_amd requires a ROCm GPU; there is no CPU fallback")
    img = img.to(torch.float32).contiguous()
    target = target.detach().to(device=img.device, dtype=torch.float32).contiguous()
    return _L1SSIM.apply(img, target, w_l1, w_ssim)


class _Pointwise(torch.autograd.Function):
    @staticmethod
    def forward(ctx, img, tgt, mode):
        lib = _lib.load()
        dev = img.device
        n = img.numel()
        loss = torch.empty((), dtype=torch.float32, device=dev)
        ws = torch.empty(int(lib.fgs_pointwise_loss_workspace_bytes(n)), dtype=torch.uint8,
                         device=dev)
        with _stage("loss_fwd"):
            _lib.check(lib.fgs_pointwise_loss_fwd(_p(img), _p(tgt), n, mode, _p(ws), _p(loss),
                                                  _stream(dev)))
        ctx.save_for_backward(img, tgt)
        ctx.mode = mode
        return loss

    @staticmethod
    def backward(ctx, g):
        lib = _lib.load()
        img, tgt = ctx.saved_tensors
        g = g.to(torch.float32).contiguous()
        dimg = torch.empty_like(img)
        with _stage("loss_bwd"):
            _lib.check(lib.fgs_pointwise_loss_bwd(_p(img), _p(tgt), img.numel(), ctx.mode, _p(g),
                                                  _p(dimg), _stream(img.device)))
        return dimg, None, None


def _pointwise(img: torch.Tensor, target: torch.Tensor, mode: int, name: str) -> torch.Tensor:
    if img.shape != target.shape or img.numel() == 0:
        raise ValueError(f"{name} expects two non-empty tensors of one shape, got "
                         f"{tuple(img.shape)} and {tuple(target.shape)}")
    if not img.is_cuda:
        raise RuntimeError("fastgs_core_amd requires a ROCm GPU; there is no CPU fallback")
    img = img.to(torch.float32).contiguous()
    target = target.detach().to(device=img.device, dtype=torch.float32).contiguous()
    return _Pointwise.apply(img, target, mode)


def l1_loss(img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean |img - target| (the training script's L1, train_scanner_fastgs.py:962):
    one HIP kernel pair each way, sums in double; differentiable in ``img``."""
    return _pointwise(img, target, 0, "l1_loss")


def mse_loss(img: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """mean (img - target)^2 (the training script's MSE, train_scanner_fastgs.py:963)."""
    return _pointwise(img, target, 1, "mse_loss")
