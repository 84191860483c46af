"""Fused L1 + SSIM loss (csrc/fgs_loss.hip) against a float64 PyTorch reference
of the same loss (separable 11x11 Gaussian window, sigma 1.5, zero padding,
C1 = 0.01^2, C2 = 0.03^2), value and gradient."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _ref_loss(torch, img, tgt, w_l1, w_ssim):
    import torch.nn.functional as F

    x = torch.arange(11, dtype=torch.float64) - 5
    g = torch.exp(-(x * x) / (2 * 1.5 * 1.5))
    g = g / g.sum()
    C = img.shape[0]
    kx = g.view(1, 1, 1, 11).expand(C, 1, 1, 11).contiguous()
    ky = g.view(1, 1, 11, 1).expand(C, 1, 11, 1).contiguous()

    def blur(z):
        return F.conv2d(F.conv2d(z, kx, padding=(0, 5), groups=C), ky, padding=(5, 0), groups=C)

    a, b = img.unsqueeze(0), tgt.unsqueeze(0)
    mu_a, mu_b = blur(a), blur(b)
    saa = blur(a * a) - mu_a * mu_a
    sbb = blur(b * b) - mu_b * mu_b
    sab = blur(a * b) - mu_a * mu_b
    C1, C2 = 0.01 ** 2, 0.03 ** 2
    s = ((2 * mu_a * mu_b + C1) * (2 * sab + C2)) / ((mu_a ** 2 + mu_b ** 2 + C1) * (saa + sbb + C2))
    return w_l1 * (img - tgt).abs().mean() + w_ssim * (1 - s.mean())


@pytest.mark.parametrize("shape,w", [((3, 67, 93), (1.0, 0.2)), ((3, 128, 96), (0.8, 0.2)),
                                     ((1, 33, 31), (0.0, 1.0))])
def test_l1_ssim_matches_torch_float64(shape, w):
    import torch

    import fastgs_core_amd

    print("[gpu-test] fused loss", shape, w, flush=True)
    rng = np.random.default_rng(sum(shape))
    # smooth-ish images so SSIM is far from its trivial regime
    base = rng.uniform(0, 1, shape).astype(np.float32)
    tgt = np.clip(base + rng.normal(0, 0.1, shape), 0, 1).astype(np.float32)
    img_ref = torch.from_numpy(base.astype(np.float64)).requires_grad_(True)
    ref = _ref_loss(torch, img_ref, torch.from_numpy(tgt.astype(np.float64)), *w)
    ref.backward()
    img = torch.from_numpy(base).cuda().requires_grad_(True)
    loss = fastgs_core_amd.l1_ssim_loss(img, torch.from_numpy(tgt).cuda(), *w)
    (3.0 * loss).backward()
    assert abs(float(loss) - float(ref)) <= 2e-6 * abs(float(ref)) + 1e-7
    g = img.grad.cpu().numpy().astype(np.float64)
    r = 3.0 * img_ref.grad.numpy()
    np.testing.assert_allclose(g, r, rtol=1e-4, atol=1e-5 * np.abs(r).max())
