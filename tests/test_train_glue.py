"""Training-step glue (csrc/fgs_train.hip, fastgs_core_amd/train.py): fused
parameter activations, fused Adam and the FastGS optimizer policy
(scripts/train_scanner_fastgs.py:54-182 of the reference)."""
import math

import numpy as np
import pytest

import fastgs_core_amd as fg


# ---------------------------------------------------------------------------
# CPU: policy cadence, learning-rate schedule, no CPU fallback
def test_policy_cadence_boundaries():
    main = fg.FastGSOptimizerPolicy.should_step_main
    sh = fg.FastGSOptimizerPolicy.should_step_sh
    assert all(main(i) for i in (1, 2, 15, 15000))
    # (15000, 20000]: every 32 iterations; beyond: every 64
    assert not main(15001) and main(15008) and not main(15039) and main(20000)
    assert not main(20064) and main(20096)  # 20064 % 32 == 0 but % 64 != 0
    assert [i for i in range(1, 65) if sh(i)] == [16, 32, 48, 64]
    assert not sh(15024) and sh(15040)  # 15024 % 16 == 0 but % 32 != 0
    assert not sh(20064) and sh(20096)


def test_expon_lr_schedule_closed_form():
    f = fg.expon_lr_func(1e-2, 1e-4, max_steps=1000)
    assert f(0) == pytest.approx(1e-2, rel=1e-12)
    assert f(1000) == pytest.approx(1e-4, rel=1e-12)
    assert f(500) == pytest.approx(math.sqrt(1e-2 * 1e-4), rel=1e-12)  # log-linear midpoint
    assert f(5000) == pytest.approx(1e-4, rel=1e-12)                   # clamped
    assert f(-1) == 0.0
    g = fg.expon_lr_func(1e-2, 1e-4, lr_delay_steps=100, lr_delay_mult=0.01, max_steps=1000)
    assert g(0) == pytest.approx(0.01 * 1e-2, rel=1e-12)
    assert g(100) == pytest.approx(f(100), rel=1e-12)
    assert g(50) == pytest.approx((0.01 + 0.99 * math.sin(math.pi / 4)) * f(50), rel=1e-12)


def test_glue_has_no_cpu_fallback():
    import torch

    with pytest.raises(RuntimeError, match="ROCm GPU"):
        fg.activate(torch.zeros(4, 3), torch.zeros(4, 4), torch.zeros(4))


# ---------------------------------------------------------------------------
# GPU
@pytest.mark.gpu
def test_activations_match_torch_fp32():
    import torch

    print("[gpu-test] activations", flush=True)
    rng = np.random.default_rng(3)
    P = 5000
    ls = rng.normal(-4, 1, (P, 3)).astype(np.float32)
    q = rng.normal(0, 1, (P, 4)).astype(np.float32)
    q[7] = 0.0  # zero quaternion: rotation 0, gradient d_r / 1e-8
    lg = rng.normal(0, 2, (P, 1)).astype(np.float32)
    dev = torch.device("cuda")
    args = [torch.from_numpy(a).to(dev).requires_grad_(True) for a in (ls, q, lg)]
    s, r, o = fg.activate(*args)
    ref_args = [torch.from_numpy(a).to(dev).requires_grad_(True) for a in (ls, q, lg)]
    s_ref = torch.exp(ref_args[0])
    r_ref = ref_args[1] / (ref_args[1].norm(dim=1, keepdim=True) + 1e-8)
    o_ref = torch.sigmoid(ref_args[2])
    for a, b in ((s, s_ref), (r, r_ref), (o, o_ref)):
        torch.testing.assert_close(a, b, rtol=2e-6, atol=1e-7)
    gs = [torch.from_numpy(rng.normal(0, 1, t.shape).astype(np.float32)).to(dev)
          for t in (s, r, o)]
    torch.autograd.backward([s, r, o], gs)
    torch.autograd.backward([s_ref, r_ref, o_ref], gs)
    for a, b in zip(args, ref_args):
        mask = torch.ones_like(a.grad, dtype=torch.bool)
        if a.shape[1] == 4:
            mask[7] = False  # torch's norm backward at 0 differs only in the 0/0 convention
        torch.testing.assert_close(a.grad[mask], b.grad[mask], rtol=1e-5, atol=1e-6)
    assert torch.isfinite(args[1].grad[7]).all()


@pytest.mark.gpu
def test_fused_adam_bias_corrected_matches_torch_adam():
    import torch

    print("[gpu-test] fused adam vs torch.optim.Adam", flush=True)
    dev = torch.device("cuda")
    torch.manual_seed(0)
    p0 = torch.randn(10007, device=dev)
    a = p0.clone().requires_grad_(True)
    b = p0.clone().requires_grad_(True)
    oa = fg.FusedAdam([a], lr=3e-3, betas=(0.9, 0.99), eps=1e-8, bias_correction=True)
    ob = torch.optim.Adam([b], lr=3e-3, betas=(0.9, 0.99), eps=1e-8, foreach=False)
    for _ in range(6):
        g = torch.randn_like(p0)
        a.grad = g.clone()
        b.grad = g.clone()
        oa.step()
        ob.step()
    torch.testing.assert_close(a.detach(), b.detach(), rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(oa.state[a]["exp_avg_sq"], ob.state[b]["exp_avg_sq"], rtol=1e-5,
                               atol=1e-9)


@pytest.mark.gpu
def test_fused_adam_mlx_form_constant_gradient_closed_form():
    """MLX Adam (no bias correction) with a constant gradient g:
    m_t = g (1 - b1^t), v_t = g^2 (1 - b2^t), p_t = p_0 - sum_k lr m_k / (sqrt(v_k) + eps)."""
    import torch

    print("[gpu-test] fused adam closed form", flush=True)
    dev = torch.device("cuda")
    g = torch.tensor([0.5, -2.0, 1e-3, 0.0, 7.0], device=dev)
    p = torch.zeros_like(g).requires_grad_(True)
    lr, b1, b2, eps = 1e-2, 0.9, 0.99, 1e-8
    opt = fg.FusedAdam([p], lr=lr, betas=(b1, b2), eps=eps)
    T = 12
    for _ in range(T):
        p.grad = g.clone()
        opt.step()
    gd = g.double().cpu().numpy()
    want = np.zeros_like(gd)
    for t in range(1, T + 1):
        m = gd * (1 - b1 ** t)
        v = gd * gd * (1 - b2 ** t)
        want -= lr * m / (np.sqrt(v) + eps)
    np.testing.assert_allclose(p.detach().double().cpu().numpy(), want, rtol=2e-5, atol=1e-9)
    np.testing.assert_allclose(opt.state[p]["exp_avg"].double().cpu().numpy(),
                               gd * (1 - b1 ** T), rtol=2e-6, atol=1e-12)


@pytest.mark.gpu
def test_fastgs_policy_steps_on_cadence():
    import torch

    print("[gpu-test] optimizer policy cadence", flush=True)
    dev = torch.device("cuda")
    names = ("means3d", "features_dc", "opacity_logits", "log_scales", "rotations",
             "features_rest")
    params = {n: torch.zeros(64, device=dev, requires_grad=True) for n in names}
    cfg = fg.OptimizerPolicyConfig(means_lr=1e-3, dc_lr=1e-3, sh_lr=1e-3, opacity_lr=1e-3,
                                   scaling_lr=1e-3, rotation_lr=1e-3)
    pol = fg.FastGSOptimizerPolicy(cfg, params)
    assert pol.sh_optimizer.param_groups[0]["lr"] == pytest.approx(1e-3 / 20.0)
    sh_changes = []
    for it in range(1, 33):
        for t in params.values():
            t.grad = torch.ones_like(t)
        before = params["features_rest"].detach().clone()
        m_before = params["means3d"].detach().clone()
        pol.update_learning_rate(it)
        pol.apply_gradients(it)
        assert not torch.equal(params["means3d"].detach(), m_before)  # main steps every iteration
        if not torch.equal(params["features_rest"].detach(), before):
            sh_changes.append(it)
    assert sh_changes == [16, 32]


@pytest.mark.gpu
@pytest.mark.parametrize("bias_correction", [0, 1])
def test_adam_multi_matches_single_tensor_steps(bias_correction):
    """fgs_adam_step_multi over tensors of different sizes, learning rates and
    step counts gives the bits of one fgs_adam_step per tensor."""
    import ctypes

    import torch

    from fastgs_core_amd import _lib
    from fastgs_core_amd.rasterizer import _p, _stream

    print(f"[gpu-test] adam multi vs single bc={bias_correction}", flush=True)
    lib = _lib.load()
    dev = torch.device("cuda")
    torch.manual_seed(1)
    sizes, lrs, steps = [1, 255, 256, 257, 10007, 3], [1e-3, 3e-3, 1e-4, 5e-2, 2e-3, 1.0], \
        [1, 2, 7, 30, 3, 1000]
    single = [[torch.randn(n, device=dev) for _ in range(4)] for n in sizes]
    for t in single:
        t[3] = t[3].abs()  # second moments are non-negative
    multi = [[x.clone() for x in t] for t in single]
    for (p, g, m, v), lr, st in zip(single, lrs, steps):
        _lib.check(lib.fgs_adam_step(_p(p), _p(g), _p(m), _p(v), p.numel(), lr, 0.9, 0.99, 1e-8,
                                     st, bias_correction, _stream(dev)))
    groups = [_lib.AdamGroup(_p(p), _p(g), _p(m), _p(v), p.numel(), lr, st)
              for (p, g, m, v), lr, st in zip(multi, lrs, steps)]
    arr = (_lib.AdamGroup * len(groups))(*groups)
    _lib.check(lib.fgs_adam_step_multi(arr, len(groups), 0.9, 0.99, 1e-8, bias_correction,
                                       _stream(dev)))
    for a, b in zip(single, multi):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    with pytest.raises(ValueError):
        over = (_lib.AdamGroup * 9)(*(groups + groups[:3]))
        _lib.check(lib.fgs_adam_step_multi(over, 9, 0.9, 0.99, 1e-8, 0, _stream(dev)))


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["l1", "mse"])
def test_pointwise_loss_matches_torch_float64(mode):
    import torch

    print(f"[gpu-test] pointwise loss {mode}", flush=True)
    dev = torch.device("cuda")
    torch.manual_seed(2)
    x = torch.rand(3, 97, 131, device=dev)
    y = torch.rand(3, 97, 131, device=dev)
    y[0, 0, :7] = x[0, 0, :7]  # ties: the L1 gradient is 0 there
    xa = x.clone().requires_grad_(True)
    fn = fg.l1_loss if mode == "l1" else fg.mse_loss
    loss = fn(xa, y)
    loss.backward(torch.tensor(1.7, device=dev))
    xd = x.double().cpu().requires_grad_(True)
    d = xd - y.double().cpu()
    ref = d.abs().mean() if mode == "l1" else (d * d).mean()
    (ref * 1.7).backward()
    assert abs(float(loss) - float(ref)) <= 1e-6 * abs(float(ref))
    torch.testing.assert_close(xa.grad.double().cpu(), xd.grad, rtol=1e-6, atol=1e-12)
    if mode == "l1":
        assert (xa.grad[0, 0, :7] == 0).all()
