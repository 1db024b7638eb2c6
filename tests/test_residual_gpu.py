"""The pre-norm block's residual add with dropout (naju_amd.residual, the
reference's u + Dropout(p)(mix), naju/mixer.py:131-144) and the RMSNorm
fork whose backward adds the residual gradient (naju_amd.rmsnorm
.rms_norm_fork): against torch expressions in float64 / bitwise where the
arithmetic is the same."""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,dtype", [(16384 * 768, torch.bfloat16), (1000 * 37, torch.bfloat16),
                                     (4096 * 64, torch.float32)])
def test_residual_dropout_forward_backward(gpu, n, dtype):
    from naju_amd.residual import residual_dropout
    p = 0.1
    g = torch.Generator(device=gpu).manual_seed(n % 1000)
    u = torch.randn(n, generator=g, device=gpu)
    mix = torch.randn(n, generator=g, device=gpu).to(dtype)
    gout = torch.randn(n, generator=g, device=gpu)
    print(f"residual dropout n={n} {dtype} (vector path: {n % 8 == 0})", flush=True)
    ur, mr = u.clone().requires_grad_(True), mix.clone().requires_grad_(True)
    torch.manual_seed(7)
    out = residual_dropout(ur, mr, p)
    out.backward(gout)
    torch.cuda.synchronize()
    # the mask of that seed, read off a run with u = 0 and mix = 1
    torch.manual_seed(7)
    keep = residual_dropout(torch.zeros_like(u), torch.ones_like(mix), p) != 0
    frac = 1.0 - float(keep.float().mean())
    assert abs(frac - p) < 6 * math.sqrt(p * (1 - p) / n) + 1e-4, frac
    scale = 1.0 / (1.0 - p)
    kept_val = u + (mix.float() * scale).to(dtype).float()
    assert torch.equal(out[keep], kept_val[keep])
    assert torch.equal(out[~keep], u[~keep])
    # the backward draws the same mask: mix's gradient is g * scale where kept, 0 elsewhere
    assert torch.equal(ur.grad, gout)
    assert mr.grad.dtype == dtype
    assert torch.all(mr.grad[~keep] == 0)
    assert torch.equal(mr.grad[keep], (gout * scale).to(dtype)[keep])
    # the same torch seed gives the same mask
    torch.manual_seed(7)
    assert torch.equal(residual_dropout(u, mix, p), out.detach())


def test_residual_without_dropout_is_the_plain_sum(gpu):
    from naju_amd.residual import residual_dropout
    g = torch.Generator(device=gpu).manual_seed(1)
    u = torch.randn(8, 2048, 768, generator=g, device=gpu)
    mix = torch.randn(8, 2048, 768, generator=g, device=gpu).to(torch.bfloat16)
    assert torch.equal(residual_dropout(u, mix, 0.0), u + mix.float())


@pytest.mark.parametrize("shape", [(8, 2048, 768), (3, 70, 32)])
def test_rms_norm_fork_adds_the_residual_gradient(gpu, shape):
    """(x, rms_norm(x)) with gradients (dres, dy): dx = dres + the norm's
    gradient, against float64 autograd of the reference expression
    (naju/mixer.py:51-58)."""
    from naju_amd.rmsnorm import rms_norm_fork
    g = torch.Generator(device=gpu).manual_seed(shape[-1])
    x = torch.randn(*shape, generator=g, device=gpu)
    w = 1.0 + 0.1 * torch.randn(shape[-1], generator=g, device=gpu)
    dres = torch.randn(*shape, generator=g, device=gpu)
    dy = torch.randn(*shape, generator=g, device=gpu).to(torch.bfloat16)
    xh, wh = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    xr, y = rms_norm_fork(xh, wh, 1e-5, out_dtype=torch.bfloat16)
    assert torch.equal(xr, x) and y.dtype == torch.bfloat16
    torch.autograd.backward([xr, y], [dres, dy])
    x64, w64 = x.double().requires_grad_(True), w.double().requires_grad_(True)
    y64 = w64 * x64 * torch.rsqrt(x64.pow(2).mean(-1, keepdim=True) + 1e-5)
    torch.autograd.backward([x64, y64], [dres.double(), dy.double()])
    rel = lambda a, b: float((a.detach().double() - b.detach()).abs().max() / b.detach().abs().max())  # noqa: E731
    assert rel(y.float(), y64.detach()) < 2 ** -8
    assert rel(xh.grad, x64.grad) < 1e-5
    assert rel(wh.grad, w64.grad) < 1e-5
