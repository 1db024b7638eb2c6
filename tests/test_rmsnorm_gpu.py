"""GPU parity of the fused RMSNorm (include/naju_mixer.h, naju_amd/rmsnorm.py)
against the reference's expression weight * x * rsqrt(mean(x^2) + eps)
(naju/mixer.py:51-58), evaluated on the CPU in float64 with autograd."""
import pytest
import torch

from naju_amd.mixer import RMSNorm
from naju_amd.rmsnorm import rms_norm, supported

pytestmark = pytest.mark.gpu


def _ref(x, w, eps, dy):
    xr = x.detach().cpu().double().requires_grad_(True)
    wr = w.detach().cpu().double().requires_grad_(True)
    y = wr * xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + eps)
    y.backward(dy.detach().cpu().double())
    return y.detach(), xr.grad, wr.grad


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _run(dev, shape, x_dtype=torch.float32, out_dtype=torch.float32, seed=0, eps=1e-5):
    g = torch.Generator().manual_seed(seed)
    d = shape[-1]
    x = (torch.randn(*shape, generator=g) * 2 + 0.5).to(x_dtype)
    w = 1 + 0.1 * torch.randn(d, generator=g)
    dy = torch.randn(*shape, generator=g).to(out_dtype)
    xg = x.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    assert supported(xg)
    y = rms_norm(xg, wg, eps, out_dtype)
    assert y.dtype == out_dtype and y.shape == x.shape
    y.backward(dy.to(dev))
    yr, dxr, dwr = _ref(x, w, eps, dy)
    return (y.detach(), yr), (xg.grad, dxr), (wg.grad, dwr)


@pytest.mark.parametrize("d", [4, 8, 252, 768, 1000, 2048, 2052, 4096])
@pytest.mark.parametrize("rows", [1, 17, 100])
def test_rmsnorm_fp32_matches_reference(gpu, d, rows):
    (y, yr), (dx, dxr), (dw, dwr) = _run(gpu, (rows, d), seed=d + rows)
    assert _rel(y, yr) < 1e-6
    assert _rel(dx, dxr) < 1e-5
    assert _rel(dw, dwr) < 1e-5


def test_rmsnorm_bf16_output_for_autocast_gemm(gpu):
    """y written in bf16 (what the GEMM's autocast cast would give), bf16 dy
    from that GEMM's backward, float32 dx and dw."""
    (y, yr), (dx, dxr), (dw, dwr) = _run(gpu, (4, 512, 768), out_dtype=torch.bfloat16, seed=1)
    err = (y.double().cpu() - yr).abs()
    assert float((err / yr.abs().clamp_min(1e-30)).max()) <= 2.0 ** -8 + 1e-6
    assert dx.dtype == torch.float32
    assert _rel(dx, dxr) < 1e-5
    assert _rel(dw, dwr) < 1e-5


def test_rmsnorm_bf16_input(gpu):
    (y, yr), (dx, dxr), (dw, dwr) = _run(gpu, (300, 768), x_dtype=torch.bfloat16, out_dtype=torch.bfloat16, seed=2)
    assert dx.dtype == torch.bfloat16
    assert _rel(y, yr) < 2e-3
    assert _rel(dx, dxr) < 2e-3
    assert _rel(dw, dwr) < 1e-5


def test_rmsnorm_deterministic_lm_shape(gpu):
    """The C5 residual stream: 16384 rows x 768, dweight bitwise repeatable."""
    torch.manual_seed(3)
    x = torch.randn(8, 2048, 768, device=gpu)
    w = (1 + 0.1 * torch.randn(768, device=gpu)).requires_grad_(True)
    dy = torch.randn(8, 2048, 768, device=gpu).to(torch.bfloat16)
    outs = []
    for _ in range(2):
        w.grad = None
        xg = x.clone().requires_grad_(True)
        y = rms_norm(xg, w, 1e-5, torch.bfloat16)
        y.backward(dy)
        outs.append((y.clone(), xg.grad.clone(), w.grad.clone()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)
    yr, dxr, dwr = _ref(x, w, 1e-5, dy)
    assert _rel(outs[0][1], dxr) < 1e-5
    assert _rel(outs[0][2], dwr) < 1e-5


def test_rmsnorm_module_matches_reference_expression(gpu):
    """The module's default output dtype follows the reference expression;
    shapes the kernels do not serve take that expression itself."""
    torch.manual_seed(4)
    for d in (768, 6):
        m = RMSNorm(d).to(gpu)
        with torch.no_grad():
            m.weight.add_(0.1 * torch.randn(d, device=gpu))
        x = torch.randn(5, 7, d, device=gpu)
        y = m(x)
        ref = m.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + m.eps)
        assert y.dtype == ref.dtype
        assert _rel(y, ref) < 1e-6
        assert supported(x) == (d == 768)
