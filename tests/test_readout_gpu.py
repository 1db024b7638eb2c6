"""GPU parity of the mixer's readout epilogue (include/naju_mixer.h,
naju_amd/readout.py), y = (cx * scale + D * h) * SiLU(z) as in
naju/mixer.py:123-124, against the same expression in float64 on the CPU with
autograd."""
import pytest
import torch
import torch.nn.functional as F

from naju_amd.readout import readout

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _case(dev, B, T, C, dtype, out_dtype, strided_z=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    cx = torch.randn(B, T, C, generator=g).to(dtype)
    h = torch.randn(B, T, C, generator=g).to(dtype)
    zz = torch.randn(B, T, 2 * C if strided_z else C, generator=g).to(dtype)
    D = torch.randn(C, generator=g)
    dy = torch.randn(B, T, C, generator=g)
    scale = 0.125
    # reference
    r = [t.double().requires_grad_(True) for t in (cx, h, zz, D)]
    zr = r[2][..., C:] if strided_z else r[2]
    yr = (r[0] * scale + r[3] * r[1]) * F.silu(zr)
    yr.backward(dy.double())
    # HIP
    k = [t.to(dev).requires_grad_(True) for t in (cx, h, zz, D)]
    zk = k[2][..., C:] if strided_z else k[2]
    y = readout(k[0], k[1], zk, k[3], scale, out_dtype=out_dtype)
    assert y.dtype == out_dtype
    y.backward(dy.to(dev).to(out_dtype))
    names = ("y", "dcx", "dh", "dz", "dD")
    return {n: (a, b) for n, a, b in zip(names, (y, k[0].grad, k[1].grad, k[2].grad, k[3].grad),
                                          (yr, r[0].grad, r[1].grad, r[2].grad, r[3].grad))}


@pytest.mark.parametrize("T", [1, 63, 64, 130])
def test_readout_fp32(gpu, T):
    for name, (a, b) in _case(gpu, 2, T, 72, torch.float32, torch.float32, seed=T).items():
        assert _rel(a, b) < 1e-5, (T, name, _rel(a, b))


def test_readout_strided_z(gpu):
    for name, (a, b) in _case(gpu, 2, 100, 300, torch.float32, torch.float32, strided_z=True).items():
        assert _rel(a, b) < 1e-5, (name, _rel(a, b))


def test_readout_bf16(gpu):
    """bf16 reads, float32 arithmetic, one rounding per bf16 output."""
    for name, (a, b) in _case(gpu, 2, 200, 264, torch.bfloat16, torch.bfloat16, strided_z=True).items():
        tol = 2e-3 if name == "dD" else 8e-3
        assert _rel(a, b) < tol, (name, _rel(a, b))


def test_readout_dD_deterministic_and_long_sum(gpu):
    """The C5 shape: dD sums 16384 rows per channel, in a fixed order."""
    torch.manual_seed(3)
    B, T, C = 8, 2048, 1536
    cx, h, z = (torch.randn(B, T, C, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    D = torch.randn(C, device=gpu, requires_grad=True)
    dy = torch.randn(B, T, C, device=gpu, dtype=torch.bfloat16)
    outs = []
    for _ in range(2):
        D.grad = None
        readout(cx, h, z, D, 0.125, out_dtype=torch.bfloat16).backward(dy)
        outs.append(D.grad.clone())
    assert torch.equal(outs[0], outs[1])
    ref = (dy.double() * F.silu(z.double()) * h.double()).sum((0, 1))
    assert _rel(outs[0], ref) < 1e-5
