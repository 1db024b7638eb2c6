"""GPU parity of the fused cross-entropy (include/naju_loss.h,
naju_amd/xent.py) against the reference's loss call,
nn.functional.cross_entropy(logits.reshape(-1, V), y.reshape(-1)) with its
defaults (evals/lm/train.py:74), evaluated on the CPU in float64 on the same
(quantised) logits, with autograd for the gradient."""
import math

import pytest
import torch
import torch.nn.functional as F

from naju_amd.xent import cross_entropy

pytestmark = pytest.mark.gpu


def _ref(x, t, ignore_index=-100, dloss=1.0):
    xr = x.detach().cpu().double().requires_grad_(True)
    loss = F.cross_entropy(xr, t.cpu(), ignore_index=ignore_index)
    (loss * dloss).backward()
    return loss.detach(), xr.grad


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _case(dev, rows, cols, dtype, seed=0, ignore_frac=0.0, spread=3.0, strided=False, dloss=1.0):
    g = torch.Generator().manual_seed(seed)
    width = cols + 3 if strided else cols
    xs = (torch.randn(rows, width, generator=g) * spread).to(dtype)
    t = torch.randint(0, cols, (rows,), generator=g)
    if ignore_frac > 0:
        t[torch.rand(rows, generator=g) < ignore_frac] = -100
    xg = xs.to(dev).requires_grad_(True)
    xin = xg[:, :cols] if strided else xg
    loss = cross_entropy(xin, t.to(dev))
    (loss * dloss).backward()
    lr, gr = _ref(xs[:, :cols], t, dloss=dloss)
    gx = xg.grad[:, :cols] if strided else xg.grad
    if strided:
        assert torch.count_nonzero(xg.grad[:, cols:]) == 0
    return loss.detach(), lr, gx, gr


@pytest.mark.parametrize("cols", [1, 7, 8, 9, 1000, 1001, 4099])
def test_xent_fp32_matches_cross_entropy(gpu, cols):
    """fp32 logits, widths below / at / around the 16-byte vector and odd
    widths (every row starts at a different alignment)."""
    loss, lr, gx, gr = _case(gpu, 37, cols, torch.float32, seed=cols)
    assert loss.dtype == torch.float32 and loss.dim() == 0
    assert abs(float(loss) - float(lr)) <= 2e-6 * max(1.0, abs(float(lr)))
    assert gx.dtype == torch.float32
    assert _rel(gx, gr) < 1e-5


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_xent_half_logits_lm_vocab(gpu, dtype):
    """The LM's vocabulary (50257, odd: rows at every 2-byte alignment), half
    logits read directly, float32 arithmetic, the gradient in the logits'
    dtype (one rounding, 2^-8 relative for bf16, 2^-11 for fp16)."""
    loss, lr, gx, gr = _case(gpu, 64, 50257, dtype, seed=3)
    assert abs(float(loss) - float(lr)) <= 2e-6 * abs(float(lr))
    assert gx.dtype == dtype
    u = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = (gx.double().cpu() - gr).abs()
    assert float(err.max()) <= u * float(gr.abs().max()) * 1.01
    assert _rel(gx, gr) < 2e-3


def test_xent_ignore_index_and_strided_rows(gpu):
    loss, lr, gx, gr = _case(gpu, 50, 333, torch.float32, seed=7, ignore_frac=0.3, strided=True, dloss=2.5)
    assert abs(float(loss) - float(lr)) <= 2e-6 * abs(float(lr))
    assert _rel(gx, gr) < 1e-5


def test_xent_all_ignored_is_nan_with_zero_grad(gpu):
    x = torch.randn(4, 10, device=gpu, requires_grad=True)
    t = torch.full((4,), -100, dtype=torch.int64, device=gpu)
    loss = cross_entropy(x, t)
    loss.backward()
    loss = loss.detach()
    ref = F.cross_entropy(x.detach().cpu(), t.cpu())
    assert math.isnan(float(loss)) and math.isnan(float(ref))
    assert torch.count_nonzero(x.grad) == 0


def test_xent_bad_target_gives_nan_not_fault(gpu):
    x = torch.randn(3, 10, device=gpu, requires_grad=True)
    t = torch.tensor([1, 10, 2], device=gpu)  # 10 is out of range
    loss = cross_entropy(x, t)
    loss.backward()
    assert math.isnan(float(loss.detach()))
    assert torch.isnan(x.grad[1]).all() and torch.isfinite(x.grad[0]).all() and torch.isfinite(x.grad[2]).all()


def test_xent_extreme_logits(gpu):
    """Large spreads (exp underflows for most classes) and -inf logits."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(16, 777, generator=g) * 60.0
    x[0, :100] = -float("inf")
    t = torch.randint(100, 777, (16,), generator=g)
    xg = x.to(gpu).requires_grad_(True)
    loss = cross_entropy(xg, t.to(gpu))
    loss.backward()
    loss = loss.detach()
    lr, gr = _ref(x, t)
    assert abs(float(loss) - float(lr)) <= 2e-6 * abs(float(lr))
    assert _rel(xg.grad, gr) < 1e-5
    assert torch.count_nonzero(xg.grad[0, :100]) == 0


def test_xent_deterministic_and_matches_lm_shape(gpu):
    """Bitwise-identical repeats at 2048 rows x 50257 bf16 (one eighth of the
    C5 batch), and agreement with torch's own float32 path."""
    torch.manual_seed(2)
    x = (torch.randn(2048, 50257, device=gpu) * 2).to(torch.bfloat16)
    t = torch.randint(0, 50257, (2048,), device=gpu)
    outs = []
    for _ in range(2):
        xg = x.clone().requires_grad_(True)
        loss = cross_entropy(xg, t)
        loss.backward()
        outs.append((loss.detach().clone(), xg.grad.clone()))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    xt = x.float().requires_grad_(True)
    lt = F.cross_entropy(xt, t)
    lt.backward()
    lt = lt.detach()
    assert abs(float(outs[0][0]) - float(lt)) <= 2e-6 * float(lt)
    assert _rel(outs[0][1], xt.grad) < 2e-3


@pytest.mark.parametrize("dloss", [1.0, 0.5])
def test_xent_gradient_from_forward_matches_two_passes(gpu, dloss):
    """With logits that require grad the forward also writes the gradient
    (naju_xent_fwd_grad) and the backward keeps it when dloss is 1
    (naju_xent_bwd_if_scaled), else rewrites it: bitwise what
    naju_xent_fwd + naju_xent_bwd give, with ignored rows; a retained graph's
    second backward recomputes."""
    from naju_amd import _lib
    L = _lib.lib()
    rows, cols = 96, 50257
    g = torch.Generator(device=gpu).manual_seed(11)
    x = (torch.randn(rows, cols, generator=g, device=gpu) * 3).to(torch.bfloat16)
    t = torch.randint(0, cols, (rows,), generator=g, device=gpu)
    t[::7] = -100
    xg = x.clone().requires_grad_(True)
    loss = cross_entropy(xg, t)
    (loss * dloss).backward(retain_graph=True)
    g1 = xg.grad.clone()
    (loss * dloss).backward()
    # the two-pass calls
    st = torch.cuda.current_stream(gpu).cuda_stream
    lse = torch.empty(rows, device=gpu)
    loss2, scale = torch.empty((), device=gpu), torch.empty((), device=gpu)
    ws = torch.empty(L.naju_xent_workspace_bytes(rows), dtype=torch.uint8, device=gpu)
    _lib.check_loss(L.naju_xent_fwd(x.data_ptr(), cols, t.data_ptr(), rows, cols, _lib.DT_BF16, -100, lse.data_ptr(),
                                    loss2.data_ptr(), scale.data_ptr(), ws.data_ptr(), ws.numel(), st))
    dl = torch.full((), dloss, device=gpu)
    dx = torch.empty_like(x)
    _lib.check_loss(L.naju_xent_bwd(x.data_ptr(), cols, t.data_ptr(), rows, cols, _lib.DT_BF16, -100, lse.data_ptr(),
                                    scale.data_ptr(), dl.data_ptr(), dx.data_ptr(), cols, _lib.DT_BF16, st))
    torch.cuda.synchronize()
    assert torch.equal(loss.detach(), loss2)
    assert torch.equal(g1, dx)
    assert torch.equal(xg.grad, dx + dx)
    assert torch.count_nonzero(dx[::7]) == 0
