"""The mixer's linear layers (naju_amd.linear): the forward and the input
gradient are the GEMMs bf16 autocast runs for nn.Linear (bitwise), the
weight gradient is the split-K float32 product, checked against float64."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _ref_autocast(x, w, dy):
    xr = x.detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = F.linear(xr, wr)
    y.backward(dy)
    return y.detach(), xr.grad, wr.grad


@pytest.mark.parametrize("shape,n_out", [
    ((8, 2048, 1536), 768),    # out_proj of the C5 LM step: 8 token parts
    ((8, 2048, 1536), 3200),   # f / i / x projections in one GEMM: 2 parts
    ((8, 2048, 768), 3072),    # in_proj: 4 parts
    ((2, 333, 96), 40),        # ragged token count: one part
])
def test_linear_matches_autocast_and_float64(gpu, shape, n_out):
    from naju_amd.linear import _parts, linear
    g = torch.Generator(device=gpu).manual_seed(sum(shape) + n_out)
    x = torch.randn(*shape, generator=g, device=gpu).to(torch.bfloat16)
    w = torch.randn(n_out, shape[-1], generator=g, device=gpu) / shape[-1] ** 0.5
    dy = torch.randn(*shape[:-1], n_out, generator=g, device=gpu).to(torch.bfloat16)
    K = x.numel() // shape[-1]
    print(f"linear {shape} -> {n_out}: {_parts(K, n_out, shape[-1])} token parts", flush=True)
    y_ref, dx_ref, _ = _ref_autocast(x, w, dy)
    xh = x.detach().clone().requires_grad_(True)
    wh = w.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = linear(xh, wh)
    y.backward(dy)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and torch.equal(y, y_ref)
    assert xh.grad.dtype == torch.bfloat16 and torch.equal(xh.grad, dx_ref)
    assert wh.grad.dtype == torch.float32
    # dW against float64 on the same bf16 operands
    dw64 = dy.reshape(-1, n_out).double().t() @ x.reshape(-1, shape[-1]).double()
    err = float((wh.grad.double() - dw64).abs().max() / dw64.abs().max())
    assert err <= 1e-5, err



@pytest.mark.parametrize("n_parts,n,offset", [(2, 4096, 0), (4, 1000, 0), (8, 768 * 1536, 0), (16, 64, 0),
                                              (3, 999, 0), (8, 1024, 1)])
def test_sum_parts_adds_in_part_order(gpu, n_parts, n, offset):
    """naju_sum_parts: the float32 sum of the parts in part order, bitwise
    (the vector kernels for 2, 4, 8, 16 aligned parts, the element kernel
    for other counts, sizes and an unaligned start)."""
    from naju_amd import _lib
    g = torch.Generator(device=gpu).manual_seed(n_parts * 7 + n)
    buf = torch.randn(n_parts * n + offset, generator=g, device=gpu)
    parts = buf[offset:].view(n_parts, n)
    out = torch.empty(n, device=gpu)
    L = _lib.lib()
    _lib.check_mixer(L.naju_sum_parts(parts.data_ptr(), n_parts, n, out.data_ptr(),
                                      torch.cuda.current_stream(gpu).cuda_stream))
    ref = parts[0].clone()
    for q in range(1, n_parts):
        ref += parts[q]
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    with pytest.raises(_lib.NajuScanError):
        _lib.check_mixer(L.naju_sum_parts(parts.data_ptr(), 17, n, out.data_ptr(), 0))


def _rel64(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm())


@pytest.mark.parametrize("V,d,rows,via", [
    (1000, 64, (2, 96), "naju"),     # padded to 1024, gradient from naju_amd.xent
    (1000, 64, (2, 96), "torch"),    # the same with torch's cross_entropy: unpadded GEMMs
    (50257, 768, (1, 512), "naju"),  # the LM's vocabulary, padded to 50304
    (1024, 32, (3, 50), "naju"),     # already aligned: no padding
])
def test_lm_head_padded_matches_float64(gpu, monkeypatch, V, d, rows, via):
    """The padded LM head (naju_amd.linear.lm_head): logits equal F.linear's
    on the bf16 operands (a [..., V] view with row stride Vp), and with the
    loss on top the input and weight gradients agree with float64 autograd
    of the same bf16-rounded operands to the bf16 rounding of the logits'
    gradient; the padded backward GEMMs are taken exactly when the gradient
    comes from naju_amd.xent.cross_entropy in the padded layout."""
    from naju_amd import linear as lin
    from naju_amd.xent import cross_entropy
    hits = []
    real = lin.zero_padded_rows

    def spy(g, ld):
        r = real(g, ld)
        hits.append(r is not None)
        return r

    monkeypatch.setattr(lin, "zero_padded_rows", spy)
    g = torch.Generator(device=gpu).manual_seed(V + d)
    x = torch.randn(*rows, d, generator=g, device=gpu).to(torch.bfloat16).requires_grad_(True)
    w = (torch.randn(V, d, generator=g, device=gpu) * 0.5 / d ** 0.5).requires_grad_(True)
    tgt = torch.randint(0, V, (x.numel() // d,), generator=g, device=gpu)
    logits = lin.lm_head(x, w)
    Vp = -(-V // lin.HEAD_ALIGN) * lin.HEAD_ALIGN
    assert logits.shape == (*rows, V) and logits.stride(-2) == Vp and logits.dtype == torch.bfloat16
    wb = w.detach().to(torch.bfloat16)
    ref = F.linear(x.detach(), wb)
    assert _rel64(logits, ref) < 4e-3
    if via == "naju":
        loss = cross_entropy(logits.view(-1, V), tgt)
    else:
        loss = F.cross_entropy(logits.float().view(-1, V), tgt)
    loss.backward()
    torch.cuda.synchronize()
    padded = Vp > V and via == "naju"
    assert hits == ([padded] if Vp > V else []), hits
    assert w.grad.dtype == torch.float32 and w.grad.shape == (V, d)
    x64 = x.detach().double().requires_grad_(True)
    w64 = wb.double().requires_grad_(True)
    F.cross_entropy(F.linear(x64, w64).view(-1, V), tgt).backward()
    assert _rel64(x.grad, x64.grad) < 1e-2
    assert _rel64(w.grad, w64.grad) < 1e-2
