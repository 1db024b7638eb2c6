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
