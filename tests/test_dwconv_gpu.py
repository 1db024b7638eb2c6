"""GPU parity of the depthwise causal convolution kernels (include/naju_mixer.h,
naju_amd/dwconv.py) against the reference's formulation: nn.functional.conv1d
with groups = C, padding k-1 and the slice [..., :T] on the [B, C, T]
transpose (naju/mixer.py:108-110, 115), evaluated on the CPU in float64 with
autograd for the gradients."""
import pytest
import torch
import torch.nn.functional as F

from naju_amd.dwconv import dwconv

pytestmark = pytest.mark.gpu


def _ref(x, w, bias, add, silu):
    """float64 CPU reference of y = act(add + bias + causal_dwconv(x))."""
    T, C = x.shape[1], x.shape[2]
    K = w.shape[-1]
    y = F.conv1d(x.transpose(1, 2), w.view(C, 1, K), bias, padding=K - 1, groups=C)[..., :T].transpose(1, 2)
    if add is not None:
        y = y + add
    return F.silu(y) if silu else y


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _run(dev, B, T, C, K, silu, has_bias, has_add, x_dtype, out_dtype, strided=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    xs = torch.randn(B, T, 2 * C if strided else C, generator=g)
    w = torch.randn(C, 1, K, generator=g) / K
    bias = torch.randn(C, generator=g) if has_bias else None
    add = torch.randn(B, T, C, generator=g) if has_add else None
    dy = torch.randn(B, T, C, generator=g)
    # quantise the inputs to the dtype the kernel reads, so the reference sees the same values
    xs = xs.to(x_dtype)
    if add is not None:
        add = add.to(x_dtype)

    # reference (float64, CPU)
    xr = xs.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = bias.double().requires_grad_(True) if bias is not None else None
    ar = add.double().requires_grad_(True) if add is not None else None
    yr = _ref(xr[..., :C], wr, br, ar, silu)
    yr.backward(dy.double())

    # HIP
    xg = xs.to(dev).requires_grad_(True)
    wg = w.to(dev).requires_grad_(True)
    bg = bias.to(dev).requires_grad_(True) if bias is not None else None
    ag = add.to(dev).requires_grad_(True) if add is not None else None
    xin = xg[..., :C] if strided else xg
    if strided:
        assert xin.stride(1) == 2 * C  # the view goes to the kernel without a copy
    y = dwconv(xin, wg, bg, add=ag, silu=silu, out_dtype=out_dtype)
    assert y.dtype == out_dtype and y.shape == (B, T, C)
    y.backward(dy.to(dev).to(out_dtype))
    res = {"y": (y, yr), "dx": (xg.grad, xr.grad), "dw": (wg.grad, wr.grad)}
    if bias is not None:
        res["db"] = (bg.grad, br.grad)
    if add is not None:
        res["dadd"] = (ag.grad, ar.grad)
    return res


@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("silu", [False, True])
def test_dwconv_fp32_matches_conv1d(gpu, K, silu):
    res = _run(gpu, B=2, T=150, C=72, K=K, silu=silu, has_bias=True, has_add=not silu,
               x_dtype=torch.float32, out_dtype=torch.float32)
    for name, (a, b) in res.items():
        assert _rel(a, b) < 1e-5, (name, _rel(a, b))


@pytest.mark.parametrize("T", [1, 3, 63, 64, 65, 129])
def test_dwconv_ragged_lengths(gpu, T):
    """T below K, at and around the 64-row block boundary."""
    for silu in (False, True):
        res = _run(gpu, B=3, T=T, C=40, K=4, silu=silu, has_bias=True, has_add=False,
                   x_dtype=torch.float32, out_dtype=torch.float32, seed=T)
        for name, (a, b) in res.items():
            assert _rel(a, b) < 1e-5, (T, silu, name, _rel(a, b))


def test_dwconv_strided_input_no_bias(gpu):
    """x as the first half of a [B, T, 2C] projection, as in the mixer."""
    res = _run(gpu, B=2, T=100, C=300, K=4, silu=True, has_bias=False, has_add=False,
               x_dtype=torch.float32, out_dtype=torch.float32, strided=True)
    for name, (a, b) in res.items():
        assert _rel(a, b) < 1e-5, (name, _rel(a, b))


@pytest.mark.parametrize("silu,out", [(True, torch.bfloat16), (False, torch.float32)])
def test_dwconv_bf16_inputs(gpu, silu, out):
    """bf16 reads, float32 arithmetic, one rounding at a bf16 output."""
    res = _run(gpu, B=2, T=200, C=264, K=4, silu=silu, has_bias=True, has_add=not silu,
               x_dtype=torch.bfloat16, out_dtype=out, strided=silu)
    for name, (a, b) in res.items():
        tol = 2e-3 if name in ("dw", "db") else 8e-3  # bf16 outputs carry one rounding (2^-9 relative)
        assert _rel(a, b) < tol, (name, _rel(a, b))


def test_dwconv_mixer_shape_and_determinism(gpu):
    """The C5 mixer's shape (d_inner 1536, T 2048, k 4): float64 agreement of
    the long dw / dbias sums, and bit-identical repeats."""
    dev = gpu
    B, T, C, K = 2, 2048, 1536, 4
    torch.manual_seed(5)
    x = torch.randn(B, T, C, device=dev, dtype=torch.bfloat16)
    w = (torch.randn(C, 1, K, device=dev) / K).requires_grad_(True)
    b = torch.randn(C, device=dev).requires_grad_(True)
    dy = torch.randn(B, T, C, device=dev, dtype=torch.bfloat16)
    grads = []
    for _ in range(2):
        w.grad = b.grad = None
        y = dwconv(x, w, b, silu=True, out_dtype=torch.bfloat16)
        y.backward(dy)
        grads.append((y.clone(), w.grad.clone(), b.grad.clone()))
    for a, c in zip(grads[0], grads[1]):
        assert torch.equal(a, c)
    wr = w.detach().cpu().double().requires_grad_(True)
    br = b.detach().cpu().double().requires_grad_(True)
    yr = _ref(x.cpu().double(), wr, br, None, True)
    yr.backward(dy.cpu().double())
    assert _rel(grads[0][1], wr.grad) < 1e-5
    assert _rel(grads[0][2], br.grad) < 1e-5
    assert _rel(grads[0][0], yr) < 8e-3


def test_dwconv_empty_batch_zero_grads(gpu):
    w = torch.randn(8, 1, 3, device=gpu, requires_grad=True)
    b = torch.randn(8, device=gpu, requires_grad=True)
    x = torch.zeros(0, 5, 8, device=gpu, requires_grad=True)
    y = dwconv(x, w, b)
    y.sum().backward()
    assert torch.equal(w.grad, torch.zeros_like(w)) and torch.equal(b.grad, torch.zeros_like(b))


@pytest.mark.parametrize("x_dtype,C", [(torch.float32, 72), (torch.bfloat16, 264), (torch.bfloat16, 100)])
def test_dwconv_strided_add(gpu, x_dtype, C):
    """add as one slice of a wider projection output (row stride 3C + 8, as
    the fused gate projection passes it): read in place, same result as a
    contiguous add, gradient of the slice = dy."""
    g = torch.Generator().manual_seed(C)
    B, T, K = 2, 90, 4
    x = torch.randn(B, T, C, generator=g).to(x_dtype)
    w = torch.randn(C, 1, K, generator=g) / K
    bias = torch.randn(C, generator=g)
    wide = torch.randn(B, T, 3 * C + 8, generator=g).to(x_dtype)
    dy = torch.randn(B, T, C, generator=g)
    wg = wide.to(gpu).requires_grad_(True)
    add = wg[..., C:2 * C]
    assert add.stride(1) == 3 * C + 8
    y = dwconv(x.to(gpu), w.to(gpu), bias.to(gpu), add=add, out_dtype=torch.float32)
    y.backward(dy.to(gpu))
    y2 = dwconv(x.to(gpu), w.to(gpu), bias.to(gpu), add=add.detach().contiguous(), out_dtype=torch.float32)
    assert torch.equal(y.detach(), y2)
    yr = _ref(x.double(), w.double(), bias.double(), wide[..., C:2 * C].double(), False)
    assert _rel(y, yr) < 1e-5
    gr = torch.zeros(B, T, 3 * C + 8, dtype=torch.float64)
    gr[..., C:2 * C] = dy.to(x_dtype).double()
    assert _rel(wg.grad, gr) < 1e-6


def test_gradsink_split_matches_plain_split(gpu):
    """Pieces of gradsink.split() whose consumers write their gradients in
    place give the same gradient as autograd's split + concatenation, also
    when a piece has a second consumer (summed gradient: copied in) or none
    (zero-filled)."""
    from naju_amd import gradsink
    from naju_amd.readout import readout
    torch.manual_seed(9)
    B, T, C = 2, 40, 32
    base = torch.randn(B, T, 3 * C + 16, device=gpu).to(torch.bfloat16)
    cx = torch.randn(B, T, C, device=gpu).to(torch.bfloat16)
    h = torch.randn(B, T, C, device=gpu).to(torch.bfloat16)
    w = torch.randn(C, 1, 4, device=gpu) / 4
    bias = torch.randn(C, device=gpu)
    D = torch.randn(C, device=gpu)
    gy = [torch.randn(B, T, C, device=gpu) for _ in range(3)]
    grads = []
    for use_sink in (True, False):
        t = base.clone().requires_grad_(True)
        if use_sink:
            x, z, p, q = gradsink.split(t, [C, C, C, 16])
        else:
            x, z, p, q = t.split([C, C, C, 16], dim=-1)
        y0 = dwconv(x, w, bias, silu=True, out_dtype=torch.float32)
        y1 = readout(cx, h, z, D, 0.5, out_dtype=torch.float32)
        y2 = dwconv(h, w, bias, add=p, out_dtype=torch.float32)
        loss = (y0 * gy[0]).sum() + (y1 * gy[1]).sum() + (y2 * gy[2]).sum() + 0.5 * x.float().sum()
        loss.backward()
        grads.append(t.grad.clone())
    assert torch.equal(grads[0], grads[1])
    assert torch.count_nonzero(grads[0][..., 3 * C:]) == 0


@pytest.mark.parametrize("C,dtype", [(1536, torch.bfloat16), (100, torch.bfloat16), (96, torch.float32)])
def test_bwd_accumulates_dx_in_place(gpu, C, dtype):
    """naju_dwconv_bwd with NAJU_DWCONV_ACCUM_DX adds the gradient to what dx
    holds (one rounding of the sum to dx's dtype): a buffer holding g0 comes
    back as g0 + dx, on the vector path (C a multiple of 8, bf16) and the
    element path, dw and dbias unchanged by the flag."""
    import ctypes
    from naju_amd import _lib
    from naju_amd.dwconv import _DT, _WS
    L = _lib.lib()
    g = torch.Generator(device=gpu).manual_seed(C)
    B, T, K = 2, 300, 4
    x = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)
    w = torch.randn(C, K, generator=g, device=gpu)
    bias = torch.randn(C, generator=g, device=gpu)
    dy = torch.randn(B, T, C, generator=g, device=gpu)
    g0 = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)
    st = torch.cuda.current_stream(gpu).cuda_stream
    ws = _WS.get(gpu, st, L.naju_dwconv_workspace_bytes(B, T, C, K))
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731

    def bwd(dx, act, dw, db):
        _lib.check_mixer(L.naju_dwconv_bwd(p(x), C, p(w), p(bias), p(dy), p(dx), C, p(dw), p(db), None, C, B, T, C,
                                           K, act, _DT[dtype], _DT[torch.float32], _DT[dx.dtype], 0, p(ws),
                                           ws.numel(), st))

    for act in (0, 1):
        # the gradient alone, in float32 (element path)
        ref = torch.empty(B, T, C, dtype=torch.float32, device=gpu)
        dw0, db0 = torch.empty(C, K, device=gpu), torch.empty(C, device=gpu)
        bwd(ref, act, dw0, db0)
        acc = g0.clone()
        dw1, db1 = torch.empty(C, K, device=gpu), torch.empty(C, device=gpu)
        bwd(acc, act | 2, dw1, db1)
        # the same call without the flag (same kernel path): same dw, dbias
        plain = torch.empty_like(g0)
        dw2, db2 = torch.empty(C, K, device=gpu), torch.empty(C, device=gpu)
        bwd(plain, act, dw2, db2)
        torch.cuda.synchronize()
        want = (g0.float() + ref).to(dtype)
        # the vector kernel forms the same gradient up to float32 rounding,
        # so the sum may land one rounding step of dtype apart
        tol = 2.0 ** -7 if dtype == torch.bfloat16 else 1e-6
        assert float(((acc.float() - want.float()).abs() / want.float().abs().clamp_min(1e-3)).max()) <= tol, act
        assert torch.equal(dw1, dw2) and torch.equal(db1, db2)
    with pytest.raises(_lib.NajuScanError, match="act must be"):
        bwd(acc, 4, None, None)


@pytest.mark.parametrize("dtype,T", [(torch.bfloat16, 2048), (torch.bfloat16, 77), (torch.float32, 100)])
def test_gate_pair_matches_two_single_convolutions(gpu, dtype, T):
    """naju_dwconv_pair_fwd / _bwd (the mixer's two gate convolutions over one
    input, adds taken in place from one projection output) against two
    dwconv calls: the logits, dw, dbias and the adds' gradients bitwise; x's
    gradient (both convolutions' transposes summed, one rounding, added to
    what the fan-out buffer holds) against float64."""
    from naju_amd import gradsink
    from naju_amd.dwconv import dwconv, dwconv_pair, pair_supported
    B, C, K = 2, 1536 if T == 2048 else 264, 4
    g = torch.Generator(device=gpu).manual_seed(T)
    x0 = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)
    P0 = torch.randn(B, T, 2 * C + 16, generator=g, device=gpu).to(dtype)
    ws = [torch.randn(C, 1, K, generator=g, device=gpu) / K for _ in range(2)]
    bs = [torch.randn(C, generator=g, device=gpu) for _ in range(2)]
    dys = [torch.randn(B, T, C, generator=g, device=gpu) for _ in range(2)]
    g_prev = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)

    def run(paired):
        x = x0.clone().requires_grad_(True)
        P = P0.clone().requires_grad_(True)
        w = [t.clone().requires_grad_(True) for t in ws]
        b = [t.clone().requires_grad_(True) for t in bs]
        # x feeds the pair and one more consumer (as h in the mixer): its
        # gradient collects in a fan-out buffer that another gradient fills first
        xa, xo = gradsink.fanout(x, 2)
        p0, p1, _ = gradsink.split(P, [C, C, 16])
        if paired:
            assert pair_supported(xa, w[0], p0, w[1], p1)
            y0, y1 = dwconv_pair(xa, w[0], b[0], p0, w[1], b[1], p1, out_dtype=torch.float32)
        else:
            y0 = dwconv(xa, w[0], b[0], add=p0, out_dtype=torch.float32)
            y1 = dwconv(xa, w[1], b[1], add=p1, out_dtype=torch.float32)
        loss = (y0 * dys[0]).sum() + (y1 * dys[1]).sum() + (xo.float() * g_prev.float()).sum()
        loss.backward()
        torch.cuda.synchronize()
        return y0.detach(), y1.detach(), x.grad, P.grad, [t.grad for t in w], [t.grad for t in b]

    y0p, y1p, dxp, dPp, dwp, dbp = run(True)
    y0s, y1s, dxs, dPs, dws, dbs = run(False)
    assert torch.equal(y0p, y0s) and torch.equal(y1p, y1s)
    assert torch.equal(dPp, dPs)
    for a, c in zip(dwp + dbp, dws + dbs):
        assert torch.equal(a, c)
    # x's gradient against float64: g_prev + conv0^T(dy0) + conv1^T(dy1)
    want = g_prev.double()
    for w, dy in zip(ws, dys):
        xr = x0.double().requires_grad_(True)
        yr = F.conv1d(xr.transpose(1, 2), w.double(), padding=K - 1, groups=C)[..., :T].transpose(1, 2)
        want = want + torch.autograd.grad(yr, xr, dy.double())[0]
    tol = 2.0 ** -7 if dtype == torch.bfloat16 else 1e-5
    assert _rel(dxp, want) < tol


@pytest.mark.parametrize("dtype,extra", [(torch.bfloat16, False), (torch.float32, False), (torch.bfloat16, True)])
def test_gate_pair_takes_handed_over_gradients(gpu, dtype, extra):
    """dwconv_pair(..., gate_grads=True): when the logits' consumer hands
    their gradients over (written into the adds' split buffer in its type,
    with their sums; naju_dwconv_pair_bwd reads them there, rows of the
    buffer's stride apart), every gradient is bitwise the ordinary path's
    for gradients of the same values, and the biases' gradients are the
    handed-over sums. With a second consumer of the logits (extra), whose
    gradient autograd adds to the hand-off's markers, the scan's part is
    added back in and the result is bitwise the ordinary path's."""
    from naju_amd import gradsink
    from naju_amd.dwconv import dwconv_pair, pair_supported
    B, T, C, K = 2, 300, 264, 4
    g = torch.Generator(device=gpu).manual_seed(5)
    x0 = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)
    P0 = torch.randn(B, T, 2 * C + 16, generator=g, device=gpu).to(dtype)
    ws = [torch.randn(C, 1, K, generator=g, device=gpu) / K for _ in range(2)]
    bs = [torch.randn(C, generator=g, device=gpu) for _ in range(2)]
    # gradients whose values the split buffer's type holds exactly
    dys = [torch.randn(B, T, C, generator=g, device=gpu).to(dtype).float() for _ in range(2)]
    sums = [d.sum((0, 1)) for d in dys]
    g_prev = torch.randn(B, T, C, generator=g, device=gpu).to(dtype)

    class Consumer(torch.autograd.Function):
        @staticmethod
        def forward(ctx, y0, y1, gg):
            ctx.gg = gg
            return y0.sum() + y1.sum()

        @staticmethod
        def backward(ctx, go):
            if ctx.gg is None:
                return dys[0], dys[1], None
            t0, t1 = ctx.gg.targets()
            t0.copy_(dys[0])
            t1.copy_(dys[1])
            m0, m1 = ctx.gg.hand_over(t0, t1, sums[0], sums[1], dys[0].shape, torch.float32, torch.float32)
            return m0, m1, None

    def run(handoff):
        x = x0.clone().requires_grad_(True)
        P = P0.clone().requires_grad_(True)
        w = [t.clone().requires_grad_(True) for t in ws]
        b = [t.clone().requires_grad_(True) for t in bs]
        xa, xo = gradsink.fanout(x, 2)
        p0, p1, _ = gradsink.split(P, [C, C, 16])
        assert pair_supported(xa, w[0], p0, w[1], p1)
        y0, y1, *gg = dwconv_pair(xa, w[0], b[0], p0, w[1], b[1], p1, out_dtype=torch.float32,
                                  gate_grads=handoff)
        loss = Consumer.apply(y0, y1, gg[0] if gg else None) + (xo.float() * g_prev.float()).sum()
        if extra:
            loss = loss + (y0 * c0).sum() + (y1 * c1).sum()
        loss.backward()
        torch.cuda.synchronize()
        return x.grad, P.grad, [t.grad for t in w], [t.grad for t in b]

    c0, c1 = (torch.randn(B, T, C, generator=g, device=gpu) for _ in range(2))
    dxh, dPh, dwh, dbh = run(True)
    dxp, dPp, dwp, dbp = run(False)
    assert torch.equal(dxh, dxp) and torch.equal(dPh, dPp)
    for a, c in zip(dwh, dwp):
        assert torch.equal(a, c)
    for a, s, c in zip(dbh, sums, dbp):
        if extra:
            assert torch.equal(a, c)
        else:
            assert torch.equal(a, s)
            assert torch.allclose(a, c, rtol=1e-5, atol=1e-5)
