"""naju_scan_fwd_strided / naju_scan_bwd_strided: B and C read from rows
bc_ld elements apart (column slices of one wider tensor, as the mixer's
projection output holds them) and dB, dC written to rows dbc_ld apart. Every
output must be bitwise the contiguous calls' (naju_scan_fwd / naju_scan_bwd,
pinned against the fp64 oracle by the parity tests), the columns of the
wide gradient buffer outside dB and dC must stay as they were, and the
autograd path that uses the strided calls (B, C from one gradsink.split)
must give the gradients of the plain one bitwise."""
import pytest
import torch

from naju_amd import _lib
from tests._helpers import rand_inputs

pytestmark = pytest.mark.gpu

_DTC = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _p(x):
    return None if x is None else x.data_ptr()


def _abi(t, dev, flags, wide=None):
    """Forward + backward through the C ABI. wide = None: contiguous B, C,
    dB, dC. wide = (ld, boff, coff, dld, dboff, dcoff): B, C at columns boff,
    coff of a [batch, T, ld] tensor, dB, dC at columns dboff, dcoff of a
    [batch, T, dld] one filled with NaN. Returns (outputs, wide grad buffer)."""
    L = _lib.lib()
    u, fl, il, Bm, Cm, h0, dy = t["u"], t["f_logit"], t["i_logit"], t["B"], t["C"], t.get("h0"), t["dy"]
    Dk = t["D_skip"].float().contiguous()
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    dts = (_DTC[u.dtype], _DTC[fl.dtype], _DTC[Bm.dtype])
    out32 = bool(flags & _lib.FLAG_OUT_F32)
    od = lambda x: torch.float32 if out32 else x.dtype  # noqa: E731
    y = torch.empty(u.shape, dtype=od(u), device=dev)
    ck = torch.empty(max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts)), dtype=torch.float32, device=dev)
    nb = L.naju_scan_workspace_bytes_ex(Bsz, T, D, N, *dts, flags)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    g = {"du": torch.empty(u.shape, dtype=od(u), device=dev),
         "dfl": torch.empty(u.shape, dtype=od(fl), device=dev),
         "dil": torch.empty(u.shape, dtype=od(il), device=dev),
         "dD": torch.empty(D, dtype=torch.float32, device=dev)}
    if h0 is not None:
        g["dh0"] = torch.empty(h0.shape, dtype=torch.float32, device=dev)
    gbuf = None
    if wide is None:
        Bx, Cx = Bm, Cm
        g["dB"] = torch.empty(Bm.shape, dtype=od(Bm), device=dev)
        g["dC"] = torch.empty(Bm.shape, dtype=od(Cm), device=dev)
        _lib.check(L.naju_scan_fwd(_p(u), _p(fl), _p(il), _p(Bx), _p(Cx), _p(Dk), _p(h0), _p(y), _p(ck), None,
                                   Bsz, T, D, N, *dts, flags, _p(ws), ws.numel(), st))
        _lib.check(L.naju_scan_bwd(_p(u), _p(fl), _p(il), _p(Bx), _p(Cx), _p(Dk), _p(ck), _p(dy), _p(g["du"]),
                                   _p(g["dfl"]), _p(g["dil"]), _p(g["dB"]), _p(g["dC"]), _p(g["dD"]),
                                   _p(g.get("dh0")), Bsz, T, D, N, *dts, flags, _p(ws), ws.numel(), st))
    else:
        ld, bo, co, dld, dbo, dco = wide
        P = torch.randn(Bsz, T, ld, device=dev).to(Bm.dtype)
        P[..., bo:bo + N] = Bm
        P[..., co:co + N] = Cm
        Bx, Cx = P[..., bo:bo + N], P[..., co:co + N]
        gbuf = torch.full((Bsz, T, dld), float("nan"), dtype=od(Bm), device=dev)
        g["dB"], g["dC"] = gbuf[..., dbo:dbo + N], gbuf[..., dco:dco + N]
        _lib.check(L.naju_scan_fwd_strided(_p(u), _p(fl), _p(il), _p(Bx), _p(Cx), _p(Dk), _p(h0), _p(y), _p(ck),
                                           None, Bsz, T, D, N, ld, *dts, flags, _p(ws), ws.numel(), st))
        _lib.check(L.naju_scan_bwd_strided(_p(u), _p(fl), _p(il), _p(Bx), _p(Cx), _p(Dk), _p(ck), _p(dy),
                                           _p(g["du"]), _p(g["dfl"]), _p(g["dil"]), _p(g["dB"]), _p(g["dC"]),
                                           _p(g["dD"]), _p(g.get("dh0")), Bsz, T, D, N, ld, dld, *dts, flags,
                                           _p(ws), ws.numel(), st))
    torch.cuda.synchronize()
    return dict(y=y, **g), gbuf


CASES = [
    # (batch, T, D, N), dtype, gate dtype, h0_std
    ((2, 300, 96, 16), torch.float32, None, 0.5),
    ((2, 257, 128, 64), torch.bfloat16, torch.float32, 0.0),
    ((1, 190, 70, 24), torch.float16, None, 0.3),
    ((3, 77, 64, 12), torch.bfloat16, None, 0.0),
    ((1, 1100, 192, 64), torch.bfloat16, torch.float32, 0.2),
]
# (name, flags)
FLAGS = [("default", 0), ("out_f32", _lib.FLAG_OUT_F32), ("deterministic", _lib.FLAG_DETERMINISTIC),
         ("ckpt64", _lib.ckpt_rows_flag(64))]


@pytest.mark.parametrize("shape,dtype,gdt,h0_std", CASES)
@pytest.mark.parametrize("fname,flags", FLAGS)
def test_strided_calls_are_bitwise_the_contiguous_ones(shape, dtype, gdt, h0_std, fname, flags):
    dev = torch.device("cuda:0")
    N = shape[3]
    print(f"strided B/C case {shape} {dtype} gates={gdt} {fname}", flush=True)
    ins = rand_inputs(*shape, seed=sum(shape), dtype=dtype, gate_dtype=gdt, h0_std=h0_std)
    t = {k: (v.to(dev).contiguous() if v is not None else None) for k, v in ins.items()}
    ref, _ = _abi(t, dev, flags)
    # the mixer's layout (C right after B, one wide row) and a looser one
    # (C before B, gradient rows of another width)
    for wide in ((2 * N + 40, 40, 40 + N, 2 * N + 40, 40, 40 + N),
                 (3 * N + 8, 2 * N + 8, 4, 2 * N, N, 0)):
        got, gbuf = _abi(t, dev, flags, wide)
        for k in ref:
            assert torch.equal(got[k], ref[k]), (wide, k)
        dbo, dco = wide[4], wide[5]
        rest = torch.ones(gbuf.shape[-1], dtype=torch.bool, device=dev)
        rest[dbo:dbo + N] = False
        rest[dco:dco + N] = False
        assert torch.isnan(gbuf[..., rest]).all(), wide


def _mixer_like(dev, sizes, N, dtype, strided):
    """x_proj output Z [batch, T, W] cut into gate logits and B, C (the
    mixer's split), the scan over them, loss = <y, dy>; returns y and Z's
    gradient. strided=False hands the scan contiguous clones of B and C."""
    from naju_amd import gradsink, naju_scan_hip
    g = torch.Generator().manual_seed(7)
    Bsz, T, D = 2, 333, sizes[0]
    W = sum(sizes)
    Z = (torch.randn(Bsz, T, W, generator=g) * 0.3).to(dtype).to(dev).requires_grad_(True)
    u = torch.randn(Bsz, T, D, generator=g).to(dtype).to(dev)
    dy = torch.randn(Bsz, T, D, generator=g).to(dtype).to(dev)
    Dk = torch.zeros(D, device=dev)
    p_f, p_i, Bm, Cm = gradsink.split(Z, sizes)
    if not strided:
        Bm, Cm = Bm.clone(memory_format=torch.contiguous_format), Cm.clone(memory_format=torch.contiguous_format)
    y = naju_scan_hip(u, p_f.float() + 3.0, p_i.float() - 2.0, Bm, Cm, Dk)
    y.backward(dy)
    torch.cuda.synchronize()
    return y.detach(), Z.grad


@pytest.mark.parametrize("N,dtype", [(64, torch.bfloat16), (16, torch.float32)])
def test_autograd_split_path_is_bitwise_the_plain_one(N, dtype):
    dev = torch.device("cuda:0")
    sizes = [96, 96, N, N]
    y0, g0 = _mixer_like(dev, sizes, N, dtype, False)
    y1, g1 = _mixer_like(dev, sizes, N, dtype, True)
    assert torch.equal(y1, y0)
    assert torch.equal(g1, g0)


@pytest.mark.parametrize("shape,dtype,gdt,dgt", [
    ((2, 300, 96, 16), torch.bfloat16, torch.float32, torch.bfloat16),   # the mixer's: f32 gates, bf16 buffer
    ((1, 1100, 192, 64), torch.bfloat16, torch.float32, torch.bfloat16),
    ((2, 257, 128, 64), torch.float32, None, torch.float32),              # float32 model: f32 buffer
    ((3, 77, 72, 12), torch.float16, torch.float32, torch.float16),
])
def test_gate_gradient_layout_and_sums(shape, dtype, gdt, dgt):
    """naju_scan_bwd_ex with the gate-gradient options: dfl and dil written
    into a wider buffer (row stride ld) in dg_dtype are torch's rounding of
    naju_scan_bwd's float32 dfl, dil (bitwise); every other output is
    bitwise naju_scan_bwd's; the sums over batch and time match float64 sums
    of those float32 gradients; the buffer's other columns stay untouched."""
    from naju_amd import _lib
    dev = torch.device("cuda:0")
    print(f"gate-gradient layout case {shape} {dtype} gates={gdt} -> {dgt}", flush=True)
    Bsz, T, D, N = shape
    ins = rand_inputs(*shape, seed=sum(shape) + 1, dtype=dtype, gate_dtype=gdt, h0_std=0.3)
    t = {k: (v.to(dev).contiguous() if v is not None else None) for k, v in ins.items()}
    flags = _lib.FLAG_OUT_F32
    ref, _ = _abi(t, dev, flags)  # float32 outputs
    L = _lib.lib()
    u, fl, il, Bm, Cm, h0, dy = t["u"], t["f_logit"], t["i_logit"], t["B"], t["C"], t.get("h0"), t["dy"]
    Dk = t["D_skip"].float().contiguous()
    dts = (_DTC[u.dtype], _DTC[fl.dtype], _DTC[Bm.dtype])
    ck = torch.empty(max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts)), dtype=torch.float32, device=dev)
    nb = L.naju_scan_workspace_bytes_ex(Bsz, T, D, N, *dts, flags)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    y = torch.empty(u.shape, dtype=torch.float32, device=dev)
    _lib.check(L.naju_scan_fwd(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(h0), _p(y), _p(ck), None,
                               Bsz, T, D, N, *dts, flags, _p(ws), ws.numel(), st))
    ld = 2 * D + 40
    buf = torch.full((Bsz, T, ld), float("nan"), dtype=dgt, device=dev)
    dfl, dil = buf[..., 8:8 + D], buf[..., D + 40:2 * D + 40]
    g = {k: torch.empty(u.shape, dtype=torch.float32, device=dev) for k in ("du",)}
    g["dB"] = torch.empty(Bm.shape, dtype=torch.float32, device=dev)
    g["dC"] = torch.empty(Bm.shape, dtype=torch.float32, device=dev)
    g["dD"] = torch.empty(D, dtype=torch.float32, device=dev)
    g["dh0"] = torch.empty(h0.shape, dtype=torch.float32, device=dev)
    sums = torch.full((2, D), float("nan"), device=dev)
    lay = _lib.ScanBwdLayout(dg_ld=ld, dg_dtype=_DTC[dgt], dfl_sum=sums.data_ptr(), dil_sum=sums.data_ptr() + 4 * D)
    import ctypes
    _lib.check(L.naju_scan_bwd_ex(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(ck), _p(dy), _p(g["du"]),
                                  _p(dfl), _p(dil), _p(g["dB"]), _p(g["dC"]), _p(g["dD"]), _p(g["dh0"]),
                                  Bsz, T, D, N, *dts, flags, ctypes.byref(lay), _p(ws), ws.numel(), st))
    torch.cuda.synchronize()
    for k in g:
        assert torch.equal(g[k], ref[k]), k
    assert torch.equal(dfl, ref["dfl"].to(dgt)) and torch.equal(dil, ref["dil"].to(dgt))
    rest = torch.ones(ld, dtype=torch.bool, device=dev)
    rest[8:8 + D] = False
    rest[D + 40:2 * D + 40] = False
    assert torch.isnan(buf[..., rest]).all()
    for s, k in ((sums[0], "dfl"), (sums[1], "dil")):
        want = ref[k].double().sum((0, 1))
        scale = ref[k].double().abs().sum((0, 1)) + 1e-30
        assert float(((s.double() - want).abs() / scale).max()) < 1e-5, k
