"""naju_scan_fwd_noalloc: the forward on the library's static device scratch
instead of a caller workspace. Checked through the C ABI against
naju_scan_fwd on the same inputs (y, the checkpoint and hT), on two calls in
a row on one GPU, the second with a smaller input; with a memory-light
checkpoint interval feeding naju_scan_bwd; recorded into a HIP graph and
replayed; its status word (naju_scan_noalloc_status) after forced hand-off
failures; and its size limit on the host."""
import ctypes

import numpy as np
import pytest
import torch

from tests._helpers import _DTC, rand_inputs, tol_for


def _p(x):
    return None if x is None else x.data_ptr()


def _fwd_both(ins, dev, flags):
    """(y, ckpt, hT) from naju_scan_fwd with a fresh workspace and from
    naju_scan_fwd_noalloc."""
    from naju_amd import _lib
    L = _lib.lib()
    t = {k: (v.to(dev).contiguous() if v is not None else None) for k, v in ins.items()}
    u, fl, il, Bm, Cm = t["u"], t["f_logit"], t["i_logit"], t["B"], t["C"]
    Dk, h0 = t["D_skip"].float().contiguous(), t.get("h0")
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    dts = (_DTC[u.dtype], _DTC[fl.dtype], _DTC[Bm.dtype])
    nck = max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts))
    st = torch.cuda.current_stream(dev).cuda_stream
    outs = []
    for noalloc in (False, True):
        y = torch.full(u.shape, float("nan"), dtype=torch.float32 if flags & _lib.FLAG_OUT_F32 else u.dtype,
                       device=dev)
        ck = torch.full((nck,), float("nan"), dtype=torch.float32, device=dev)
        hT = torch.full((Bsz, D, N), float("nan"), dtype=torch.float32, device=dev)
        if noalloc:
            rc = L.naju_scan_fwd_noalloc(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(h0), _p(y), _p(ck),
                                         _p(hT), Bsz, T, D, N, *dts, flags, st)
        else:
            nb = L.naju_scan_workspace_bytes(Bsz, T, D, N, *dts)
            ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
            rc = L.naju_scan_fwd(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(h0), _p(y), _p(ck), _p(hT),
                                 Bsz, T, D, N, *dts, flags, _p(ws), ws.numel(), st)
        _lib.check(rc)
        torch.cuda.synchronize()
        outs.append((y, ck, hT))
    return outs


def _close(name, a, b, dtype):
    a64, b64 = a.double().cpu().numpy(), b.double().cpu().numpy()
    assert np.all(np.isfinite(a64)), f"{name}: non-finite output"
    err = np.abs(a64 - b64).max() / max(np.abs(b64).max(), 1e-30)
    assert err <= tol_for(dtype)[0], f"{name}: rel err {err:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("N,first,second,dtype", [
    (1, (8, 4096, 1024), (2, 700, 320), torch.bfloat16),
    (1, (2, 1000, 256), (1, 37, 64), torch.float32),
    (64, (8, 1024, 1024), (2, 300, 96), torch.float32),
    (16, (8, 200, 6144), (1, 100, 64), torch.bfloat16),
])
def test_noalloc_matches_workspace_forward(gpu, N, first, second, dtype):
    """Two calls in a row, the second smaller: every output of the
    allocation-free forward equals naju_scan_fwd's (bit for bit with fixed-order
    carries; the general-N call at N = 64 may use fewer time segments to fit
    its scratch, so it is compared at the float32 tolerance)."""
    from naju_amd import _lib
    for i, shape in enumerate((first, second)):
        ins = rand_inputs(*shape, N, seed=31 + i + N, dtype=dtype, h0_std=0.3)
        for flags in (_lib.FLAG_DETERMINISTIC, _lib.FLAG_OUT_F32):
            (y0, c0, h0), (y1, c1, h1) = _fwd_both(ins, gpu, flags)
            if flags & _lib.FLAG_DETERMINISTIC and N != 64:
                assert torch.equal(y0, y1), f"call {i}: y differs"
                assert torch.equal(c0, c1), f"call {i}: ckpt differs"
                assert torch.equal(h0, h1), f"call {i}: hT differs"
            else:
                _close(f"call {i} y", y1, y0, y0.dtype)
                _close(f"call {i} ckpt", c1, c0, torch.float32)
                _close(f"call {i} hT", h1, h0, torch.float32)


@pytest.mark.gpu
def test_noalloc_status_stays_clean_and_repeats(gpu):
    """Repeated calls on the shared scratch leave no state behind: the same
    inputs give the same outputs every time (fixed-order carries)."""
    from naju_amd import _lib
    ins = rand_inputs(4, 2000, 512, 1, seed=5, h0_std=0.2)
    first = None
    for _ in range(5):
        (_, _, _), (y, ck, hT) = _fwd_both(ins, gpu, _lib.FLAG_DETERMINISTIC)
        if first is None:
            first = (y.clone(), ck.clone(), hT.clone())
        else:
            assert torch.equal(y, first[0]) and torch.equal(ck, first[1]) and torch.equal(hT, first[2])


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """The size check runs on the host, before any device work (no GPU
    needed): at N = 1 the forward's hand-off words of benchmark configuration
    c4 (32 x 8192 x 4096) far exceed the static scratch."""
    from naju_amd import _lib
    L = _lib.lib()
    rc = L.naju_scan_fwd_noalloc(*([None] * 10), 32, 8192, 4096, 1, 1, 1, 1, 0, None)
    assert rc == _lib.ERR_WORKSPACE
    msg = L.naju_scan_last_error().decode()
    assert "static maximum" in msg and str(32 << 20) in msg
    rc = L.naju_scan_fwd_noalloc(*([None] * 10), 2, 16, 8, 0, 0, 0, 0, 0, None)
    assert rc == _lib.ERR_INVALID


def _noalloc_fwd_bwd(t, dev, flags, out_f32=True):
    """naju_scan_fwd_noalloc, then naju_scan_bwd on its checkpoint (same
    flags, so the same checkpoint interval). Returns y and the gradients."""
    from naju_amd import _lib
    L = _lib.lib()
    u, fl, il, Bm, Cm = t["u"], t["f_logit"], t["i_logit"], t["B"], t["C"]
    Dk, h0, dy = t["D_skip"], t.get("h0"), t["dy"]
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    dts = (_DTC[u.dtype], _DTC[fl.dtype], _DTC[Bm.dtype])
    flags |= _lib.FLAG_OUT_F32 if out_f32 else 0
    nck = L.naju_scan_ckpt_elems_ex(Bsz, T, D, N, *dts, flags)
    assert nck > 0, L.naju_scan_last_error()
    st = torch.cuda.current_stream(dev).cuda_stream
    f32 = dict(dtype=torch.float32, device=dev)
    y = torch.full(u.shape, float("nan"), **f32)
    ck = torch.full((nck,), float("nan"), **f32)
    _lib.check(L.naju_scan_fwd_noalloc(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(h0), _p(y), _p(ck), None,
                                       Bsz, T, D, N, *dts, flags, st))
    g = {k: torch.full(u.shape, float("nan"), **f32) for k in ("du", "dfl", "dil")}
    g.update({k: torch.full(Bm.shape, float("nan"), **f32) for k in ("dB", "dC")})
    g["dD"] = torch.full((D,), float("nan"), **f32)
    g["dh0"] = torch.full((Bsz, D, N), float("nan"), **f32) if h0 is not None else None
    nb = L.naju_scan_workspace_bytes_ex(Bsz, T, D, N, *dts, flags)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=dev)
    _lib.check(L.naju_scan_bwd(_p(u), _p(fl), _p(il), _p(Bm), _p(Cm), _p(Dk), _p(ck), _p(dy), _p(g["du"]),
                               _p(g["dfl"]), _p(g["dil"]), _p(g["dB"]), _p(g["dC"]), _p(g["dD"]), _p(g["dh0"]),
                               Bsz, T, D, N, *dts, flags, _p(ws), ws.numel(), st))
    torch.cuda.synchronize()
    return y, g


@pytest.mark.gpu
@pytest.mark.parametrize("shape,dtype,rows", [
    # the scratch holds no time segments here (one forward segment instead of
    # the two naju_scan_fwd takes)
    ((8, 1024, 4096, 64), torch.bfloat16, 32),
    ((2, 1000, 320, 48), torch.float32, 64),
    ((2, 700, 96, 16), torch.float16, 128),
])
def test_noalloc_checkpoint_interval_feeds_the_backward(gpu, shape, dtype, rows):
    """A memory-light checkpoint written by the allocation-free forward: the
    backward's recompute from it gives bitwise the outputs of the default
    interval (both forwards on the scratch take the same segmentation,
    whatever the interval), and those match the fp64 oracle's tolerance
    against naju_scan_fwd's."""
    from naju_amd import _lib
    print(f"noalloc interval case {shape} {dtype} rows={rows}", flush=True)
    ins = rand_inputs(*shape, seed=sum(shape) + rows, dtype=dtype, h0_std=0.2)
    t = {k: (v.to(gpu).contiguous() if v is not None else None) for k, v in ins.items()}
    t["D_skip"] = t["D_skip"].float()
    y0, g0 = _noalloc_fwd_bwd(t, gpu, 0)
    y1, g1 = _noalloc_fwd_bwd(t, gpu, _lib.ckpt_rows_flag(rows))
    assert torch.equal(y1, y0), "y differs between the intervals"
    for k in g0:
        if g0[k] is not None:
            assert torch.equal(g1[k], g0[k]), f"{k} differs between the intervals"
    # against the workspace forward (whose segmentation may differ)
    from tests._helpers import run_abi
    yr, gr = run_abi(ins, gpu, out_f32=True)
    _close("y", y0, yr, torch.float32)
    for k in gr:
        _close(k, g0[k], gr[k], torch.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("N,shape,dtype", [(1, (2, 1000, 256), torch.bfloat16), (16, (2, 300, 128), torch.float32)])
def test_noalloc_graph_capture_replays(gpu, N, shape, dtype):
    """naju_scan_fwd_noalloc recorded into a HIP graph (after an eager call,
    which sets up the device's scratch) and replayed back to back on new
    inputs copied into the captured buffers: every replay equals an eager
    naju_scan_fwd with a workspace on its own inputs, bit for bit
    (fixed-order carries)."""
    from naju_amd import _lib
    L = _lib.lib()
    ins0 = rand_inputs(*shape, N, seed=90 + N, dtype=dtype, h0_std=0.2)
    t = {k: (v.to(gpu).contiguous() if v is not None else None) for k, v in ins0.items()}
    t["D_skip"] = t["D_skip"].float()
    Bsz, T, D = t["u"].shape
    dts = (_DTC[t["u"].dtype], _DTC[t["f_logit"].dtype], _DTC[t["B"].dtype])
    flags = _lib.FLAG_DETERMINISTIC
    y = torch.empty_like(t["u"])
    ck = torch.empty(max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts)), dtype=torch.float32, device=gpu)
    hT = torch.empty((Bsz, D, N), dtype=torch.float32, device=gpu)

    def call():
        st = torch.cuda.current_stream(gpu).cuda_stream
        _lib.check(L.naju_scan_fwd_noalloc(_p(t["u"]), _p(t["f_logit"]), _p(t["i_logit"]), _p(t["B"]), _p(t["C"]),
                                           _p(t["D_skip"]), _p(t["h0"]), _p(y), _p(ck), _p(hT), Bsz, T, D, N, *dts,
                                           flags, st))

    s = torch.cuda.Stream(gpu)
    with torch.cuda.stream(s):
        call()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call()
    torch.cuda.synchronize()
    for rep in range(4):
        ins = rand_inputs(*shape, N, seed=200 * rep + N, dtype=dtype, h0_std=0.2)
        for k in ("u", "f_logit", "i_logit", "B", "C", "D_skip", "h0"):
            t[k].copy_(ins[k].to(gpu))
        for o in (y, ck, hT):
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        (y_ref, ck_ref, hT_ref), _ = _fwd_both(ins, gpu, flags)
        assert torch.equal(y, y_ref), f"replay {rep}: y differs from an eager call on its inputs"
        assert torch.equal(ck, ck_ref), f"replay {rep}: ckpt differs"
        assert torch.equal(hT, hT_ref), f"replay {rep}: hT differs"
    st = ctypes.c_uint32(7)
    _lib.check(L.naju_scan_noalloc_status(torch.cuda.current_stream(gpu).cuda_stream, ctypes.byref(st)))
    assert st.value == 0


@pytest.mark.gpu
def test_noalloc_status_reports_a_failed_handoff_and_clears(gpu, monkeypatch):
    """With every carry hand-off forced to give up at once (the library's
    NAJU_DEBUG_SPIN_LIMIT=0 test hook; every kernel still exits normally),
    the scratch's status word reads 1 through naju_scan_noalloc_status, which
    clears it and rewinds the scratch's ticket counters: the next call is
    correct again."""
    from naju_amd import _lib
    L = _lib.lib()
    ins = rand_inputs(2, 4096, 256, 1, seed=17, dtype=torch.float32, h0_std=0.2)
    stream = torch.cuda.current_stream(gpu).cuda_stream
    st = ctypes.c_uint32(7)
    _lib.check(L.naju_scan_noalloc_status(stream, ctypes.byref(st)))
    assert st.value == 0
    monkeypatch.setenv("NAJU_DEBUG_SPIN_LIMIT", "0")
    (_, _, _), (y_bad, _, _) = _fwd_both(ins, gpu, _lib.FLAG_DETERMINISTIC)
    monkeypatch.delenv("NAJU_DEBUG_SPIN_LIMIT")
    assert bool(torch.isnan(y_bad[:, 128:]).all()), "chunks past the first must carry NaN"
    assert bool(torch.isfinite(y_bad[:, :128]).all()), "the first chunk needs no hand-off"
    _lib.check(L.naju_scan_noalloc_status(stream, ctypes.byref(st)))
    assert st.value == 1
    _lib.check(L.naju_scan_noalloc_status(stream, ctypes.byref(st)))
    assert st.value == 0
    (y0, c0, h0), (y1, c1, h1) = _fwd_both(ins, gpu, _lib.FLAG_DETERMINISTIC)
    assert torch.equal(y0, y1) and torch.equal(c0, c1) and torch.equal(h0, h1)
    _lib.check(L.naju_scan_noalloc_status(stream, ctypes.byref(st)))
    assert st.value == 0
