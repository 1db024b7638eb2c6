"""naju_scan_fwd_noalloc: the forward on the library's static device scratch
instead of a caller workspace. Checked through the C ABI against
naju_scan_fwd on the same inputs (y, the checkpoint and hT), on two calls in
a row on one GPU, the second with a smaller input, and its size limit on
the host."""
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
