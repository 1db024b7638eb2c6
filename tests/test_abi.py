"""CPU tests of the C ABI boundary and of the host-side Python mirror.

No GPU is touched: every call here either only queries sizes or fails the
host-side argument checks (which run before any device work), or returns
before launching (empty batch / channel axes).
"""
import ctypes
import os
import re
import types

import pytest
import torch

from naju_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("naju_scan.h", "naju_mixer.h", "naju_loss.h", "naju_optim.h")]
F32, BF16, F16 = 0, 1, 2


def header_functions():
    names = set()
    for h in HEADERS:
        txt = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(naju_\w+)\s*\(", txt))
    return sorted(names)


def test_library_exports_every_header_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert len(names) >= 21
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"
    assert set(names) == set(_lib.EXPORTED)
    assert lib.naju_scan_version() >= 1


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", os.path.join(ROOT, "no_such_lib.so"))
    with pytest.raises(RuntimeError, match="missing"):
        _lib.lib()


def test_size_queries():
    L = _lib.lib()
    # benchmark configuration c2 at N=1: ckpt = one float per (b, chunk, d)
    n = L.naju_scan_ckpt_elems(8, 4096, 1024, 1, BF16, BF16, BF16)
    assert n > 0 and n % (8 * 1024) == 0 and n <= 8 * 1024 * 4096
    ws = L.naju_scan_workspace_bytes(8, 4096, 1024, 1, BF16, BF16, BF16)
    assert ws > 0 and ws % 256 == 0
    # general N: one float per (b, sub-block, d, n); the chunked kernels
    # (9 <= N <= 64) keep the state entering every 16-row sub-block, the
    # others every 32 rows
    n64 = L.naju_scan_ckpt_elems(8, 4096, 1024, 64, BF16, F32, BF16)
    assert n64 == 8 * (4096 // 16) * 1024 * 64
    n8 = L.naju_scan_ckpt_elems(8, 4096, 1024, 8, BF16, F32, BF16)
    assert n8 == 8 * (4096 // 32) * 1024 * 8
    # invalid requests report 0 / -1 and set the message
    assert L.naju_scan_workspace_bytes(8, 4096, 1024, 0, BF16, BF16, BF16) == 0
    assert b"N" in L.naju_scan_last_error()
    assert L.naju_scan_ckpt_elems(-1, 4, 4, 1, F32, F32, F32) == -1


def _fwd(L, **kw):
    a = dict(u=1, fl=1, il=1, B=1, C=1, Dk=1, h0=None, y=1, ck=None, hT=None, batch=2, T=8, D=16, N=1,
             x=F32, g=F32, bc=F32, of=0, ws=None, wsb=0, st=None)
    a.update(kw)
    return L.naju_scan_fwd(a["u"], a["fl"], a["il"], a["B"], a["C"], a["Dk"], a["h0"], a["y"], a["ck"], a["hT"],
                           a["batch"], a["T"], a["D"], a["N"], a["x"], a["g"], a["bc"], a["of"], a["ws"],
                           a["wsb"], a["st"])


def _bwd(L, **kw):
    a = dict(u=1, fl=1, il=1, B=1, C=1, Dk=1, ck=1, dy=1, du=None, dfl=None, dil=None, dB=None, dC=None, dD=None,
             dh0=None, batch=2, T=8, D=16, N=1, x=F32, g=F32, bc=F32, of=0, ws=None, wsb=0, st=None)
    a.update(kw)
    return L.naju_scan_bwd(a["u"], a["fl"], a["il"], a["B"], a["C"], a["Dk"], a["ck"], a["dy"], a["du"],
                           a["dfl"], a["dil"], a["dB"], a["dC"], a["dD"], a["dh0"], a["batch"], a["T"], a["D"],
                           a["N"], a["x"], a["g"], a["bc"], a["of"], a["ws"], a["wsb"], a["st"])


@pytest.mark.parametrize("kw,code,msg", [
    (dict(batch=-1), _lib.ERR_INVALID, "negative"),
    (dict(N=0), _lib.ERR_INVALID, "N"),
    (dict(x=7), _lib.ERR_INVALID, "dtype"),
    (dict(x=BF16, g=F16), _lib.ERR_UNSUPPORTED, "gate"),
    (dict(x=F32, g=BF16), _lib.ERR_UNSUPPORTED, "gate"),
    (dict(x=BF16, g=BF16, bc=F16), _lib.ERR_UNSUPPORTED, "B/C"),
    (dict(N=129), _lib.ERR_UNSUPPORTED, "N"),
    (dict(u=None), _lib.ERR_INVALID, "null"),
    (dict(y=None), _lib.ERR_INVALID, "null"),
    (dict(ws=None), _lib.ERR_WORKSPACE, "workspace"),
    (dict(ws=256, wsb=16), _lib.ERR_WORKSPACE, "workspace"),
    (dict(N=2, D=1 << 25), _lib.ERR_UNSUPPORTED, "2^25"),
])
def test_fwd_argument_checks(kw, code, msg):
    L = _lib.lib()
    assert _fwd(L, **kw) == code
    assert msg.encode() in L.naju_scan_last_error()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(ck=None), _lib.ERR_INVALID, "ckpt"),
    (dict(dy=None), _lib.ERR_INVALID, "null"),
    (dict(T=-3), _lib.ERR_INVALID, "negative"),
    (dict(ws=None), _lib.ERR_WORKSPACE, "workspace"),
    (dict(N=2, D=1 << 25), _lib.ERR_UNSUPPORTED, "2^25"),
])
def test_bwd_argument_checks(kw, code, msg):
    L = _lib.lib()
    assert _bwd(L, **kw) == code
    assert msg.encode() in L.naju_scan_last_error()


def test_misaligned_workspace_rejected():
    L = _lib.lib()
    need = L.naju_scan_workspace_bytes(2, 8, 16, 1, F32, F32, F32)
    assert _fwd(L, ws=256 + 8, wsb=need + 64) == _lib.ERR_WORKSPACE
    assert b"aligned" in L.naju_scan_last_error()


def test_empty_axes_return_without_work():
    L = _lib.lib()
    assert _fwd(L, batch=0, u=None, y=None) == _lib.OK
    assert _fwd(L, D=0, u=None, y=None) == _lib.OK
    # T == 0 with no final-state output: nothing to write
    assert _fwd(L, T=0) == _lib.OK
    assert L.naju_scan_last_error() == b""


def test_check_raises_with_message():
    L = _lib.lib()
    _fwd(L, N=0)
    with pytest.raises(_lib.NajuScanError, match="d_state"):
        _lib.check(_lib.ERR_INVALID)


# ------------------------------------------------------- Python mirror

def test_resolve_backend_order(monkeypatch):
    """explicit > NAJU_SCAN_BACKEND > "hip" with a GPU, "reference" without
    (naju/scan.py:48-52)."""
    from naju_amd import scan
    monkeypatch.delenv("NAJU_SCAN_BACKEND", raising=False)
    monkeypatch.setattr(scan.torch.cuda, "is_available", lambda: True)
    assert scan.resolve_backend() == "hip"
    monkeypatch.setattr(scan.torch.cuda, "is_available", lambda: False)
    assert scan.resolve_backend() == "reference"
    monkeypatch.setenv("NAJU_SCAN_BACKEND", "HIP")
    assert scan.resolve_backend() == "hip"
    assert scan.resolve_backend("Other") == "other"


def test_cpu_default_backend_raises_clearly(monkeypatch):
    """No CPU scan ships with the package: the CPU default names what to
    register instead of falling back to anything."""
    from naju_amd import scan
    monkeypatch.delenv("NAJU_SCAN_BACKEND", raising=False)
    monkeypatch.setattr(scan.torch.cuda, "is_available", lambda: False)
    monkeypatch.setattr(scan, "_BACKEND_CACHE", {})
    x = torch.zeros(1, 2, 3)
    with pytest.raises(ValueError, match="no CPU scan backend"):
        scan.naju_scan(x, x, x, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1), torch.zeros(3))
    scan._BACKEND_CACHE["reference"] = lambda *a: "registered"
    assert scan.naju_scan(x, x, x, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1), torch.zeros(3)) == "registered"


def test_unknown_backend_raises():
    from naju_amd.scan import naju_scan
    x = torch.zeros(1, 2, 3)
    with pytest.raises(ValueError, match="unknown scan backend"):
        naju_scan(x, x, x, torch.zeros(1, 2, 1), torch.zeros(1, 2, 1), torch.zeros(3), backend="chunk")


def test_register_inserts_into_dispatch_cache():
    from naju_amd import naju_scan_hip, register
    fake = types.SimpleNamespace(_BACKEND_CACHE={})
    assert register("HIP", scan_module=fake) is naju_scan_hip
    assert fake._BACKEND_CACHE["hip"] is naju_scan_hip
    register("chunk", scan_module=fake)
    assert fake._BACKEND_CACHE["chunk"] is naju_scan_hip


@pytest.mark.parametrize("bad,msg", [
    (dict(u=torch.zeros(2, 3)), r"\[B, T, D\]"),
    (dict(f_logit=torch.zeros(2, 3, 5)), "f_logit"),
    (dict(B=torch.zeros(2, 4, 1)), "B and C"),
    (dict(D_skip=torch.zeros(3)), "D_skip"),
    (dict(h0=torch.zeros(2, 4, 2)), "h0"),
    ({}, "GPU"),
])
def test_shape_and_device_checks(bad, msg):
    from naju_amd import naju_scan_hip
    a = dict(u=torch.zeros(2, 3, 4), f_logit=torch.zeros(2, 3, 4), i_logit=torch.zeros(2, 3, 4),
             B=torch.zeros(2, 3, 1), C=torch.zeros(2, 3, 1), D_skip=torch.zeros(4), h0=None)
    a.update(bad)
    with pytest.raises(ValueError, match=msg):
        naju_scan_hip(a["u"], a["f_logit"], a["i_logit"], a["B"], a["C"], a["D_skip"], a["h0"])


def test_algorithmic_bytes_headline():
    """22 B per element at bf16 (fwd 8 + bwd 14) plus B/C and h0 terms."""
    from naju_amd.workloads import algorithmic_bytes
    E = 8 * 4096 * 1024
    tot = algorithmic_bytes(8, 4096, 1024, 1, 2, 2, 2, False)
    assert tot == 22 * E + 6 * 2 * 8 * 4096
    with_h0 = algorithmic_bytes(8, 4096, 1024, 1, 2, 2, 2, True)
    assert with_h0 - tot == 12 * 8 * 1024


def test_build_flags_disable_packed_fp32():
    from naju_amd import build
    flags = " ".join(build.HIPCC_FLAGS)
    assert "--offload-arch=gfx950" in flags
    assert "-target-feature -Xclang -packed-fp32-ops" in flags


# --- include/naju_mixer.h: host-side checks of the depthwise conv calls ----

def _dw_fwd(L, K=4, act=0, x_ld=16, add=None, add_ld=16, C=16, batch=2, T=8, dts=(F32, F32, F32)):
    fake = 0x1000  # never dereferenced: every case here returns before a launch
    return L.naju_dwconv_fwd(fake, x_ld, fake, None, add, add_ld, fake, batch, T, C, K, act, dts[0], dts[1], dts[2],
                             None)


def test_dwconv_host_checks():
    L = _lib.lib()
    assert _dw_fwd(L, K=9) == _lib.ERR_UNSUPPORTED and b"K" in L.naju_mixer_last_error()
    assert _dw_fwd(L, K=0) == _lib.ERR_UNSUPPORTED
    assert _dw_fwd(L, x_ld=15) == _lib.ERR_INVALID and b"x_ld" in L.naju_mixer_last_error()
    assert _dw_fwd(L, act=2) == _lib.ERR_INVALID
    assert _dw_fwd(L, act=1, add=0x2000) == _lib.ERR_UNSUPPORTED
    assert _dw_fwd(L, add=0x2000, add_ld=15) == _lib.ERR_INVALID and b"add_ld" in L.naju_mixer_last_error()
    assert _dw_fwd(L, dts=(F32, F32, 7)) == _lib.ERR_INVALID
    assert _dw_fwd(L, batch=-1) == _lib.ERR_INVALID
    # empty shapes return before any launch
    assert _dw_fwd(L, batch=0) == _lib.OK and L.naju_mixer_last_error() == b""
    assert _dw_fwd(L, T=0) == _lib.OK
    # null required pointer
    assert L.naju_dwconv_fwd(None, 16, 0x1000, None, None, 16, 0x1000, 2, 8, 16, 4, 0, F32, F32, F32, None) \
        == _lib.ERR_INVALID


def test_dwconv_workspace_size_and_check():
    L = _lib.lib()
    # one partial row of (K dw + 1 dbias) floats per channel per 64-row block per batch row
    assert L.naju_dwconv_workspace_bytes(8, 2048, 1536, 4) >= 8 * 32 * 1536 * 5 * 4
    assert L.naju_dwconv_workspace_bytes(1, 65, 8, 4) >= 2 * 8 * 5 * 4
    assert L.naju_dwconv_workspace_bytes(1, 8, 8, 9) == 0
    fake = 0x1000
    def bwd(dx_ld=16, dw=fake, dadd=None, dadd_ld=16, batch=2, act=0):
        return L.naju_dwconv_bwd(fake, 16, fake, None, fake, fake, dx_ld, dw, None, dadd, dadd_ld, batch, 8, 16, 4,
                                 act, F32, F32, F32, BF16, None, 0, None)
    assert bwd() == _lib.ERR_WORKSPACE and b"workspace" in L.naju_mixer_last_error()
    assert bwd(dx_ld=15) == _lib.ERR_INVALID and b"dx_ld" in L.naju_mixer_last_error()
    assert bwd(dadd=fake, dadd_ld=12) == _lib.ERR_INVALID and b"dadd_ld" in L.naju_mixer_last_error()
    assert bwd(dadd=fake, act=1) == _lib.ERR_UNSUPPORTED
    # dx only: no sums, no workspace needed -- but it would launch, so check only the no-op case
    assert bwd(dw=None, batch=0) == _lib.OK


def test_dwconv_python_rejects_cpu_tensors():
    from naju_amd.dwconv import dwconv
    with pytest.raises(RuntimeError, match="CUDA"):
        dwconv(torch.zeros(1, 4, 4), torch.zeros(4, 1, 4))


def test_readout_host_checks():
    L = _lib.lib()
    fake = 0x1000
    def fwd(z_ld=16, dts=(F32, F32, F32, F32), rows=4, C=16, y=fake):
        return L.naju_readout_fwd(fake, fake, fake, z_ld, fake, 0.125, y, rows, C, *dts, None)
    assert fwd(z_ld=15) == _lib.ERR_INVALID and b"z_ld" in L.naju_mixer_last_error()
    assert fwd(dts=(F32, F32, 9, F32)) == _lib.ERR_INVALID
    assert fwd(rows=-1) == _lib.ERR_INVALID
    assert fwd(rows=64 * 65535 + 1) == _lib.ERR_UNSUPPORTED
    assert fwd(y=None) == _lib.ERR_INVALID
    assert fwd(rows=0) == _lib.OK and L.naju_mixer_last_error() == b""
    assert L.naju_readout_workspace_bytes(16384, 1536) >= 256 * 1536 * 4
    rc = L.naju_readout_bwd(fake, fake, fake, 16, fake, 0.125, fake, None, None, None, 16, fake, 4, 16,
                            *([F32] * 7), None, 0, None)
    assert rc == _lib.ERR_WORKSPACE
    rc = L.naju_readout_bwd(None, fake, fake, 16, fake, 0.125, fake, None, None, fake, 16, None, 4, 16,
                            *([F32] * 7), None, 0, None)
    assert rc == _lib.ERR_INVALID and b"cx" in L.naju_mixer_last_error()
    rc = L.naju_readout_bwd(fake, fake, fake, 16, fake, 0.125, fake, None, None, fake, 8, None, 4, 16,
                            *([F32] * 7), None, 0, None)
    assert rc == _lib.ERR_INVALID and b"dz_ld" in L.naju_mixer_last_error()


def test_xent_host_checks():
    L = _lib.lib()
    fake = 0x1000
    ws_need = L.naju_xent_workspace_bytes(16)
    assert ws_need >= 16 * 8
    def fwd(ld=32, rows=16, cols=32, dt=F32, loss=fake, ws=fake, ws_bytes=ws_need):
        return L.naju_xent_fwd(fake, ld, fake, rows, cols, dt, -100, fake, loss, fake, ws, ws_bytes, None)
    assert fwd(ld=31) == _lib.ERR_INVALID and b"x_ld" in L.naju_loss_last_error()
    assert fwd(dt=7) == _lib.ERR_INVALID
    assert fwd(rows=-1) == _lib.ERR_INVALID
    assert fwd(rows=1 << 31) == _lib.ERR_UNSUPPORTED
    assert fwd(loss=None) == _lib.ERR_INVALID
    assert fwd(cols=0, ld=0) == _lib.ERR_INVALID and b"n_cols" in L.naju_loss_last_error()
    assert fwd(ws_bytes=ws_need - 1) == _lib.ERR_WORKSPACE
    assert fwd(ws=None) == _lib.ERR_WORKSPACE
    def bwd(dx_ld=32, rows=16, cols=32, dx_dt=BF16, dloss=fake):
        return L.naju_xent_bwd(fake, 32, fake, rows, cols, F32, -100, fake, fake, dloss, fake, dx_ld, dx_dt, None)
    assert bwd(dx_ld=31) == _lib.ERR_INVALID and b"dx_ld" in L.naju_loss_last_error()
    assert bwd(dx_dt=5) == _lib.ERR_INVALID
    assert bwd(dloss=None) == _lib.ERR_INVALID and b"dloss" in L.naju_loss_last_error()
    assert bwd(rows=0) == _lib.OK and L.naju_loss_last_error() == b""


def test_rmsnorm_host_checks():
    L = _lib.lib()
    fake = 0x1000
    def fwd(d=768, rows=4, x_dt=F32, y_dt=BF16, x=fake, y=fake):
        return L.naju_rmsnorm_fwd(x, fake, 1e-5, y, fake, rows, d, x_dt, y_dt, None)
    assert fwd(d=6) == _lib.ERR_UNSUPPORTED and b"multiple of 4" in L.naju_mixer_last_error()
    assert fwd(d=4100) == _lib.ERR_UNSUPPORTED
    assert fwd(x_dt=F16) == _lib.ERR_UNSUPPORTED
    assert fwd(y_dt=9) == _lib.ERR_INVALID
    assert fwd(rows=-1) == _lib.ERR_INVALID
    assert fwd(x=fake + 4) == _lib.ERR_UNSUPPORTED and b"aligned" in L.naju_mixer_last_error()
    assert fwd(y=None) == _lib.ERR_INVALID
    assert fwd(rows=0) == _lib.OK and L.naju_mixer_last_error() == b""
    need = L.naju_rmsnorm_workspace_bytes(16384, 768)
    assert need >= (16384 // 16) * 768 * 4
    def bwd(dx_dt=F32, ws=fake, ws_bytes=need, dw=fake):
        return L.naju_rmsnorm_bwd(fake, fake, fake, fake, fake, dw, 16384, 768, F32, BF16, dx_dt, ws, ws_bytes, None)
    assert bwd(dx_dt=BF16) == _lib.ERR_UNSUPPORTED and b"dx" in L.naju_mixer_last_error()
    assert bwd(ws_bytes=need - 1) == _lib.ERR_WORKSPACE
    assert bwd(ws=None) == _lib.ERR_WORKSPACE


def test_rmsnorm_module_cpu_uses_reference_expression():
    from naju_amd.mixer import RMSNorm
    m = RMSNorm(8)
    x = torch.randn(3, 8)
    ref = m.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + m.eps)
    assert torch.equal(m(x), ref)
    assert m(x, out_dtype=torch.bfloat16).dtype == torch.bfloat16


def test_xent_python_rejects_cpu_tensors():
    from naju_amd.xent import cross_entropy
    with pytest.raises(RuntimeError, match="CUDA"):
        cross_entropy(torch.zeros(2, 5), torch.zeros(2, dtype=torch.int64))


def test_readout_python_rejects_cpu_tensors():
    from naju_amd.readout import readout
    x = torch.zeros(1, 2, 4)
    with pytest.raises(RuntimeError, match="CUDA"):
        readout(x, x, x, torch.zeros(4), 0.5)


def test_unknown_flag_bits_rejected():
    L = _lib.lib()
    fake = 0x1000
    rc = L.naju_scan_fwd(*([fake] * 6), None, fake, fake, None, 2, 8, 16, 1, F32, F32, F32, 4, fake, 1 << 30, None)
    assert rc == _lib.ERR_INVALID and b"flag" in L.naju_scan_last_error()


def test_checkpoint_interval_size_queries_and_checks():
    """NAJU_CKPT_ROWS: the checkpoint shrinks with the interval on the
    matrix-core path (9 <= N <= 64) while the backward's workspace gains the
    recomputed per-sub-block states; other N accept only their default."""
    L = _lib.lib()
    fl = _lib.ckpt_rows_flag
    B_, T, D = 8, 4096, 1024
    base = L.naju_scan_ckpt_elems(B_, T, D, 64, BF16, F32, BF16)
    assert L.naju_scan_ckpt_elems_ex(B_, T, D, 64, BF16, F32, BF16, 0) == base
    assert L.naju_scan_ckpt_elems_ex(B_, T, D, 64, BF16, F32, BF16, fl(16)) == base
    for rows in (32, 64, 128):
        # the interval states only: the forward's time segments start at
        # interval boundaries, so no other state is kept
        n = L.naju_scan_ckpt_elems_ex(B_, T, D, 64, BF16, F32, BF16, fl(rows))
        assert n == B_ * (-(-T // rows)) * D * 64
    # intervals that do not divide the forward's 128-row segment unit
    for rows in (48, 96, 256, 4080):
        assert L.naju_scan_ckpt_elems_ex(B_, T, D, 64, BF16, F32, BF16, fl(rows)) == -1
        assert b"interval" in L.naju_scan_last_error()
    # a longer interval is always lighter than the default, also on small
    # grids whose forward takes many time segments (one per 16-row sub-block
    # here: 2 channel tiles, 63 sub-blocks)
    small = L.naju_scan_ckpt_elems(1, 1000, 128, 64, BF16, F32, BF16)
    assert small == 1 * 63 * 128 * 64
    for rows in (32, 64, 128):
        n = L.naju_scan_ckpt_elems_ex(1, 1000, 128, 64, BF16, F32, BF16, fl(rows))
        assert n == -(-1000 // rows) * 128 * 64 and n < small
    ws0 = L.naju_scan_workspace_bytes_ex(B_, T, D, 64, BF16, F32, BF16, 0)
    assert ws0 == L.naju_scan_workspace_bytes(B_, T, D, 64, BF16, F32, BF16)
    ws64 = L.naju_scan_workspace_bytes_ex(B_, T, D, 64, BF16, F32, BF16, fl(64))
    # the recomputed states: one float per (b, 16-row sub-block, d, n)
    assert ws64 >= ws0 + B_ * (T // 16) * D * 64 * 4
    # ragged T: the last interval is partial
    assert L.naju_scan_ckpt_elems_ex(2, 300, 96, 33, F32, F32, F32, fl(64)) == 2 * 5 * 96 * 33
    # other N: only the default interval (32 rows at N <= 8 and N > 64, the
    # backward's chunk at N = 1)
    assert L.naju_scan_ckpt_elems_ex(2, 300, 96, 4, F32, F32, F32, fl(32)) == 2 * 10 * 96 * 4
    for N, rows in ((4, 64), (128, 64), (1, 32), (8, 16)):
        assert L.naju_scan_ckpt_elems_ex(2, 300, 96, N, F32, F32, F32, fl(rows)) == -1
        assert b"interval" in L.naju_scan_last_error()
        assert L.naju_scan_workspace_bytes_ex(2, 300, 96, N, F32, F32, F32, fl(rows)) == 0
        assert b"interval" in L.naju_scan_last_error()
        # the scan calls reject it on the host, before touching any pointer
        fake = 0x1000
        rc = L.naju_scan_fwd(*([fake] * 6), None, fake, fake, None, 2, 300, 96, N, F32, F32, F32, fl(rows), fake,
                             1 << 30, None)
        assert rc == _lib.ERR_UNSUPPORTED and b"interval" in L.naju_scan_last_error()
        rc = L.naju_scan_bwd(*([fake] * 8), *([None] * 7), 2, 300, 96, N, F32, F32, F32, fl(rows), fake, 1 << 30,
                             None)
        assert rc == _lib.ERR_UNSUPPORTED and b"interval" in L.naju_scan_last_error()
    with pytest.raises(ValueError):
        fl(24)
    with pytest.raises(ValueError):
        fl(4096)


def test_noalloc_status_host_checks():
    """naju_scan_noalloc_status rejects a null status pointer on the host."""
    L = _lib.lib()
    assert L.naju_scan_noalloc_status(None, None) == _lib.ERR_INVALID
    assert b"status" in L.naju_scan_last_error()


def test_env_checkpoint_interval_default(monkeypatch):
    """NAJU_CKPT_ROWS sets the interval of calls that name none, where it is
    served (9 <= N <= 64); other N keep their default."""
    from naju_amd import scan as scan_mod
    monkeypatch.delenv("NAJU_CKPT_ROWS", raising=False)
    assert scan_mod._default_ckpt_rows(64) == 0
    monkeypatch.setenv("NAJU_CKPT_ROWS", "128")
    assert scan_mod._default_ckpt_rows(64) == 128
    assert scan_mod._default_ckpt_rows(9) == 128
    assert scan_mod._default_ckpt_rows(1) == 0
    assert scan_mod._default_ckpt_rows(8) == 0
    assert scan_mod._default_ckpt_rows(65) == 0


def test_strided_bc_rejections():
    """Row strides the kernels do not serve return an error, not a wrong
    answer (host checks only: nothing is launched)."""
    L = _lib.lib()

    def fwd(N, ld, B=256, C=256):
        return L.naju_scan_fwd_strided(256, 256, 256, B, C, 256, None, 256, 256, None, 1, 8, 16, N, ld,
                                       0, 0, 0, 0, 256, 1 << 20, None)

    assert fwd(16, 8) == _lib.ERR_INVALID
    assert fwd(1, 4) == _lib.ERR_UNSUPPORTED
    assert fwd(128, 260) == _lib.ERR_UNSUPPORTED
    assert fwd(16, 34) == _lib.ERR_UNSUPPORTED
    assert fwd(16, 36, B=260) == _lib.ERR_UNSUPPORTED
    assert fwd(16, (1 << 24) + 4) == _lib.ERR_UNSUPPORTED


def test_gate_gradient_layout_rejections():
    """naju_scan_bwd_ex's gate-gradient options off the matrix-core path or
    with a stride it cannot serve return an error (host checks only)."""
    import ctypes
    L = _lib.lib()

    def bwd(N, **kw):
        lay = _lib.ScanBwdLayout(**kw)
        return L.naju_scan_bwd_ex(256, 256, 256, 256, 256, 256, 256, 256, 256, 256, 256, None, None, None, None,
                                  1, 8, 16, N, 0, 0, 0, 0, ctypes.byref(lay), 256, 1 << 20, None)

    assert bwd(1, dg_ld=20) == _lib.ERR_UNSUPPORTED
    assert bwd(1, dfl_sum=256) == _lib.ERR_UNSUPPORTED
    assert bwd(128, dg_dtype=_lib.DT_BF16) == _lib.ERR_UNSUPPORTED
    assert bwd(16, dg_ld=8) == _lib.ERR_INVALID
    assert bwd(16, dg_ld=18) == _lib.ERR_UNSUPPORTED
    assert bwd(16, dg_dtype=7) == _lib.ERR_INVALID
