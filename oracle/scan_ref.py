"""TEST INFRASTRUCTURE ONLY -- CPU oracle for the Naju gated state-space scan.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker. The product path (naju_amd/) never calls
it and fails loudly when its HIP library is missing.

Two independent restatements of the reference's sequential scan:

* ``scan_loop_torch`` -- the same Python loop over T with torch CPU ops as
  /root/reference/naju/scan.py:79-93 (naju_scan_reference), with the optional
  initial state h0 added (the reference starts at zero, scan.py:84). Gradients
  come from torch autograd, so they do not depend on hand-derived adjoint
  formulas. This is also the CPU baseline algorithm of bench.py.
* ``oracle_fwd`` / ``oracle_bwd`` -- fp64 C (oracle/scan_ref.c) with the
  explicit adjoint of /root/reference/naju/cuda/naju_cuda.cu:104-141.

How each function is pinned (tests/test_oracle.py):
  scan_loop_torch fwd : closed forms (geometric series for constant gates,
                        f==0, f==1 prefix sum, i==0 decay of h0), causality.
  scan_loop_torch bwd : torch.autograd.gradcheck (finite differences, fp64).
  oracle_fwd          : equals scan_loop_torch (fp64) and the closed forms.
  oracle_bwd          : equals autograd of scan_loop_torch (fp64); exact
                        zeros of dfl at f in {0,1}; dD == sum dy*u.
  h0 / dh0 extension  : reduced to the reference's zero-init 6-argument
                        scan by prepending N "load" tokens (test_oracle.py).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libnaju_oracle.so")
_lib = None


def build():
    """Compile oracle/scan_ref.c into oracle/libnaju_oracle.so (gcc)."""
    import subprocess
    subprocess.check_call(["make", "-s", "-C", _HERE, "libnaju_oracle.so"])


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        lib.naju_oracle_fwd.argtypes = [P] * 7 + [I] * 4 + [P, P]
        lib.naju_oracle_fwd.restype = None
        lib.naju_oracle_bwd.argtypes = [P] * 8 + [I] * 4 + [P] * 7
        lib.naju_oracle_bwd.restype = None
        lib.naju_oracle_fwd_channels.argtypes = [P] * 7 + [I] * 4 + [P, I, P]
        lib.naju_oracle_fwd_channels.restype = None
        lib.naju_oracle_bwd_channels.argtypes = [P] * 8 + [I] * 4 + [P, I] + [P] * 4
        lib.naju_oracle_bwd_channels.restype = None
        _lib = lib
    return _lib


def _f32(a):
    """Contiguous float32 numpy view/copy of a numpy array or torch tensor."""
    if a is None:
        return None
    if hasattr(a, "detach"):
        a = a.detach().float().cpu().numpy()
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def oracle_fwd(u, fl, il, Bm, Cm, Dsk, h0=None, want_hT=False):
    """fp64 forward. Inputs: arrays/tensors of shapes [B,T,D]x3, [B,T,N]x2,
    [D], optional h0 [B,D,N]. Returns y [B,T,D] float64 (and hT [B,D,N])."""
    lib = _load()
    u, fl, il, Bm, Cm, Dsk, h0 = map(_f32, (u, fl, il, Bm, Cm, Dsk, h0))
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    y = np.empty((Bsz, T, D), np.float64)
    hT = np.empty((Bsz, D, N), np.float64) if want_hT else None
    lib.naju_oracle_fwd(_ptr(u), _ptr(fl), _ptr(il), _ptr(Bm), _ptr(Cm),
                        _ptr(Dsk), _ptr(h0), Bsz, T, D, N, _ptr(y), _ptr(hT))
    return (y, hT) if want_hT else y


def oracle_bwd(u, fl, il, Bm, Cm, Dsk, dy, h0=None):
    """fp64 explicit backward. Returns dict du, dfl, dil, dB, dC, dD, dh0."""
    lib = _load()
    u, fl, il, Bm, Cm, Dsk, dy, h0 = map(_f32, (u, fl, il, Bm, Cm, Dsk, dy, h0))
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    out = {
        "du": np.empty((Bsz, T, D)), "dfl": np.empty((Bsz, T, D)),
        "dil": np.empty((Bsz, T, D)), "dB": np.empty((Bsz, T, N)),
        "dC": np.empty((Bsz, T, N)), "dD": np.empty((D,)),
        "dh0": np.empty((Bsz, D, N)),
    }
    lib.naju_oracle_bwd(_ptr(u), _ptr(fl), _ptr(il), _ptr(Bm), _ptr(Cm),
                        _ptr(Dsk), _ptr(h0), _ptr(dy), Bsz, T, D, N,
                        *[_ptr(out[k]) for k in ("du", "dfl", "dil", "dB", "dC", "dD", "dh0")])
    return out


def oracle_fwd_channels(u, fl, il, Bm, Cm, Dsk, chans, h0=None):
    """fp64 forward for a subset of channels chans (flat b*D+d). -> [nch, T]."""
    lib = _load()
    u, fl, il, Bm, Cm, Dsk, h0 = map(_f32, (u, fl, il, Bm, Cm, Dsk, h0))
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    ch = np.ascontiguousarray(chans, dtype=np.int64)
    y = np.empty((len(ch), T), np.float64)
    lib.naju_oracle_fwd_channels(_ptr(u), _ptr(fl), _ptr(il), _ptr(Bm), _ptr(Cm),
                                 _ptr(Dsk), _ptr(h0), Bsz, T, D, N, _ptr(ch),
                                 len(ch), _ptr(y))
    return y


def oracle_bwd_channels(u, fl, il, Bm, Cm, Dsk, dy, chans, h0=None):
    """fp64 per-channel backward: dict du, dfl, dil ([nch,T]) and dh0 ([nch,N])."""
    lib = _load()
    u, fl, il, Bm, Cm, Dsk, dy, h0 = map(_f32, (u, fl, il, Bm, Cm, Dsk, dy, h0))
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    ch = np.ascontiguousarray(chans, dtype=np.int64)
    out = {"du": np.empty((len(ch), T)), "dfl": np.empty((len(ch), T)),
           "dil": np.empty((len(ch), T)), "dh0": np.empty((len(ch), N))}
    lib.naju_oracle_bwd_channels(_ptr(u), _ptr(fl), _ptr(il), _ptr(Bm), _ptr(Cm),
                                 _ptr(Dsk), _ptr(h0), _ptr(dy), Bsz, T, D, N,
                                 _ptr(ch), len(ch),
                                 *[_ptr(out[k]) for k in ("du", "dfl", "dil", "dh0")])
    return out


def scan_loop_torch(u, f_logit, i_logit, B, C, D_skip, h0=None):
    """Restatement of naju_scan_reference (scan.py:79-93): sequential loop over
    T of torch ops; optional h0 [B,D,N] replaces the zero init of scan.py:84.
    Differentiable with torch autograd; runs on whatever device/dtype it gets."""
    import torch
    Bsz, T, D = u.shape
    N = B.shape[-1]
    f = torch.sigmoid(f_logit)                       # scan.py:82
    i = torch.sigmoid(i_logit)                       # scan.py:83
    x = u.new_zeros(Bsz, D, N) if h0 is None else h0.to(u.dtype)
    ys = []
    for t in range(T):                               # scan.py:86
        f_t = f[:, t].unsqueeze(-1)
        i_t = i[:, t].unsqueeze(-1)
        B_t = B[:, t].unsqueeze(1)
        C_t = C[:, t].unsqueeze(1)
        u_t = u[:, t].unsqueeze(-1)
        x = f_t * x + i_t * B_t * u_t                # scan.py:90
        ys.append((C_t * x).sum(-1) + D_skip.unsqueeze(0) * u[:, t])   # scan.py:91
    return torch.stack(ys, dim=1)                    # scan.py:93


def rel_err(out, ref):
    """(max-abs error / max|ref|, ||err||_2 / ||ref||_2) -- the tolerance
    measure used by every parity test."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = out - ref
    den_max = max(np.abs(ref).max(), 1e-30)
    den_l2 = max(np.linalg.norm(ref), 1e-30)
    return float(np.abs(err).max() / den_max), float(np.linalg.norm(err) / den_l2)
