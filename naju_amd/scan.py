"""Naju scan on MI355X behind the reference's scan-backend interface.

Public surface, mirroring /root/reference/naju/scan.py:

* ``naju_scan_hip(u, f_logit, i_logit, B, C, D_skip, h0=None,
  return_final_state=False)`` -- the backend callable, same 6-tensor
  signature as every reference backend (scan.py:3-13, chunk_triton.py:203,
  cuda/__init__.py:66) plus an optional initial state ``h0`` [B, D, N] (the
  reference always starts from zero, scan.py:84). Differentiable; the
  backward returns the gradients of all inputs, including ``h0``. With
  ``return_final_state=True`` it returns ``(y, hT)``, hT = x_{T-1} [B, D, N]
  float32, the state a streaming decoder resumes from (pass it as ``h0`` of
  the next segment); hT is not differentiable (no gradient flows back
  through it), which is what inference needs.
* ``naju_scan(..., backend=None)`` / ``resolve_backend`` / ``_BACKEND_CACHE``
  -- the dispatch of scan.py:45-76 for code that runs without the reference
  package. The only backend name served here is ``"hip"``. Without a GPU the
  default name is ``"reference"`` as in scan.py:50-51, but no CPU scan ships
  with this package: the call raises until one is registered under that
  name (the tests register the oracle's loop).
* ``workspace_status(device=None)`` -- reads (and clears) the status word of
  the current stream's workspace. After every N = 1 call (the only kernels
  that hand carries between workgroups) the wrapper copies that word to
  pinned host memory asynchronously; the next call or backward on the same
  stream reads the copy once it has landed (no synchronisation) and raises
  ``NajuScanError`` when a hand-off failed, clearing the word so the
  workspace is usable again. ``NAJU_CHECK_STATUS=1`` checks synchronously
  after every call instead.
* ``register(name="hip", scan_module=None)`` -- inserts ``naju_scan_hip`` into
  the reference's ``naju.scan._BACKEND_CACHE``. ``_get`` returns cached entries
  before it validates names (scan.py:55-57) and ``resolve_backend`` lower-cases
  (scan.py:52), so ``NAJU_SCAN_BACKEND=hip`` or ``NajuMixer(scan_backend="hip")``
  then routes unmodified NajuMixer / NajuLM code to these kernels.

Tensor conventions follow the reference (scan.py:7-11): [B,T,D]
streams with D contiguous, [B,T,N] for B and C, [D] for D_skip. Inputs are
never modified. ``y`` has u's dtype (the convention of the GPU training
backends, chunk_triton.py:181 and chunk_affine_triton.py:288); each gradient
has its input's dtype. Arithmetic and state are float32.
"""
import ctypes
import os

import torch

from naju_amd import _lib
from naju_amd.gradsink import acc_sink_of, sink_of

_BACKEND_CACHE = {}

_DT = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}


def _ptr(t):
    return None if t is None else t.data_ptr()


class _Workspace:
    """One zero-filled workspace per (device, stream), grown on demand. The
    kernels return it to a reusable state after every call, so it is zeroed
    only when (re)allocated. Per workspace also a pinned host copy of its
    status word and the event that marks when the copy has landed."""

    def __init__(self):
        self._bufs = {}
        self._status = {}

    def get(self, device, stream, nbytes):
        key = (device.index, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WS = _Workspace()


def _flags():
    """NAJU_FLAG_DETERMINISTIC when torch's deterministic mode is on
    (torch.use_deterministic_algorithms(True)): bitwise repeatable N = 1
    carries, at a cost in speed."""
    return _lib.FLAG_DETERMINISTIC if torch.are_deterministic_algorithms_enabled() else 0


def _stream_handle(device):
    return torch.cuda.current_stream(device).cuda_stream


_STATUS_MSG = {1: "a carry hand-off between workgroups exceeded its bounded wait (outputs are NaN)",
               2: "a ticket counter was out of range: the workspace was not zero-filled (outputs are NaN)"}


def workspace_status(device=None):
    """Status word of the workspace of (device, current stream): 0 healthy,
    1 or 2 after a failed call (then cleared, so the workspace is usable
    again). Synchronises the stream."""
    import ctypes
    dev = torch.device("cuda", torch.cuda.current_device() if device is None else torch.device(device).index)
    stream = _stream_handle(dev)
    buf = _WS._bufs.get((dev.index, stream))
    if buf is None:
        return 0
    st = ctypes.c_uint32(0)
    _lib.check(_lib.lib().naju_scan_workspace_status(buf.data_ptr(), stream, ctypes.byref(st)))
    return st.value


def _check_status(dev):
    if os.environ.get("NAJU_CHECK_STATUS", "0") not in ("", "0"):
        st = workspace_status(dev)
        if st:
            raise _lib.NajuScanError(st, _STATUS_MSG.get(st, f"status {st}"))


def _watch_status(dev, stream, ws):
    """Queue an asynchronous copy of the workspace's status word (word 0) to
    pinned host memory behind the call just issued on `stream`, and mark its
    landing with an event. Not while the stream is being captured into a
    graph (the copy would be recorded too)."""
    if torch.cuda.is_current_stream_capturing():
        return
    key = (dev.index, stream)
    ent = _WS._status.get(key)
    if ent is None:
        ent = (torch.zeros(1, dtype=torch.int32, pin_memory=True), torch.cuda.Event())
        _WS._status[key] = ent
    ent[0].copy_(ws[:4].view(torch.int32), non_blocking=True)
    ent[1].record()


def _raise_pending(dev, stream):
    """Raise NajuScanError if the last landed status copy of this stream's
    workspace is nonzero (a failed hand-off in an earlier call: its outputs
    were NaN). Does not wait for a copy still in flight: the word stays set
    on the device until cleared, so a later copy shows it. On raising, the
    word is cleared (synchronously), so the workspace is usable again.
    Nothing is queried while the stream is being captured into a graph."""
    if torch.cuda.is_current_stream_capturing():
        return
    ent = _WS._status.get((dev.index, stream))
    if ent is None or not ent[1].query():
        return
    st = int(ent[0][0])
    if st:
        ent[0].zero_()
        workspace_status(dev)  # clears the word and rewinds the counters
        raise _lib.NajuScanError(st, "an earlier scan call on this stream failed: "
                                 + _STATUS_MSG.get(st, f"status {st}"))


def _norm_inputs(u, f_logit, i_logit, B, C, D_skip, h0, bc_strided=False):
    """Contiguous tensors in a dtype combination the kernels serve:
    u in {f32,bf16,f16}; gates and B/C each f32 or u's dtype; D_skip, h0 f32.
    bc_strided: B and C stay as they are when their dtype is served (the
    strided scan calls read their rows in place)."""
    if u.dtype not in _DT:
        u = u.float()
    xd = u.dtype
    if not (f_logit.dtype == i_logit.dtype and f_logit.dtype in (xd, torch.float32)):
        f_logit, i_logit = f_logit.float(), i_logit.float()
    if xd == torch.float32 and f_logit.dtype != torch.float32:
        f_logit, i_logit = f_logit.float(), i_logit.float()
    if not (B.dtype == C.dtype and B.dtype in (xd, torch.float32)):
        B, C = B.float(), C.float()
    D_skip = D_skip.float()
    if h0 is not None:
        h0 = h0.float().contiguous()
    if not bc_strided:
        B, C = B.contiguous(), C.contiguous()
    return (u.contiguous(), f_logit.contiguous(), i_logit.contiguous(), B, C, D_skip.contiguous(), h0)


def _check_shapes(u, f_logit, i_logit, B, C, D_skip, h0):
    if u.dim() != 3:
        raise ValueError(f"u must be [B, T, D], got shape {tuple(u.shape)}")
    Bsz, T, D = u.shape
    if f_logit.shape != u.shape or i_logit.shape != u.shape:
        raise ValueError("f_logit and i_logit must have u's shape [B, T, D]")
    if B.dim() != 3 or B.shape[:2] != u.shape[:2] or C.shape != B.shape:
        raise ValueError("B and C must be [B, T, N] with u's batch and time sizes")
    if D_skip.shape != (D,):
        raise ValueError(f"D_skip must be [D]={D}, got {tuple(D_skip.shape)}")
    N = B.shape[-1]
    if h0 is not None and tuple(h0.shape) != (Bsz, D, N):
        raise ValueError(f"h0 must be [B, D, N]=({Bsz}, {D}, {N}), got {tuple(h0.shape)}")
    devs = {t.device for t in (u, f_logit, i_logit, B, C, D_skip) + ((h0,) if h0 is not None else ())}
    if len(devs) != 1 or next(iter(devs)).type != "cuda":
        raise ValueError("all scan inputs must live on one GPU device")
    return Bsz, T, D, N


def _bc_pair(B, C, N, in_place=True):
    """B and C as the scan reads them, and their row stride: on the
    matrix-core path (9 <= N <= 64), when C's columns directly follow B's in
    one tensor (the mixer's x_proj slices of its projection output), the
    scan reads them in place (rows B.stride(1) apart; the saved tensors then
    keep that whole output alive until the backward) when in_place and the
    stride and addresses are 4-element aligned, else from one copy of the 2N
    columns (B, C: its two halves, rows 2N apart); otherwise (B, C, N), for
    _norm_inputs to make contiguous."""
    if not (8 < N <= 64 and B.dtype == C.dtype and B.stride() == C.stride() and B.stride(2) == 1):
        return B, C, N
    es = B.element_size()
    ld = B.stride(1)
    if C.data_ptr() != B.data_ptr() + N * es or ld < 2 * N or B.stride(0) != B.shape[1] * ld:
        return B, C, N
    if in_place and ld % 4 == 0 and B.data_ptr() % (4 * es) == 0 and C.data_ptr() % (4 * es) == 0 and ld <= 1 << 24:
        return B, C, ld
    bc = torch.as_strided(B, (B.shape[0], B.shape[1], 2 * N), B.stride()).contiguous()
    return bc[..., :N], bc[..., N:], 2 * N


class NajuScanHip(torch.autograd.Function):
    """Autograd wrapper of naju_scan_fwd / naju_scan_bwd (include/naju_scan.h)."""

    @staticmethod
    def forward(ctx, u, f_logit, i_logit, B, C, D_skip, h0=None, want_hT=False, ckpt_rows=0, du_skip=None,
                gate_grads=None):
        Bsz, T, D, N = _check_shapes(u, f_logit, i_logit, B, C, D_skip, h0)
        out_dtype = u.dtype
        b_sinks = (sink_of(B), sink_of(C))
        # a memory-light checkpoint interval keeps B and C as a copy, so the
        # projection output is not held until the backward
        Bp, Cp, bc_ld = _bc_pair(B, C, N, in_place=int(ckpt_rows or 0) <= 16)
        u_, fl_, il_, B_, C_, D_, h0_ = _norm_inputs(u, f_logit, i_logit, Bp, Cp, D_skip, h0, bc_ld != N)
        if bc_ld != N and (B_.data_ptr() != Bp.data_ptr() or C_.data_ptr() != Cp.data_ptr()):
            # _norm_inputs converted their dtype: contiguous copies after all
            B_, C_, bc_ld = B_.contiguous(), C_.contiguous(), N
        dts = (_DT[u_.dtype], _DT[fl_.dtype], _DT[B_.dtype])
        L = _lib.lib()
        dev = u_.device
        stream = _stream_handle(dev)
        need_grad = any(ctx.needs_input_grad)
        flags = _flags() | _lib.ckpt_rows_flag(ckpt_rows)
        ckpt = None
        if need_grad:
            n = L.naju_scan_ckpt_elems_ex(Bsz, T, D, N, *dts, flags)
            if n < 0:
                _lib.check(_lib.ERR_UNSUPPORTED if "interval" in _lib.last_error() else _lib.ERR_INVALID)
            ckpt = torch.empty(max(n, 1), dtype=torch.float32, device=dev)
        nbytes = L.naju_scan_workspace_bytes_ex(Bsz, T, D, N, *dts, flags)
        if nbytes == 0 and Bsz * T * D > 0:
            _lib.check(_lib.ERR_UNSUPPORTED if "interval" in _lib.last_error() else _lib.ERR_INVALID)
        _raise_pending(dev, stream)
        ws = _WS.get(dev, stream, nbytes)
        y = torch.empty((Bsz, T, D), dtype=u_.dtype, device=dev)
        hT = torch.empty((Bsz, D, N), dtype=torch.float32, device=dev) if want_hT else None
        if bc_ld != N:
            _lib.check(L.naju_scan_fwd_strided(
                _ptr(u_), _ptr(fl_), _ptr(il_), _ptr(B_), _ptr(C_), _ptr(D_), _ptr(h0_),
                _ptr(y), _ptr(ckpt), _ptr(hT), Bsz, T, D, N, bc_ld, *dts, flags, ws.data_ptr(), ws.numel(), stream))
        else:
            _lib.check(L.naju_scan_fwd(
                _ptr(u_), _ptr(fl_), _ptr(il_), _ptr(B_), _ptr(C_), _ptr(D_), _ptr(h0_),
                _ptr(y), _ptr(ckpt), _ptr(hT), Bsz, T, D, N, *dts, flags, ws.data_ptr(), ws.numel(), stream))
        if N == 1:
            _watch_status(dev, stream, ws)
        _check_status(dev)
        if need_grad:
            # du_skip: the skip coefficient of du's D dy term in place of
            # D_skip (naju_scan_hip's doc)
            D_b = D_ if du_skip is None else du_skip.detach().float().contiguous()
            ctx.save_for_backward(u_, fl_, il_, B_, C_, D_, ckpt, D_b)
            ctx.meta = (Bsz, T, D, N, dts, flags, h0 is not None,
                        (u.dtype, f_logit.dtype, i_logit.dtype, B.dtype, C.dtype, D_skip.dtype))
            # u is a gradsink.fanout() alias: du goes into the fan-out's
            # buffer when it is the first gradient there
            ctx.u_acc = acc_sink_of(u) if u_ is u else None
            ctx.bc_ld = bc_ld
            # the gate logits' gradients may go straight to their consumer
            # (naju_amd.dwconv.GateGrads: the gate convolutions' backward)
            ctx.gate_grads = gate_grads
            # B and C are pieces of one gradsink.split (the mixer's
            # projection output): dB and dC can go straight into its buffer
            s0, s1 = b_sinks
            ctx.bc_sinks = b_sinks if (bc_ld != N and s0 is not None and s1 is not None and s0[0] is s1[0]
                                       and s0[0].dtype == B_.dtype) else None
        y = y if y.dtype == out_dtype else y.to(out_dtype)
        if want_hT:
            ctx.mark_non_differentiable(hT)
            return y, hT
        return y

    @staticmethod
    def backward(ctx, dy, *_unused_dhT):
        u_, fl_, il_, B_, C_, D_, ckpt, D_b = ctx.saved_tensors
        Bsz, T, D, N, dts, flags, has_h0, in_dtypes = ctx.meta
        ng = ctx.needs_input_grad
        dev = u_.device
        dy = dy.to(u_.dtype).contiguous()
        du = du_ret = None
        if ng[0]:
            if ctx.u_acc is not None and ctx.u_acc.buf is None:
                du, _ = ctx.u_acc.target()
                du_ret = ctx.u_acc.marker()
            else:
                du = torch.empty_like(u_)
        # both gate gradients into the projection gradient buffer the gate
        # logits' consumer names (its type and row stride), with the float32
        # sums of both (the gate biases' gradients), on the matrix-core path
        gg = getattr(ctx, "gate_grads", None)
        gtgt = gg.targets() if (gg is not None and ng[1] and ng[2] and 8 < N <= 64
                                and not (flags & _lib.FLAG_OUT_F32)) else None
        if gtgt is not None:
            dfl, dil = gtgt
            gsum = torch.empty((2, D), dtype=torch.float32, device=dev)
        else:
            dfl = torch.empty_like(fl_) if ng[1] else None
            dil = torch.empty_like(il_) if ng[2] else None
        dB = dC = None
        dbc_ld = N
        if ctx.bc_ld != N and (ng[3] or ng[4]):
            if ctx.bc_sinks is not None and not (flags & _lib.FLAG_OUT_F32):
                # written in place into the split's gradient buffer, which its
                # backward then takes as it is
                (sb, cb), (sc, cc) = ctx.bc_sinks
                dB, dC = sb.slice(cb, N), sc.slice(cc, N)
            else:
                dbc = torch.empty((Bsz, T, 2 * N), dtype=B_.dtype, device=dev)
                dB, dC = dbc[..., :N], dbc[..., N:]
            dbc_ld = dB.stride(1)
            if dC.stride(1) != dbc_ld:
                dbc = torch.empty((Bsz, T, 2 * N), dtype=B_.dtype, device=dev)
                dB, dC, dbc_ld = dbc[..., :N], dbc[..., N:], 2 * N
            dB, dC = (dB if ng[3] else None), (dC if ng[4] else None)
        else:
            dB = torch.empty_like(B_) if ng[3] else None
            dC = torch.empty_like(C_) if ng[4] else None
        dD = torch.empty((D,), dtype=torch.float32, device=dev) if ng[5] else None
        want_h0 = has_h0 and len(ng) > 6 and ng[6]
        dh0 = torch.empty((Bsz, D, N), dtype=torch.float32, device=dev) if want_h0 else None
        L = _lib.lib()
        stream = _stream_handle(dev)
        _raise_pending(dev, stream)
        ws = _WS.get(dev, stream, L.naju_scan_workspace_bytes_ex(Bsz, T, D, N, *dts, flags))
        if gtgt is not None:
            lay = _lib.ScanBwdLayout(bc_ld=ctx.bc_ld, dbc_ld=dbc_ld, dg_ld=dfl.stride(1), dg_dtype=_DT[dfl.dtype],
                                     dfl_sum=gsum.data_ptr(), dil_sum=gsum.data_ptr() + 4 * D)
            _lib.check(L.naju_scan_bwd_ex(
                _ptr(u_), _ptr(fl_), _ptr(il_), _ptr(B_), _ptr(C_), _ptr(D_b), _ptr(ckpt), _ptr(dy),
                _ptr(du), _ptr(dfl), _ptr(dil), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dh0),
                Bsz, T, D, N, *dts, flags, ctypes.byref(lay), ws.data_ptr(), ws.numel(), stream))
        elif ctx.bc_ld != N or dbc_ld != N:
            _lib.check(L.naju_scan_bwd_strided(
                _ptr(u_), _ptr(fl_), _ptr(il_), _ptr(B_), _ptr(C_), _ptr(D_b), _ptr(ckpt), _ptr(dy),
                _ptr(du), _ptr(dfl), _ptr(dil), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dh0),
                Bsz, T, D, N, ctx.bc_ld, dbc_ld, *dts, flags, ws.data_ptr(), ws.numel(), stream))
        else:
            _lib.check(L.naju_scan_bwd(
                _ptr(u_), _ptr(fl_), _ptr(il_), _ptr(B_), _ptr(C_), _ptr(D_b), _ptr(ckpt), _ptr(dy),
                _ptr(du), _ptr(dfl), _ptr(dil), _ptr(dB), _ptr(dC), _ptr(dD), _ptr(dh0),
                Bsz, T, D, N, *dts, flags, ws.data_ptr(), ws.numel(), stream))
        if N == 1:
            _watch_status(dev, stream, ws)
        _check_status(dev)
        grads = [du, dfl, dil, dB, dC, dD]
        if gtgt is not None:
            # the consumer takes them from gg; autograd carries markers
            grads[1], grads[2] = gg.hand_over(dfl, dil, gsum[0], gsum[1], fl_.shape, in_dtypes[1], in_dtypes[2])
        grads = [g if g is None or g.dtype == dt else g.to(dt) for g, dt in zip(grads, in_dtypes)]
        if du_ret is not None:
            grads[0] = du_ret
        return (*grads, dh0, None, None, None, None)


def _default_ckpt_rows(N):
    """The checkpoint interval of calls that name none: NAJU_CKPT_ROWS from
    the environment where it is served (9 <= N <= 64), else the default. It
    lets unmodified NajuMixer / NajuLM code run the memory-light mode, as
    NAJU_SCAN_BACKEND=cuda selects the reference's recompute backend."""
    v = os.environ.get("NAJU_CKPT_ROWS", "")
    return int(v) if v and 9 <= N <= 64 else 0


def naju_scan_hip(u, f_logit, i_logit, B, C, D_skip, h0=None, return_final_state=False, ckpt_rows=None,
                  du_skip=None, gate_grads=None):
    """y = scan(u, f_logit, i_logit, B, C, D_skip[, h0]) on the GPU (see module
    doc); (y, hT) with return_final_state=True. ckpt_rows: the checkpoint
    interval kept for the backward (None = NAJU_CKPT_ROWS from the
    environment where served, else the default; 32, 64 or 128 rows, served
    at 9 <= N <= 64, is the memory-light mode: the backward recomputes the
    states between, with bitwise the same outputs).

    du_skip ([D], no gradient): the backward forms du = i dws + du_skip dy
    instead of i dws + D_skip dy (the forward still adds D_skip u to y). A
    caller that multiplies y by s and adds D u itself (the mixer's readout,
    naju/mixer.py:123-124, called with D_skip = 0) passes du_skip = D / s:
    then du already holds the gradient of that D u term, which the caller's
    own backward can leave out (one gradient fewer to add)."""
    if ckpt_rows is None:
        ckpt_rows = _default_ckpt_rows(B.shape[-1])
    return NajuScanHip.apply(u, f_logit, i_logit, B, C, D_skip, h0, bool(return_final_state), int(ckpt_rows),
                             du_skip, gate_grads)


def resolve_backend(backend=None):
    """Selection order of scan.py:48-52: explicit > NAJU_SCAN_BACKEND > "hip"
    when a GPU is visible, else "reference"."""
    b = backend or os.environ.get("NAJU_SCAN_BACKEND") or ("hip" if torch.cuda.is_available() else "reference")
    return b.lower()


def _get(b):
    fn = _BACKEND_CACHE.get(b)
    if fn is None:
        if b in ("hip", "naju_amd"):
            fn = naju_scan_hip
        elif b == "reference":
            raise ValueError("no CPU scan backend ships with naju_amd (the reference's CPU default, "
                             "naju/scan.py:50-51, is its sequential loop): register a callable with the "
                             "6-tensor scan signature as _BACKEND_CACHE['reference'], or run on a GPU "
                             "with backend 'hip'")
        else:
            raise ValueError(f"unknown scan backend {b!r}; valid: hip")
        _BACKEND_CACHE[b] = fn
    return fn


def naju_scan(u, f_logit, i_logit, B, C, D_skip, backend=None, h0=None):
    """Dispatching entry point with the signature of scan.py:75-76 (+ h0)."""
    fn = _get(resolve_backend(backend))
    if h0 is None:
        return fn(u, f_logit, i_logit, B, C, D_skip)
    return fn(u, f_logit, i_logit, B, C, D_skip, h0)


def register(name="hip", scan_module=None):
    """Register naju_scan_hip as backend `name` of the reference dispatcher.

    scan_module defaults to ``naju.scan`` (imported lazily); pass the module
    explicitly when it lives elsewhere. Registering as "chunk" also captures
    the reference's automatic GPU default (scan.py:51)."""
    if scan_module is None:
        import importlib
        scan_module = importlib.import_module("naju.scan")
    scan_module._BACKEND_CACHE[name.lower()] = naju_scan_hip
    _BACKEND_CACHE[name.lower()] = naju_scan_hip
    return naju_scan_hip
