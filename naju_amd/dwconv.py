"""Depthwise causal convolutions of the mixer on the HIP kernels of
include/naju_mixer.h.

``dwconv(x, weight, bias=None, add=None, silu=False, out_dtype=None)``

    y[:, t] = act(add[:, t] + bias + sum_j w[:, j] * x[:, t - (k-1) + j])

for x and add [B, T, C] (C contiguous; a row stride above C is taken as it
is, so one slice of a chunked projection needs no copy), weight [C, 1, k] or [C, k]
(nn.Conv1d with groups = C), bias [C]. ``silu`` applies SiLU to the result
(then ``add`` must be None). Differentiable in x, weight, bias and add; the
backward is deterministic. This is the reference's Conv1d(groups=C,
padding=k-1) + slice (naju/mixer.py:108-110, 115) in the [B, T, C] layout the
scan uses, with float32 arithmetic and one rounding at the output.

CUDA tensors only: there is no other implementation behind this function,
and a missing library raises.
"""
import torch

from naju_amd import _lib
from naju_amd.gradsink import _zero, acc_sink_of, sink_of

_DT = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}
# naju_dwconv_bwd: dx += the gradient (include/naju_mixer.h)
_ACCUM_DX = 2


class _Workspace:
    """Per-(device, stream) scratch for the backward's partial sums, grown on
    demand (the kernels overwrite every byte they later read)."""

    def __init__(self):
        self._bufs = {}

    def get(self, device, stream, nbytes):
        key = (device.index, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WS = _Workspace()


def _ptr(t):
    return None if t is None else t.data_ptr()


def _rows(x):
    """(x, row stride in elements) with C contiguous and [B, T] collapsible."""
    B, T, C = x.shape
    if x.stride(2) != 1 or x.stride(0) != T * x.stride(1) or x.stride(1) < C:
        x = x.contiguous()
    return x, x.stride(1)


class _DwConv(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, bias, add, silu, out_dtype, x_sink, add_sink, x_acc):
        B, T, C = x.shape
        K = w.shape[1]
        x, ldx = _rows(x)
        y = torch.empty((B, T, C), dtype=out_dtype, device=x.device)
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        ld_add = C
        if add is not None:
            add, ld_add = _rows(add)
        _lib.check_mixer(L.naju_dwconv_fwd(
            _ptr(x), ldx, _ptr(w), _ptr(bias), _ptr(add), ld_add, _ptr(y), B, T, C, K, int(silu), _DT[x.dtype],
            _DT[add.dtype] if add is not None else 0, _DT[out_dtype], stream))
        ctx.save_for_backward(x, w, bias)
        ctx.silu = silu
        ctx.add_dtype = None if add is None else add.dtype
        # pieces of a gradsink.split(): their gradients go into its buffer
        ctx.x_sink, ctx.add_sink = x_sink, add_sink
        # x is a gradsink.fanout() alias: dx is written into, or added to,
        # the fan-out's buffer
        ctx.x_acc = x_acc
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, bias = ctx.saved_tensors
        B, T, C = x.shape
        K = w.shape[1]
        if dy.dtype not in _DT:
            dy = dy.float()
        dy = dy.contiguous()
        need_x, need_w, need_b, need_add = ctx.needs_input_grad[:4]
        dx = None
        act = int(ctx.silu)
        dx_ret = None
        if need_x:
            if ctx.x_sink is not None:
                sink, col = ctx.x_sink
                dx = sink.slice(col, C)
            elif ctx.x_acc is not None:
                dx, accumulate = ctx.x_acc.target()
                if accumulate:
                    act |= _ACCUM_DX
                dx_ret = ctx.x_acc.marker()
            else:
                dx = torch.empty((B, T, C), dtype=x.dtype, device=x.device)
        dw = torch.empty((C, K), dtype=torch.float32, device=x.device) if need_w else None
        db = torch.empty((C,), dtype=torch.float32, device=x.device) if (need_b and bias is not None) else None
        # the gradient of add is dy: written by the kernel into the sink's
        # buffer (in add's dtype and row stride), or a cast of dy
        dadd = None
        if need_add and ctx.add_dtype is not None and ctx.add_sink is not None and not ctx.silu:
            sink, col = ctx.add_sink
            dadd = sink.slice(col, C)
        if dx is not None or dw is not None or db is not None or dadd is not None:
            L = _lib.lib()
            stream = torch.cuda.current_stream(x.device).cuda_stream
            nbytes = L.naju_dwconv_workspace_bytes(B, T, C, K)
            ws = _WS.get(x.device, stream, nbytes)
            _lib.check_mixer(L.naju_dwconv_bwd(
                _ptr(x), x.stride(1), _ptr(w), _ptr(bias), _ptr(dy), _ptr(dx), dx.stride(1) if dx is not None else C,
                _ptr(dw), _ptr(db), _ptr(dadd), dadd.stride(1) if dadd is not None else C, B, T, C, K,
                act, _DT[x.dtype], _DT[dy.dtype], _DT[x.dtype],
                _DT[dadd.dtype] if dadd is not None else 0, _ptr(ws), ws.numel(), stream))
        if dadd is None and need_add and ctx.add_dtype is not None:
            dadd = dy.to(ctx.add_dtype)
        return dx if dx_ret is None else dx_ret, dw, db, dadd, None, None, None, None, None


def dwconv(x, weight, bias=None, add=None, silu=False, out_dtype=None):
    if not x.is_cuda:
        raise RuntimeError("naju_amd.dwconv runs on the HIP kernels only: x must be a CUDA tensor")
    if x.dim() != 3:
        raise ValueError(f"x must be [B, T, C], got {tuple(x.shape)}")
    C = x.shape[2]
    w = weight.reshape(C, -1)
    if w.dtype != torch.float32:
        w = w.float()
    w = w.contiguous()
    if bias is not None:
        bias = bias.float().contiguous()
    if silu and add is not None:
        raise ValueError("add is not supported together with silu")
    if add is not None:
        if add.shape != x.shape:
            raise ValueError(f"add must have x's shape {tuple(x.shape)}, got {tuple(add.shape)}")
    x_sink, add_sink, x_acc = sink_of(x), sink_of(add), acc_sink_of(x)
    if x.dtype not in _DT:
        x, x_sink, x_acc = x.float(), None, None
    if x_acc is not None and (x.stride(2) != 1 or x.stride(0) != x.shape[1] * x.stride(1) or x.stride(1) != C):
        x_acc = None  # the fan-out's buffer is contiguous: dx must be too
    if add is not None and add.dtype not in _DT:
        add, add_sink = add.float(), None
    if out_dtype is None:
        out_dtype = x.dtype
    return _DwConv.apply(x, w, bias, add, bool(silu), out_dtype, x_sink, add_sink, x_acc)


class GateGrads:
    """Hand-off of the two gate logits' gradients from the scan's backward
    to the gate pair's backward (naju_amd.scan.naju_scan_hip(...,
    gate_grads=)). The logits are add + bias + conv(x) with the adds pieces of
    one gradsink.split (the mixer's projection output), so their gradients
    are the adds' gradients: the scan writes them straight into the split's
    gradient buffer in its type and row stride (naju_scan_bwd_ex), with
    their float32 sums over batch and time (the biases' gradients). Autograd
    then carries zero-stride markers in their place; the pair's backward
    reads the buffer slices as its dy, writes no adds' gradients of its own,
    and takes the sums as the biases' gradients. A scan backward that cannot
    serve this returns ordinary gradients, and the pair's backward runs as
    usual."""

    def __init__(self, sinks, C):
        self.sinks, self.C = sinks, C
        self._result = None
        self._markers = None

    def targets(self):
        """The two buffer slices the scan writes (the adds' gradients)."""
        (s0, c0), (s1, c1) = self.sinks
        return s0.slice(c0, self.C), s1.slice(c1, self.C)

    def hand_over(self, g0, g1, sum0, sum1, shape, dtype0, dtype1):
        """Record what the scan wrote; returns the markers for autograd
        (zeros of the logits' shape without storage of their own)."""
        dev = g0.device
        self._result = (g0, g1, sum0, sum1)
        self._markers = (_zero(dtype0, dev).expand(shape), _zero(dtype1, dev).expand(shape))
        return self._markers

    def take(self, dy0, dy1):
        """(result, dy0, dy1) for the pair's backward, the hand-off taken
        once: (the scan's result, None, None) when dy0, dy1 are its markers;
        (None, dy0, dy1) when nothing was handed over; and when the logits
        had another consumer too (autograd added its gradient to the
        markers), (None, its gradient plus the scan's part, ...), which the
        ordinary path then writes over the scan's part in the buffer."""
        r, m = self._result, self._markers
        self._result = self._markers = None
        if r is None:
            return None, dy0, dy1
        if all(d.data_ptr() == k.data_ptr() and all(st == 0 for st in d.stride()) for d, k in zip((dy0, dy1), m)):
            return r, None, None
        return None, dy0.float() + r[0].float(), dy1.float() + r[1].float()


class _DwConvPair(torch.autograd.Function):
    """The mixer's two gate convolutions over one input in one pass each way
    (naju_dwconv_pair_fwd / _bwd): y0 = add0 + b0 + conv(x, w0), y1 = add1 +
    b1 + conv(x, w1); x's gradient from both formed with one rounding."""

    @staticmethod
    def forward(ctx, x, w0, b0, add0, w1, b1, add1, out_dtype, sinks, x_acc, gate_grads):
        B, T, C = x.shape
        K = w0.shape[1]
        ldx, ld_add = x.stride(1), add0.stride(1)
        y0 = torch.empty((B, T, C), dtype=out_dtype, device=x.device)
        y1 = torch.empty_like(y0)
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check_mixer(L.naju_dwconv_pair_fwd(
            _ptr(x), ldx, _ptr(w0), _ptr(b0), _ptr(add0), _ptr(w1), _ptr(b1), _ptr(add1), ld_add, _ptr(y0), _ptr(y1),
            B, T, C, K, _DT[x.dtype], _DT[out_dtype], stream))
        ctx.save_for_backward(x, w0, w1)
        ctx.has_b = (b0 is not None, b1 is not None)
        ctx.sinks, ctx.x_acc, ctx.gate_grads = sinks, x_acc, gate_grads
        return y0, y1

    @staticmethod
    def backward(ctx, dy0, dy1):
        x, w0, w1 = ctx.saved_tensors
        B, T, C = x.shape
        K = w0.shape[1]
        need = ctx.needs_input_grad
        gg = None
        if ctx.gate_grads is not None:
            gg, dy0, dy1 = ctx.gate_grads.take(dy0, dy1)
        if gg is not None:
            # the scan wrote dy0, dy1 as the adds' gradients into the split's
            # buffer and summed them for the biases
            dy0, dy1, gs0, gs1 = gg
        else:
            if dy1.dtype != dy0.dtype:
                dy0, dy1 = dy0.float(), dy1.float()
            dy0, dy1 = dy0.contiguous(), dy1.contiguous()
        dx = dx_ret = None
        acc = 0
        if need[0]:
            if ctx.x_acc is not None:
                dx, accumulate = ctx.x_acc.target()
                acc = int(accumulate)
                dx_ret = ctx.x_acc.marker()
            else:
                dx = torch.empty((B, T, C), dtype=x.dtype, device=x.device)
        f32 = dict(dtype=torch.float32, device=x.device)
        dw0 = torch.empty((C, K), **f32) if need[1] else None
        dw1 = torch.empty((C, K), **f32) if need[4] else None
        if gg is not None:
            db0 = gs0 if need[2] and ctx.has_b[0] else None
            db1 = gs1 if need[5] and ctx.has_b[1] else None
            # already in the split's buffer: returned as they are, not written
            dadd0 = dy0 if need[3] else None
            dadd1 = dy1 if need[6] else None
            wr0 = wr1 = wb0 = wb1 = None
            ld_dadd = C
        else:
            db0 = torch.empty((C,), **f32) if need[2] and ctx.has_b[0] else None
            db1 = torch.empty((C,), **f32) if need[5] and ctx.has_b[1] else None
            # the adds' gradients are dy0, dy1: written into the split's
            # buffer in x's dtype (pair_supported checked that the adds are
            # pieces of one gradsink.split with x's dtype)
            (s0, col0), (s1, col1) = ctx.sinks
            dadd0 = s0.slice(col0, C) if need[3] else None
            dadd1 = s1.slice(col1, C) if need[6] else None
            wr0, wr1, wb0, wb1 = dadd0, dadd1, db0, db1
            ld_dadd = (dadd0 if dadd0 is not None else dadd1).stride(1) if (dadd0 is not None
                                                                           or dadd1 is not None) else C
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        nbytes = L.naju_dwconv_pair_workspace_bytes(B, T, C, K)
        ws = _WS.get(x.device, stream, nbytes)
        _lib.check_mixer(L.naju_dwconv_pair_bwd(
            _ptr(x), x.stride(1), _ptr(w0), _ptr(w1), _ptr(dy0), _ptr(dy1), dy0.stride(1), _ptr(dx),
            dx.stride(1) if dx is not None else C, _ptr(dw0), _ptr(wb0), _ptr(dw1), _ptr(wb1), _ptr(wr0),
            _ptr(wr1), ld_dadd, B, T, C, K, acc, _DT[x.dtype], _DT[dy0.dtype], _ptr(ws), ws.numel(), stream))
        return (dx if dx_ret is None else dx_ret, dw0, db0, dadd0, dw1, db1, dadd1, None, None, None, None)


def pair_supported(x, w0, add0, w1, add1):
    """Whether dwconv_pair serves these tensors: CUDA [B, T, C] x with C and
    its row stride multiples of 8, kernel size 4, and adds that are pieces
    of one gradsink.split (one row stride, x's dtype), 16-byte aligned."""
    if not (x.is_cuda and x.dim() == 3 and x.dtype in _DT and add0.shape == x.shape and add1.shape == x.shape):
        return False
    C = x.shape[2]
    if C % 8 or w0.numel() != 4 * C or w1.numel() != 4 * C:
        return False
    s0, s1 = sink_of(add0), sink_of(add1)
    if s0 is None or s1 is None or s0[0] is not s1[0]:
        return False
    if add0.dtype != x.dtype or add1.dtype != x.dtype or add0.stride() != add1.stride():
        return False
    for t in (x, add0, add1):
        if t.stride(2) != 1 or t.stride(0) != t.shape[1] * t.stride(1) or t.stride(1) % 8 or t.data_ptr() % 16:
            return False
    return True


def dwconv_pair(x, w0, b0, add0, w1, b1, add1, out_dtype, gate_grads=False):
    """(add0 + b0 + conv(x, w0), add1 + b1 + conv(x, w1)) in one pass each
    way, for what pair_supported accepts: the two gate logits of the mixer,
    each as dwconv(x, w, b, add=add, out_dtype=out_dtype) computes it.
    gate_grads=True returns (y0, y1, GateGrads) for the logits' consumer
    (naju_scan_hip(..., gate_grads=)) to hand their gradients over."""
    C = x.shape[2]
    ws = []
    for w in (w0, w1):
        w = w.reshape(C, -1)
        ws.append((w if w.dtype == torch.float32 else w.float()).contiguous())
    bs = [None if b is None else b.float().contiguous() for b in (b0, b1)]
    x_acc = acc_sink_of(x)
    if x_acc is not None and x.stride(1) != C:
        x_acc = None
    sinks = (sink_of(add0), sink_of(add1))
    gg = GateGrads(sinks, C) if gate_grads else None
    y0, y1 = _DwConvPair.apply(x, ws[0], bs[0], add0, ws[1], bs[1], add1, out_dtype, sinks, x_acc, gg)
    return (y0, y1, gg) if gate_grads else (y0, y1)
