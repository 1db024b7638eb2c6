"""Cross-entropy of the LM training step on the HIP kernels of
include/naju_loss.h.

``cross_entropy(logits, target, ignore_index=-100)``

    mean over rows r with target[r] != ignore_index of
        logsumexp(logits[r]) - logits[r, target[r]]

for logits [rows, V] (a row stride above V is taken as it is) and int64
targets [rows]: the reference's ``nn.functional.cross_entropy(logits.reshape(
-1, V), y.reshape(-1))`` under bf16 autocast (evals/lm/train.py:74), which
evaluates it in float32 on the upcast logits. Here the logits are read in
their own dtype (no float32 copy) and the arithmetic is float32; the gradient
comes back in the logits' dtype, as autocast's cast would return it. The
loss is float32 and deterministic. A target outside [0, V) that is not
ignore_index gives a NaN loss instead of a device assertion.

Logits whose rows are padded (a row stride a little above V, as the padded
LM head of naju_amd.linear returns them) get their gradient in the same
layout, the padding columns zero, so that the head's backward can read whole
padded rows (``zero_padded_rows``).

CUDA tensors only: there is no other implementation behind this function,
and a missing library raises.
"""
import weakref

import torch

from naju_amd import _lib

_DT = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}


class _Workspace:
    """Per-(device, stream) scratch for the per-row losses, grown on demand
    (the forward overwrites every byte it later reads)."""

    def __init__(self):
        self._bufs = {}

    def get(self, device, stream, nbytes):
        key = (device.index, stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf


_WS = _Workspace()

# row strides up to this many elements above the class count are kept in the
# gradient (padded rows); wider strides (a column slice of a wider tensor)
# get a contiguous gradient
_MAX_PAD = 512

# gradient buffers [rows, ld] whose columns past the class count hold zeros,
# by data pointer (an entry lives as long as its buffer)
_ZERO_PADDED = weakref.WeakValueDictionary()


def _grad_buffer(x, rows, cols):
    """The logits' gradient [rows, cols]: with x's row stride when it pads
    the rows by at most _MAX_PAD elements (a view of a [rows, stride] buffer
    whose padding columns are zero), else contiguous."""
    ld = x.stride(0)
    if ld == cols or ld > cols + _MAX_PAD or rows == 0:
        return torch.empty((rows, cols), dtype=x.dtype, device=x.device)
    buf = torch.empty((rows, ld), dtype=x.dtype, device=x.device)
    buf[:, cols:].zero_()
    _ZERO_PADDED[buf.data_ptr()] = buf
    return buf[:, :cols]


def zero_padded_rows(g, ld):
    """The [rows, ld] buffer behind g [rows, cols] when g is a gradient this
    module wrote with padded rows (columns cols .. ld of the buffer zero),
    else None."""
    if g.dim() != 2 or g.stride() != (ld, 1) or g.shape[1] >= ld:
        return None
    buf = _ZERO_PADDED.get(g.data_ptr())
    if buf is None or tuple(buf.shape) != (g.shape[0], ld) or buf.dtype != g.dtype or buf.device != g.device:
        return None
    return buf


class _CrossEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, target, ignore_index, want_grad):
        rows, cols = x.shape
        dev = x.device
        lse = torch.empty(rows, dtype=torch.float32, device=dev)
        loss = torch.empty((), dtype=torch.float32, device=dev)
        scale = torch.empty((), dtype=torch.float32, device=dev)
        L = _lib.lib()
        stream = torch.cuda.current_stream(dev).cuda_stream
        nbytes = L.naju_xent_workspace_bytes(rows)
        ws = _WS.get(dev, stream, nbytes)
        ctx.dx = None
        if want_grad:
            # the gradient (for dloss = 1) in the same pass over the logits;
            # the backward keeps it when dloss is 1
            dx = _grad_buffer(x, rows, cols)
            _lib.check_loss(L.naju_xent_fwd_grad(
                x.data_ptr(), x.stride(0), target.data_ptr(), rows, cols, _DT[x.dtype], ignore_index, lse.data_ptr(),
                loss.data_ptr(), scale.data_ptr(), dx.data_ptr(), dx.stride(0), _DT[x.dtype], ws.data_ptr(),
                ws.numel(), stream))
            ctx.dx = dx
        else:
            _lib.check_loss(L.naju_xent_fwd(x.data_ptr(), x.stride(0), target.data_ptr(), rows, cols, _DT[x.dtype],
                                            ignore_index, lse.data_ptr(), loss.data_ptr(), scale.data_ptr(),
                                            ws.data_ptr(), ws.numel(), stream))
        ctx.save_for_backward(x, target, lse, scale)
        ctx.ignore_index = ignore_index
        return loss

    @staticmethod
    def backward(ctx, dloss):
        x, target, lse, scale = ctx.saved_tensors
        rows, cols = x.shape
        dloss = dloss.detach().float().contiguous()
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        if ctx.dx is not None:
            # the forward's gradient, rewritten only when dloss is not 1
            # (taken once: a second backward of a retained graph recomputes)
            dx, ctx.dx = ctx.dx, None
            bwd = L.naju_xent_bwd_if_scaled
        else:
            dx = _grad_buffer(x, rows, cols)
            bwd = L.naju_xent_bwd
        _lib.check_loss(bwd(x.data_ptr(), x.stride(0), target.data_ptr(), rows, cols, _DT[x.dtype], ctx.ignore_index,
                            lse.data_ptr(), scale.data_ptr(), dloss.data_ptr(), dx.data_ptr(), dx.stride(0),
                            _DT[x.dtype], stream))
        return dx, None, None, None


def cross_entropy(logits, target, ignore_index=-100):
    if not logits.is_cuda:
        raise RuntimeError("naju_amd.cross_entropy runs on the HIP kernels only: logits must be a CUDA tensor")
    if logits.dim() != 2:
        raise ValueError(f"logits must be [rows, classes], got {tuple(logits.shape)}")
    if target.shape != logits.shape[:1]:
        raise ValueError(f"target must be [{logits.shape[0]}], got {tuple(target.shape)}")
    if logits.dtype not in _DT:
        logits = logits.float()
    if logits.stride(1) != 1 or logits.stride(0) < logits.shape[1]:
        logits = logits.contiguous()
    target = target.to(device=logits.device, dtype=torch.int64).contiguous()
    # a backward will follow (a graph is being recorded): the forward also
    # writes the gradient
    want_grad = torch.is_grad_enabled() and logits.requires_grad
    return _CrossEntropy.apply(logits, target, int(ignore_index), want_grad)
