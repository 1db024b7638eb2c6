"""Gradient routing without extra copies or additions.

split(): splits whose consumers write their gradients in place.

Autograd's backward of ``t.split(sizes, -1)`` concatenates the pieces'
gradients into a new tensor of t's shape: one more read and write of t's
size. ``split(t, sizes)`` returns the same views, tagged with a GradSink.
A HIP kernel that consumes a piece (the depthwise convolution's x or add,
the readout's z) asks the sink for that piece's slice of one gradient
buffer of t's shape and writes its gradient there, with t's row stride.
The split's backward then returns that buffer itself, copying in only the
pieces whose gradient arrived in another tensor (a piece that also had
other consumers, whose gradients autograd summed elsewhere, or one whose
consumer does not use the sink) and zero-filling pieces without a gradient.

fanout(): aliases of one tensor for several consumers whose gradients
collect in one buffer: the first consumer to get there writes it, later ones
add into it in place (the depthwise convolution with NAJU_DWCONV_ACCUM_DX, a
GEMM with addmm_), and the fan-out returns the buffer as the tensor's
gradient, where autograd would otherwise add the consumers' separate
gradients one by one (one read-read-write pass of the tensor per addition).
"""
import torch


class GradSink:
    """One gradient buffer, allocated at the first request of a backward."""

    def __init__(self, like):
        self.shape, self.dtype, self.device = like.shape, like.dtype, like.device
        self.buf = None

    def slice(self, col0, width):
        if self.buf is None:
            self.buf = torch.empty(self.shape, dtype=self.dtype, device=self.device)
        return self.buf[..., col0:col0 + width]


class _Split(torch.autograd.Function):
    @staticmethod
    def forward(ctx, t, sizes, sink):
        ctx.sizes = sizes
        ctx.sink = sink
        return t.split(list(sizes), dim=-1)

    @staticmethod
    def backward(ctx, *grads):
        sink, sizes = ctx.sink, ctx.sizes
        if sink.buf is None:
            parts = [g if g is not None else torch.zeros(sink.shape[:-1] + (w,), dtype=sink.dtype, device=sink.device)
                     for g, w in zip(grads, sizes)]
            return torch.cat(parts, dim=-1), None, None
        buf = sink.buf
        sink.buf = None  # a later backward through the same graph allocates anew
        col = 0
        for g, w in zip(grads, sizes):
            dst = buf[..., col:col + w]
            if g is None:
                dst.zero_()
            elif g.data_ptr() != dst.data_ptr() or g.stride() != dst.stride() or g.dtype != dst.dtype:
                dst.copy_(g)
            col += w
        return buf, None, None


def split(t, sizes):
    """t.split(sizes, -1), with the pieces tagged for in-place gradients."""
    sink = GradSink(t)
    pieces = _Split.apply(t, tuple(int(w) for w in sizes), sink)
    col = 0
    for p, w in zip(pieces, sizes):
        p._naju_sink = (sink, col)
        col += int(w)
    return pieces


def sink_of(t):
    """(sink, first column) of a piece returned by split(), else None."""
    return getattr(t, "_naju_sink", None) if t is not None else None


_ZEROS = {}


def _zero(dtype, device):
    """A cached 0-dim zero per (dtype, device): the storage of every marker."""
    key = (dtype, device)
    z = _ZEROS.get(key)
    if z is None:
        z = _ZEROS[key] = torch.zeros((), dtype=dtype, device=device)
    return z


class AccumSink:
    """One gradient buffer that the consumers of one tensor fill in turn,
    instead of each returning its own gradient for autograd to add: the
    first to call target() writes the buffer, the later ones add into it
    (kernels and GEMMs with an accumulating form), and each returns
    marker() -- a zero of the tensor's shape without storage -- in place of
    its gradient. A consumer without an accumulating form returns its
    gradient as usual, and the fan-out adds it."""

    def __init__(self, like):
        self.shape, self.dtype, self.device = like.shape, like.dtype, like.device
        self.buf = None
        self._zero = _zero(like.dtype, like.device)

    def target(self):
        """(buffer, accumulate): the buffer, and whether it already holds an
        earlier consumer's gradient (add into it) or not (write it)."""
        if self.buf is None:
            self.buf = torch.empty(self.shape, dtype=self.dtype, device=self.device)
            return self.buf, False
        return self.buf, True

    def marker(self):
        return self._zero.expand(self.shape)

    def is_marker(self, g):
        return g.data_ptr() == self._zero.data_ptr() and all(s == 0 for s in g.stride())


class _Fanout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, t, n, sink):
        ctx.set_materialize_grads(False)
        ctx.sink = sink
        return tuple(t.view_as(t) for _ in range(n))

    @staticmethod
    def backward(ctx, *grads):
        sink = ctx.sink
        buf, sink.buf = sink.buf, None  # a later backward through the same graph allocates anew
        own = buf is not None
        for g in grads:
            if g is None or sink.is_marker(g):
                continue
            if buf is None:
                buf = g
            elif own:
                buf.add_(g)
            else:
                buf = buf + g
        return buf, None, None


def fanout(t, n):
    """n aliases of t, each for one consumer, tagged with one AccumSink:
    consumers that know the sink (acc_sink_of) leave their gradients in its
    buffer, and the fan-out's backward returns that buffer as t's gradient
    (plus any gradient returned the usual way)."""
    sink = AccumSink(t)
    outs = _Fanout.apply(t, int(n), sink)
    for o in outs:
        o._naju_acc = sink
    return outs


def acc_sink_of(t):
    """The AccumSink of an alias returned by fanout(), else None."""
    return getattr(t, "_naju_acc", None) if t is not None else None
