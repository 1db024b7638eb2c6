"""Linear layers of the mixer with a split-K weight gradient.

``linear(x, weight)`` is ``F.linear(x, weight)`` (no bias) computed in x's
16-bit dtype, as bf16 autocast computes the reference's nn.Linear layers
(naju/mixer.py:73-95): the forward and the input gradient are the same GEMMs
torch runs there. The weight gradient dW = dY^T X [out, in] differs: its
contraction runs over every token of the batch (16384 in the LM step) while
the output is small (768 x 1536 for out_proj: 72 tiles of 128 x 128 for 256
compute units), so a single GEMM leaves most of the GPU idle. Here the
tokens are split into S equal parts, the S partial products run as one
batched GEMM with float32 output, and the parts are added in float32
in part order (naju_sum_parts). dW comes out in float32, the parameters' dtype, without the
bfloat16 rounding and the cast back that autocast's backward applies.

CUDA tensors in float16 / bfloat16 only (the callers fall back to nn.Linear
otherwise).
"""
import torch
import torch.nn.functional as F

from naju_amd import _lib, wcast
from naju_amd.gradsink import acc_sink_of
from naju_amd.xent import zero_padded_rows

# output tiles (128 x 128) times parts kept at or below this: about two
# waves of workgroups over the 256 compute units
_TILE_BUDGET = 640
_MAX_PARTS = 16
_MIN_ROWS = 512


def _parts(K, M, N):
    """Token parts S for dW [M, N] over K tokens: the largest power of two
    (at most _MAX_PARTS) whose S x (128 x 128 output tiles) stays within
    _TILE_BUDGET, with K divisible by S and at least _MIN_ROWS tokens per
    part."""
    tiles = ((M + 127) // 128) * ((N + 127) // 128)
    s = 1
    while (s * 2 <= _MAX_PARTS and tiles * s * 2 <= _TILE_BUDGET and K % (s * 2) == 0
           and K // (s * 2) >= _MIN_ROWS):
        s *= 2
    return s


def weight_grad(dy, x):
    """dY^T X in float32 for dy [K, M] and x [K, N] (16-bit, row-major)."""
    K, M = dy.shape
    N = x.shape[1]
    s = _parts(K, M, N)
    if s == 1:
        return torch.mm(dy.t(), x, out_dtype=torch.float32)
    # the left operand is the transposed view, the right one is contiguous
    part = torch.bmm(dy.view(s, K // s, M).transpose(1, 2), x.view(s, K // s, N), out_dtype=torch.float32)
    # the parts added in part order (one pass over them, naju_sum_parts)
    out = torch.empty(M, N, dtype=torch.float32, device=dy.device)
    L = _lib.lib()
    _lib.check_mixer(L.naju_sum_parts(part.data_ptr(), s, M * N, out.data_ptr(),
                                      torch.cuda.current_stream(dy.device).cuda_stream))
    return out


class _Linear(torch.autograd.Function):
    """x @ W^T with W the row-wise concatenation of weights (one GEMM for
    layers that read the same x), wb its 16-bit copy when one is at hand
    (naju_amd.wcast), else cast here."""

    @staticmethod
    def forward(ctx, x, dtype, x_acc, wb, *weights):
        xb = x if x.dtype == dtype else x.to(dtype)
        if wb is None:
            wb = weights[0].to(dtype) if len(weights) == 1 else torch.cat([w.to(dtype) for w in weights], 0)
        ctx.save_for_backward(xb, wb)
        ctx.x_dtype, ctx.w_dtypes = x.dtype, [w.dtype for w in weights]
        ctx.rows = [w.shape[0] for w in weights]
        # x is a gradsink.fanout() alias (in the compute dtype): dx is
        # written into, or added to, the fan-out's buffer
        ctx.x_acc = x_acc if xb is x else None
        return F.linear(xb, wb)

    @staticmethod
    def backward(ctx, dy):
        xb, wb = ctx.saved_tensors
        n_out, n_in = wb.shape
        dy2 = dy.reshape(-1, n_out)
        if dy2.dtype != wb.dtype:
            dy2 = dy2.to(wb.dtype)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            if ctx.x_acc is not None:
                buf, accumulate = ctx.x_acc.target()
                b2 = buf.view(-1, n_in)
                if accumulate:
                    b2.addmm_(dy2, wb)
                else:
                    torch.mm(dy2, wb, out=b2)
                dx = ctx.x_acc.marker()
            else:
                dx = torch.mm(dy2, wb).view(*dy.shape[:-1], n_in)
                if dx.dtype != ctx.x_dtype:
                    dx = dx.to(ctx.x_dtype)
        dws = [None] * len(ctx.rows)
        if any(ctx.needs_input_grad[4:]):
            dw = weight_grad(dy2.contiguous(), xb.reshape(-1, n_in))
            # each weight's rows of the product (contiguous views)
            for i, d in enumerate(dw.split(ctx.rows, 0) if len(ctx.rows) > 1 else (dw,)):
                if ctx.needs_input_grad[4 + i]:
                    dws[i] = d if d.dtype == ctx.w_dtypes[i] else d.to(ctx.w_dtypes[i])
        return (dx, None, None, None, *dws)


# the LM head's vocabulary rows are padded to a multiple of this
HEAD_ALIGN = 128


class _Head(torch.autograd.Function):
    """logits = x W^T for a vocabulary-sized W [V, d], with W's 16-bit copy
    padded by zero rows to Vp, a multiple of HEAD_ALIGN: the GEMMs then run on
    aligned [rows, Vp] operands (a vocabulary of 50257 leaves every row of
    the logits and of their gradient at an odd offset, which the library's
    fast kernels do not take). The output is the [..., V] view of the
    [rows, Vp] product, so it holds the same values as F.linear's logits. In
    the backward, a gradient that naju_amd.xent.cross_entropy wrote in that
    padded layout (padding columns zero) is used whole: dx = G W_pad over
    K = Vp, dW = G^T x in float32 (the first V rows of the [Vp, d] product);
    any other gradient takes the unpadded GEMMs (K = V). dW comes out in
    float32, the parameter's dtype, as for the split-K weight gradients."""

    @staticmethod
    def forward(ctx, x, weight, dtype, wp, tied):
        ctx.tied = tied
        V, d = weight.shape
        Vp = -(-V // HEAD_ALIGN) * HEAD_ALIGN
        if wp is None or tuple(wp.shape) != (Vp, d):
            wp = torch.empty((Vp, d), dtype=dtype, device=weight.device)
            if Vp > V:
                wp[V:].zero_()
            wp[:V].copy_(weight)
        x2 = x.reshape(-1, d)
        if x2.dtype != dtype:
            x2 = x2.to(dtype)
        out = torch.mm(x2, wp.t())
        ctx.save_for_backward(x2, wp)
        ctx.V, ctx.x_shape, ctx.x_dtype, ctx.w_dtype = V, x.shape, x.dtype, weight.dtype
        return out[:, :V].view(*x.shape[:-1], V)

    @staticmethod
    def backward(ctx, dl):
        x2, wp = ctx.saved_tensors
        V, Vp = ctx.V, wp.shape[0]
        rows = x2.shape[0]
        g = dl.reshape(rows, V)
        if g.dtype != wp.dtype:
            g = g.to(wp.dtype)
        full = zero_padded_rows(g, Vp) if Vp > V else None
        gk, wk = (g, wp[:V]) if full is None else (full, wp)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = torch.mm(gk, wk).view(ctx.x_shape)
            if dx.dtype != ctx.x_dtype:
                dx = dx.to(ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            dw = torch.mm(gk.t(), x2, out_dtype=torch.float32)[:V]
            if dw.dtype != ctx.w_dtype:
                dw = dw.to(ctx.w_dtype)
            if ctx.tied is not None and dw.dtype == torch.float32:
                # the tied embedding's backward adds its rows into it and
                # returns the sum (naju_amd.embed.TiedGrad)
                ctx.tied.put(dw)
                dw = None
        return dx, dw, None, None, None


def lm_head(x, weight, tied=None):
    """F.linear(x, weight) for the LM head (weight [V, d], no bias) in
    compute_dtype(x) (which must not be None), through the padded GEMMs of
    _Head; the logits are a [..., V] view with row stride Vp. tied: a
    naju_amd.embed.TiedGrad that takes the weight's gradient for the tied
    embedding's backward."""
    dt = compute_dtype(x)
    if dt is None:
        raise ValueError("naju_amd.linear.lm_head serves CUDA tensors computed in float16 / bfloat16")
    return _Head.apply(x, weight, dt, wcast.lookup((weight,), dt), tied)


def compute_dtype(x):
    """The 16-bit dtype a linear layer on x computes in (the autocast dtype
    when autocast is on, else x's own), or None when it is not 16-bit or x
    is not a CUDA tensor."""
    if not x.is_cuda:
        return None
    dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
    return dt if dt in (torch.bfloat16, torch.float16) else None


def linear(x, weight):
    """x @ weight^T in compute_dtype(x) (which must not be None), with the
    split-K float32 weight gradient."""
    dt = compute_dtype(x)
    if dt is None:
        raise ValueError("naju_amd.linear.linear serves CUDA tensors computed in float16 / bfloat16")
    return linear_cat(x, (weight,))


def linear_cat(x, weights):
    """x @ cat(weights, 0)^T as linear() (one GEMM, one split-K weight
    gradient), each weight getting its rows of the gradient; the 16-bit
    concatenation comes from naju_amd.wcast when the group is active there."""
    dt = compute_dtype(x)
    if dt is None:
        raise ValueError("naju_amd.linear.linear serves CUDA tensors computed in float16 / bfloat16")
    x_acc = acc_sink_of(x)
    if x_acc is not None and not x.is_contiguous():
        x_acc = None
    weights = tuple(weights)
    return _Linear.apply(x, dt, x_acc, wcast.lookup(weights, dt), *weights)
