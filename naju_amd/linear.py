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

from naju_amd import _lib
from naju_amd.gradsink import acc_sink_of

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
    @staticmethod
    def forward(ctx, x, weight, dtype, x_acc):
        xb = x if x.dtype == dtype else x.to(dtype)
        wb = weight.to(dtype)
        ctx.save_for_backward(xb, wb)
        ctx.x_dtype, ctx.w_dtype = x.dtype, weight.dtype
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
        if ctx.needs_input_grad[1]:
            dw = weight_grad(dy2.contiguous(), xb.reshape(-1, n_in))
            if dw.dtype != ctx.w_dtype:
                dw = dw.to(ctx.w_dtype)
        return dx, dw, None, None


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
    x_acc = acc_sink_of(x)
    if x_acc is not None and not x.is_contiguous():
        x_acc = None
    return _Linear.apply(x, weight, dt, x_acc)
