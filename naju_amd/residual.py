"""The pre-norm block's residual add with dropout, u + Dropout(p)(mix)
(reference naju/mixer.py:131-144, NajuBlock's drop and residual), on the
HIP kernels of include/naju_mixer.h: one pass forward (read u and mix,
write the sum) and one pass for the dropout's backward (read the float32
gradient, write mix's gradient), where torch runs a dropout, a mixed-dtype
addition, a cast and a masked scale.

The mask is not stored: the kernels draw the keep decision of element i
from (seed, i), the backward again from the same seed. The seed is drawn
from torch's CUDA generator on the device (no synchronisation), so
torch.manual_seed makes the masks repeatable and activation checkpointing,
which saves and restores that generator's state, replays them. Kept
elements are scaled by 1 / (1 - p) and rounded to mix's dtype before the
addition, as the reference's bf16 dropout output is.
"""
import torch

from naju_amd import _lib

_DT = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}


class _ResidualDropout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, u, mix, p, seed):
        out = torch.empty_like(u)
        L = _lib.lib()
        stream = torch.cuda.current_stream(u.device).cuda_stream
        _lib.check_mixer(L.naju_residual_dropout_fwd(
            u.data_ptr(), mix.data_ptr(), seed.data_ptr() if seed is not None else None, float(p), out.data_ptr(),
            u.numel(), _DT[mix.dtype], stream))
        ctx.p = float(p)
        ctx.mix_dtype = mix.dtype
        ctx.save_for_backward(seed if seed is not None else torch.empty(0, device=u.device))
        ctx.has_seed = seed is not None
        return out

    @staticmethod
    def backward(ctx, g):
        (seed,) = ctx.saved_tensors
        g = g.float().contiguous()
        if g.data_ptr() % 16 != 0:
            g = g.clone()
        dmix = None
        if ctx.needs_input_grad[1]:
            dmix = torch.empty(g.shape, dtype=ctx.mix_dtype, device=g.device)
            L = _lib.lib()
            stream = torch.cuda.current_stream(g.device).cuda_stream
            _lib.check_mixer(L.naju_dropout_bwd(
                g.data_ptr(), seed.data_ptr() if ctx.has_seed else None, ctx.p, dmix.data_ptr(), g.numel(),
                _DT[ctx.mix_dtype], stream))
        return (g if ctx.needs_input_grad[0] else None), dmix, None, None


def supported(u, mix):
    return (u.is_cuda and u.dtype == torch.float32 and mix.dtype in _DT and mix.shape == u.shape
            and u.is_contiguous() and mix.is_contiguous())


def residual_dropout(u, mix, p, seed=None):
    """u + Dropout(p)(mix) (training-mode dropout; p = 0 is the plain sum)
    for float32 u and mix of u's shape in float32 / bfloat16 / float16.
    seed: a one-element int64 CUDA tensor to draw the mask from (a caller
    with several dropouts draws all their seeds in one call), else drawn
    here from torch's generator."""
    if not supported(u, mix):
        raise RuntimeError("naju_amd.residual_dropout: u must be a contiguous float32 CUDA tensor and mix a "
                           "contiguous CUDA tensor of u's shape in float32, bfloat16 or float16")
    p = float(p)
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout probability must be in [0, 1), got {p}")
    if p == 0.0:
        seed = None
    elif seed is None:
        seed = draw_seeds(1, u.device)
    elif not (seed.is_cuda and seed.dtype == torch.int64 and seed.numel() == 1):
        raise ValueError("naju_amd.residual_dropout: seed must be a one-element int64 CUDA tensor")
    return _ResidualDropout.apply(u, mix, p, seed)


def draw_seeds(n, device):
    """n dropout seeds from torch's generator in one call (int64 [n])."""
    return torch.randint(0, 2 ** 62, (n,), device=device, dtype=torch.int64)
