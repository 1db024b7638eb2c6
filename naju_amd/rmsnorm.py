"""RMSNorm of the Naju blocks on the HIP kernels of include/naju_mixer.h.

``rms_norm(x, weight, eps, out_dtype=None)``

    y = (weight * x) * rsqrt(mean(x^2, -1) + eps)

over the last axis, the reference's RMSNorm (naju/mixer.py:51-58) in one
kernel each way: the forward reads x once and writes y (in ``out_dtype``:
under autocast the consumer is a bf16 GEMM, so y is written in bf16 with the
values autocast's own cast would give), the backward reads x and dy once and
writes dx, with dweight summed over rows in a fixed order (deterministic).

``supported(x)`` says whether the kernels serve x (CUDA, float32 or bfloat16,
last axis a multiple of 4 up to 4096, 16-byte aligned); the module in
naju_amd.mixer uses the reference's torch formula otherwise.
"""
import torch

from naju_amd import _lib

_DT = {torch.float32: _lib.DT_F32, torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}


class _Workspace:
    """Per-(device, stream) scratch for the dweight partial sums, grown on
    demand (the backward overwrites every byte it later reads)."""

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


def supported(x):
    d = x.shape[-1] if x.dim() > 0 else 0
    return (x.is_cuda and x.dtype in (torch.float32, torch.bfloat16) and d % 4 == 0 and 0 < d <= 4096
            and x.is_contiguous() and x.data_ptr() % 16 == 0)


class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps, out_dtype):
        d = x.shape[-1]
        rows = x.numel() // d
        y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check_mixer(L.naju_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), eps, y.data_ptr(), rstd.data_ptr(), rows, d,
                                            _DT[x.dtype], _DT[out_dtype], stream))
        ctx.save_for_backward(x, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        d = x.shape[-1]
        rows = x.numel() // d
        if dy.dtype not in _DT:
            dy = dy.float()
        dy = dy.contiguous()
        if dy.data_ptr() % 16 != 0:
            dy = dy.clone()
        dx = torch.empty_like(x)
        need_w = ctx.needs_input_grad[1]
        dw = torch.empty(d, dtype=torch.float32, device=x.device) if need_w else None
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        nbytes = L.naju_rmsnorm_workspace_bytes(rows, d)
        ws = _WS.get(x.device, stream, nbytes)
        _lib.check_mixer(L.naju_rmsnorm_bwd(x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dx.data_ptr(),
                                            dw.data_ptr() if dw is not None else None, rows, d, _DT[x.dtype],
                                            _DT[dy.dtype], _DT[x.dtype], ws.data_ptr(), ws.numel(), stream))
        return dx, dw, None, None


def rms_norm(x, weight, eps, out_dtype=None):
    if not supported(x):
        raise RuntimeError("naju_amd.rms_norm: x must be a contiguous, 16-byte aligned CUDA tensor in float32 or "
                           f"bfloat16 with a last axis that is a multiple of 4 up to 4096 (got {x.dtype}, "
                           f"{tuple(x.shape)})")
    if out_dtype is None:
        out_dtype = x.dtype
    w = weight
    if w.dtype != torch.float32:
        w = w.float()
    w = w.contiguous()
    if w.data_ptr() % 16 != 0:
        w = w.clone()
    return _RMSNorm.apply(x, w, float(eps), out_dtype)


class _RMSNormFork(torch.autograd.Function):
    """(x, rms_norm(x)): the pre-norm block's residual stream and its norm
    from one input, so that the backward receives both gradients and adds
    them in the norm's pass (naju_rmsnorm_bwd_add) instead of autograd's
    separate addition."""

    @staticmethod
    def forward(ctx, x, w, eps, out_dtype):
        ctx.set_materialize_grads(False)
        d = x.shape[-1]
        rows = x.numel() // d
        y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        _lib.check_mixer(L.naju_rmsnorm_fwd(x.data_ptr(), w.data_ptr(), eps, y.data_ptr(), rstd.data_ptr(), rows, d,
                                            _DT[x.dtype], _DT[out_dtype], stream))
        ctx.save_for_backward(x, w, rstd)
        return x.view_as(x), y

    @staticmethod
    def backward(ctx, dres, dy):
        x, w, rstd = ctx.saved_tensors
        need_w = ctx.needs_input_grad[1]
        if dy is None:
            dw = torch.zeros(x.shape[-1], dtype=torch.float32, device=x.device) if need_w else None
            return dres, dw, None, None
        d = x.shape[-1]
        rows = x.numel() // d
        if dy.dtype not in _DT:
            dy = dy.float()
        dy = dy.contiguous()
        if dy.data_ptr() % 16 != 0:
            dy = dy.clone()
        if dres is not None:
            if dres.dtype != x.dtype:
                dres = dres.to(x.dtype)
            dres = dres.contiguous()
            if dres.data_ptr() % 16 != 0:
                dres = dres.clone()
        dx = torch.empty_like(x)
        dw = torch.empty(d, dtype=torch.float32, device=x.device) if need_w else None
        L = _lib.lib()
        stream = torch.cuda.current_stream(x.device).cuda_stream
        ws = _WS.get(x.device, stream, L.naju_rmsnorm_workspace_bytes(rows, d))
        _lib.check_mixer(L.naju_rmsnorm_bwd_add(
            x.data_ptr(), w.data_ptr(), rstd.data_ptr(), dy.data_ptr(), dres.data_ptr() if dres is not None else None,
            dx.data_ptr(), dw.data_ptr() if dw is not None else None, rows, d, _DT[x.dtype], _DT[dy.dtype],
            _DT[x.dtype], ws.data_ptr(), ws.numel(), stream))
        return dx, dw, None, None


def rms_norm_fork(x, weight, eps, out_dtype=None):
    """(x, rms_norm(x, weight, eps, out_dtype)) with the two gradients of x
    added in the norm's backward pass; x as rms_norm serves it."""
    if not supported(x):
        raise RuntimeError("naju_amd.rms_norm_fork serves what rms_norm serves")
    if out_dtype is None:
        out_dtype = x.dtype
    w = weight if weight.dtype == torch.float32 else weight.float()
    w = w.contiguous()
    if w.data_ptr() % 16 != 0:
        w = w.clone()
    return _RMSNormFork.apply(x, w, float(eps), out_dtype)
