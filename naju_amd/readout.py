"""Readout epilogue of the mixer on the HIP kernels of include/naju_mixer.h.

``readout(cx, h, z, D, scale, out_dtype=None)``

    y = (cx * scale + D * h) * SiLU(z)

with cx, h [B, T, C] (C contiguous), z [B, T, C] whose row stride may exceed
C (the second half of the in_proj output goes in without a copy) and D [C].
This is naju/mixer.py:123-124 (the scan's output scaled by 1/sqrt(N), the D
skip, the z gate) as one kernel, and its backward (dcx, dh, dz, dD; dD
summed in a fixed order) as another. CUDA tensors only: a missing library
raises.
"""
import torch

from naju_amd import _lib
from naju_amd.dwconv import _DT, _WS, _ptr
from naju_amd.gradsink import sink_of


def _rows_of(t):
    """[B, T, C] view -> (tensor with C contiguous and rows collapsible, row stride)."""
    B, T, C = t.shape
    if t.stride(2) != 1 or t.stride(0) != T * t.stride(1) or t.stride(1) < C:
        t = t.contiguous()
    return t, t.stride(1)


class _Readout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cx, h, z, Dv, scale, out_dtype, z_sink, dh_elsewhere):
        B, T, C = h.shape
        z, z_ld = _rows_of(z)
        y = torch.empty((B, T, C), dtype=out_dtype, device=h.device)
        L = _lib.lib()
        stream = torch.cuda.current_stream(h.device).cuda_stream
        _lib.check_mixer(L.naju_readout_fwd(
            _ptr(cx), _ptr(h), _ptr(z), z_ld, _ptr(Dv), float(scale), _ptr(y), B * T, C,
            _DT[cx.dtype], _DT[h.dtype], _DT[z.dtype], _DT[out_dtype], stream))
        ctx.save_for_backward(cx, h, z, Dv)
        ctx.scale = float(scale)
        ctx.z_sink = z_sink  # z is a piece of a gradsink.split(): dz goes into its buffer
        ctx.dh_elsewhere = dh_elsewhere
        return y

    @staticmethod
    def backward(ctx, dy):
        cx, h, z, Dv = ctx.saved_tensors
        B, T, C = h.shape
        if dy.dtype not in _DT:
            dy = dy.float()
        dy = dy.contiguous()
        need_cx, need_h, need_z, need_D = ctx.needs_input_grad[:4]
        dcx = torch.empty((B, T, C), dtype=cx.dtype, device=h.device) if need_cx else None
        need_h = need_h and not ctx.dh_elsewhere
        dh = torch.empty((B, T, C), dtype=h.dtype, device=h.device) if need_h else None
        dz = None
        if need_z:
            if ctx.z_sink is not None:
                sink, col = ctx.z_sink
                dz = sink.slice(col, C)
            else:
                dz = torch.empty((B, T, C), dtype=z.dtype, device=h.device)
        dD = torch.empty((C,), dtype=torch.float32, device=h.device) if need_D else None
        if any(t is not None for t in (dcx, dh, dz, dD)):
            L = _lib.lib()
            stream = torch.cuda.current_stream(h.device).cuda_stream
            nbytes = L.naju_readout_workspace_bytes(B * T, C)
            ws = _WS.get(h.device, stream, nbytes)
            _lib.check_mixer(L.naju_readout_bwd(
                _ptr(cx), _ptr(h), _ptr(z), z.stride(1), _ptr(Dv), ctx.scale, _ptr(dy), _ptr(dcx), _ptr(dh),
                _ptr(dz), dz.stride(1) if dz is not None else C, _ptr(dD), B * T, C, _DT[cx.dtype], _DT[h.dtype],
                _DT[z.dtype], _DT[dy.dtype], _DT[cx.dtype], _DT[h.dtype], _DT[z.dtype], _ptr(ws), ws.numel(),
                stream))
        return dcx, dh, dz, dD, None, None, None, None


def readout(cx, h, z, D, scale, out_dtype=None, dh_elsewhere=False):
    """dh_elsewhere: h's gradient through the D h term is formed by another
    consumer of h (the scan's backward with du_skip = D / scale), so this
    backward leaves it out and returns no gradient for h."""
    if not h.is_cuda:
        raise RuntimeError("naju_amd.readout runs on the HIP kernels only: h must be a CUDA tensor")
    if h.dim() != 3 or cx.shape != h.shape or z.shape != h.shape:
        raise ValueError(f"cx, h and z must share one [B, T, C] shape, got {tuple(cx.shape)}, "
                         f"{tuple(h.shape)}, {tuple(z.shape)}")
    if D.shape != (h.shape[2],):
        raise ValueError(f"D must be [C] = [{h.shape[2]}], got {tuple(D.shape)}")
    cx = (cx if cx.dtype in _DT else cx.float()).contiguous()
    h = (h if h.dtype in _DT else h.float()).contiguous()
    z_sink = sink_of(z)
    if z.dtype not in _DT:
        z, z_sink = z.float(), None
    Dv = D if D.dtype == torch.float32 else D.float()
    if out_dtype is None:
        out_dtype = torch.promote_types(torch.promote_types(cx.dtype, h.dtype), Dv.dtype)
    return _Readout.apply(cx, h, z, Dv.contiguous(), float(scale), out_dtype, z_sink, bool(dh_elsewhere))
