"""AdamW with the training loop's gradient clipping on the HIP optimizer
kernels (include/naju_optim.h).

``AdamW`` is torch.optim.AdamW's update (amsgrad and maximize off) for
float32 CUDA parameters: the same hyper-parameters, param groups and
per-parameter state ('step', 'exp_avg', 'exp_avg_sq'; state dicts load in
either direction), applied to every tensor in one multi-tensor launch.
``step(max_grad_norm=c)`` also does what the reference's loop does before
its step (/root/reference/evals/lm/train.py:79-80),

    nn.utils.clip_grad_norm_(params, c); opt.step()

with the gradients scaled inside the update instead of in place: one pass
over the gradients for the global norm, the coefficient kept on the device
(no host sync), and the update reading it. The gradients themselves are left
unscaled; ``grad_norm`` holds the total norm (clip_grad_norm_'s return value)
as a device tensor.

The tensor table the kernels read (pointers, sizes, chunk map) is uploaded
when the set of tensors or their addresses change, which in a steady
training loop is the first step only.
"""
import ctypes
import math

import numpy as np
import torch

from naju_amd import _lib

CHUNK = 8192      # NAJU_OPTIM_CHUNK
MAX_GROUPS = 16   # NAJU_OPTIM_MAX_GROUPS

# naju_adamw_tensor
TENSOR_DTYPE = np.dtype([("param", "<u8"), ("grad", "<u8"), ("exp_avg", "<u8"), ("exp_avg_sq", "<u8"),
                         ("numel", "<i8"), ("first_chunk", "<i8"), ("group", "<i4"), ("reserved", "<i4")])
assert TENSOR_DTYPE.itemsize == 56


class _Group(ctypes.Structure):
    """naju_adamw_group"""
    _fields_ = [(n, ctypes.c_float) for n in ("decay", "beta1", "one_minus_beta1", "beta2", "one_minus_beta2",
                                               "step_size", "bias_correction2_sqrt", "eps")]


def build_table(entries):
    """The kernels' table for entries of (param_ptr, grad_ptr, exp_avg_ptr,
    exp_avg_sq_ptr, numel, group): the naju_adamw_tensor records and the
    chunk -> tensor map (tensor i owns ceil(numel_i / CHUNK) consecutive
    chunks from its first_chunk). Entries with numel 0 must be left out.
    Returns (records, chunk_map)."""
    n = len(entries)
    rec = np.zeros(n, dtype=TENSOR_DTYPE)
    if n == 0:
        return rec, np.zeros(0, dtype=np.int32)
    cols = list(zip(*entries))
    for name, col in zip(("param", "grad", "exp_avg", "exp_avg_sq", "numel", "group"), cols):
        rec[name] = col
    if (rec["numel"] <= 0).any():
        raise ValueError("empty tensors have no chunks; leave them out of the table")
    chunks = (rec["numel"] + CHUNK - 1) // CHUNK
    rec["first_chunk"] = np.concatenate(([0], np.cumsum(chunks)[:-1]))
    return rec, np.repeat(np.arange(n, dtype=np.int32), chunks)


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        if not 0.0 <= lr:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= eps:
            raise ValueError(f"Invalid epsilon value: {eps}")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"Invalid beta parameters: {betas}")
        if not 0.0 <= weight_decay:
            raise ValueError(f"Invalid weight_decay value: {weight_decay}")
        # torch.optim.AdamW's group keys, so that either class loads the
        # other's state dict; the switches are fixed to what is served here
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, amsgrad=False, maximize=False,
                        foreach=None, capturable=False, differentiable=False, fused=None)
        super().__init__(params, defaults)
        self._key = None
        self._dev_table = None
        self._n_tensors = 0
        self._n_chunks = 0
        self._ws = None
        self.grad_norm = None

    def _check_group(self, group):
        if group.get("amsgrad") or group.get("maximize"):
            raise NotImplementedError("naju_amd.optim.AdamW serves amsgrad=False, maximize=False")

    def _upload(self, entries, device):
        key = tuple(entries)
        if key == self._key:
            return
        rec, cmap = build_table(entries)
        nb = rec.nbytes
        off = (nb + 255) // 256 * 256
        buf = np.zeros(off + cmap.nbytes, dtype=np.uint8)
        buf[:nb] = rec.view(np.uint8)
        buf[off:] = cmap.view(np.uint8)
        host = torch.from_numpy(buf).pin_memory()
        self._dev_table = host.to(device, non_blocking=True)
        self._map_off = off
        self._n_tensors = len(entries)
        self._n_chunks = int(cmap.size)
        self._key = key

    @torch.no_grad()
    def step(self, closure=None, max_grad_norm=None):
        """One AdamW step over every parameter with a gradient; with
        max_grad_norm, first clip the gradients' global L2 norm to it (inside
        the update) and record the norm in ``grad_norm``."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        entries, combos, combo_idx, device = [], [], {}, None
        for gi, group in enumerate(self.param_groups):
            self._check_group(group)
            beta1, beta2 = group["betas"]
            for p in group["params"]:
                g = p.grad
                if g is None:
                    continue
                if g.is_sparse:
                    raise RuntimeError("naju_amd.optim.AdamW does not support sparse gradients")
                if not (p.is_cuda and p.dtype == torch.float32 and g.dtype == torch.float32
                        and p.is_contiguous() and g.is_contiguous()):
                    raise ValueError("naju_amd.optim.AdamW serves contiguous float32 CUDA parameters and gradients")
                if device is None:
                    device = p.device
                elif p.device != device:
                    raise ValueError("naju_amd.optim.AdamW: every parameter on one device")
                st = self.state[p]
                if len(st) == 0:
                    st["step"] = torch.tensor(0.0)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.contiguous_format)
                st["step"] += 1
                t = float(st["step"])
                ci = combo_idx.get((gi, t))
                if ci is None:
                    ci = combo_idx[(gi, t)] = len(combos)
                    # in double, rounded once (as torch forms them in Python)
                    lr = group["lr"]
                    combos.append((1.0 - lr * group["weight_decay"], beta1, 1.0 - beta1, beta2, 1.0 - beta2,
                                   lr / (1.0 - beta1 ** t), math.sqrt(1.0 - beta2 ** t), group["eps"]))
                if p.numel() > 0:
                    entries.append((p.data_ptr(), g.data_ptr(), st["exp_avg"].data_ptr(),
                                    st["exp_avg_sq"].data_ptr(), p.numel(), ci))
        if not entries:
            if max_grad_norm is not None:
                self.grad_norm = torch.zeros((), device=device) if device is not None else torch.tensor(0.0)
            return loss
        if len(combos) > MAX_GROUPS:
            raise ValueError(f"naju_amd.optim.AdamW: at most {MAX_GROUPS} (param group, step) combinations per step")
        L = _lib.lib()
        self._upload(entries, device)
        tab = self._dev_table.data_ptr()
        cmap = tab + self._map_off
        stream = torch.cuda.current_stream(device).cuda_stream
        coef = None
        if max_grad_norm is not None:
            nb = L.naju_grad_norm_workspace_bytes(self._n_chunks)
            if self._ws is None or self._ws.numel() < nb:
                self._ws = torch.empty(nb, dtype=torch.uint8, device=device)
            out = torch.empty(2, device=device)
            _lib.check_optim(L.naju_grad_norm(tab, cmap, self._n_tensors, self._n_chunks, float(max_grad_norm),
                                              out.data_ptr(), out.data_ptr() + 4, self._ws.data_ptr(),
                                              self._ws.numel(), stream))
            self.grad_norm = out[0]
            coef = out.data_ptr() + 4
        groups = (_Group * len(combos))(*[_Group(*(float(v) for v in c)) for c in combos])
        _lib.check_optim(L.naju_adamw_step(tab, cmap, self._n_tensors, self._n_chunks,
                                           ctypes.cast(groups, ctypes.c_void_p), len(combos), coef, stream))
        return loss
