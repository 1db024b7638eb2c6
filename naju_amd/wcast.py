"""16-bit copies of a model's float32 weights in one launch per forward
(naju_cast_multi, include/naju_optim.h).

Under bf16 autocast each linear layer casts its float32 weight to bf16 in a
kernel of its own, and the mixer's fused f / i / x projection concatenates
its three weights first: in the LM step, 37 casts and 12 concatenations per
forward. ``WeightCopies.write(groups, dtype)`` lays the weights of every group
out in one 16-bit buffer (a group's weights back to back, so that they form
one [rows, in] matrix, padded with zero rows to a multiple of the group's
``pad_to``) and writes the whole buffer with one naju_cast_multi launch.
While ``active(copies)`` is entered, ``lookup(weights, dtype)`` returns the
16-bit matrix of a group (the same tensor objects in the same order) for a
linear layer to use in place of its own cast; outside it, and for any other
weights, the layers cast as before. The values are the casts' own (round to
nearest even), so either way the GEMMs see the same operands.

The copies are written anew at every forward from the weights as they are,
so they can never be stale; the buffer is a new allocation each time and
lives as long as the autograd graph that saved its pieces.
"""
import contextlib
import threading

import numpy as np
import torch

from naju_amd import _lib

CHUNK = 8192  # NAJU_OPTIM_CHUNK

# naju_cast_tensor
CAST_DTYPE = np.dtype([("src", "<u8"), ("dst_offset", "<i8"), ("numel", "<i8"), ("first_chunk", "<i8")])
assert CAST_DTYPE.itemsize == 32

_DT = {torch.bfloat16: _lib.DT_BF16, torch.float16: _lib.DT_F16}
_ALIGN = 64  # elements between group starts: 128-byte aligned pieces

_TLS = threading.local()


def _round_up(n, m):
    return -(-n // m) * m


def layout(groups):
    """Offsets of the groups' matrices and the naju_cast_tensor entries.

    groups: sequence of (weights, pad_to) with weights a tuple of 2-D tensors
    of one column count. Returns (total elements, [(offset, rows_padded,
    cols)] per group, [(src_ptr or 0, dst_offset, numel)] entries)."""
    off, mats, entries = 0, [], []
    for ws, pad_to in groups:
        cols = ws[0].shape[1]
        rows = sum(w.shape[0] for w in ws)
        rp = _round_up(rows, pad_to) if pad_to else rows
        mats.append((off, rp, cols))
        o = off
        for w in ws:
            if w.numel():
                entries.append((w.data_ptr(), o, w.numel()))
            o += w.numel()
        if rp > rows:
            entries.append((0, o, (rp - rows) * cols))
        off = _round_up(off + rp * cols, _ALIGN)
    return off, mats, entries


def build_table(entries):
    """naju_cast_tensor records and the chunk -> tensor map of the entries."""
    rec = np.zeros(len(entries), dtype=CAST_DTYPE)
    if not entries:
        return rec, np.zeros(0, dtype=np.int32)
    for name, col in zip(("src", "dst_offset", "numel"), zip(*entries)):
        rec[name] = col
    chunks = (rec["numel"] + CHUNK - 1) // CHUNK
    rec["first_chunk"] = np.concatenate(([0], np.cumsum(chunks)[:-1]))
    return rec, np.repeat(np.arange(len(entries), dtype=np.int32), chunks)


def servable(groups):
    """Whether every weight is a float32 CUDA tensor, contiguous, 2-D, with
    the column count of its group, all on one device."""
    dev = None
    for ws, _ in groups:
        for w in ws:
            if not (w.is_cuda and w.dtype == torch.float32 and w.dim() == 2 and w.is_contiguous()
                    and w.shape[1] == ws[0].shape[1]):
                return False
            if dev is None:
                dev = w.device
            elif w.device != dev:
                return False
    return dev is not None


class WeightCopies:
    """The device table of one set of groups (uploaded again only when the
    weights' addresses or shapes change) and the per-forward write."""

    def __init__(self):
        self._key = None
        self._tab = None
        self._n = 0
        self._chunks = 0
        self._map_off = 0
        self._layout = None

    def _upload(self, groups, device):
        key = tuple((tuple((w.data_ptr(), tuple(w.shape)) for w in ws), pad) for ws, pad in groups)
        if key == self._key:
            return
        total, mats, entries = layout(groups)
        rec, cmap = build_table(entries)
        off = (rec.nbytes + 255) // 256 * 256
        buf = np.zeros(off + cmap.nbytes, dtype=np.uint8)
        buf[:rec.nbytes] = rec.view(np.uint8)
        buf[off:] = cmap.view(np.uint8)
        self._tab = torch.from_numpy(buf).pin_memory().to(device, non_blocking=True)
        self._map_off = off
        self._n, self._chunks = len(entries), int(cmap.size)
        self._layout = (total, mats)
        self._key = key

    def write(self, groups, dtype):
        """The 16-bit matrices of the groups, written by one launch on the
        current stream: {tuple of the weights' ids: [rows_padded, cols]}."""
        device = groups[0][0][0].device
        self._upload(groups, device)
        total, mats = self._layout
        arena = torch.empty(max(total, 1), dtype=dtype, device=device)
        tab = self._tab.data_ptr()
        _lib.check_optim(_lib.lib().naju_cast_multi(tab, tab + self._map_off, self._n, self._chunks,
                                                    arena.data_ptr(), _DT[dtype],
                                                    torch.cuda.current_stream(device).cuda_stream))
        out = {}
        for (ws, _), (off, rp, cols) in zip(groups, mats):
            out[tuple(id(w) for w in ws)] = arena[off:off + rp * cols].view(rp, cols)
        return out


@contextlib.contextmanager
def active(copies, groups, dtype):
    """Within the block, lookup() serves the groups' 16-bit matrices from one
    naju_cast_multi launch made on entry (no copies when groups is empty or
    not servable, or dtype is not 16-bit)."""
    mats = None
    if groups and dtype in _DT and servable(groups):
        mats = copies.write(groups, dtype)
    prev = getattr(_TLS, "mats", None)
    _TLS.mats = (mats, dtype) if mats is not None else prev
    try:
        yield
    finally:
        _TLS.mats = prev


def lookup(weights, dtype):
    """The active 16-bit matrix of exactly these weights (as one group, in
    this order) in dtype, or None."""
    cur = getattr(_TLS, "mats", None)
    if cur is None or cur[1] != dtype:
        return None
    return cur[0].get(tuple(id(w) for w in weights))
