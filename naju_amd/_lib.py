"""ctypes binding of the C ABI declared in include/naju_scan.h,
include/naju_mixer.h, include/naju_loss.h and include/naju_optim.h.

The library is naju_amd/libnaju_scan.so (built by naju_amd/build.py). Nothing
here falls back to another implementation: if the library is missing or a
call fails, an exception is raised.
"""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnaju_scan.so")

DT_F32, DT_BF16, DT_F16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH = 0, -1, -2, -3, -4
FLAG_OUT_F32, FLAG_DETERMINISTIC = 1, 2
CKPT_SHIFT, CKPT_MASK = 8, 0xFF << 8


class ScanBwdLayout(ctypes.Structure):
    """naju_scan_bwd_layout (include/naju_scan.h); the defaults are
    NAJU_SCAN_BWD_LAYOUT_INIT's."""
    _fields_ = [("bc_ld", ctypes.c_int64), ("dbc_ld", ctypes.c_int64), ("dg_ld", ctypes.c_int64),
                ("dg_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32), ("dfl_sum", ctypes.c_void_p),
                ("dil_sum", ctypes.c_void_p)]

    def __init__(self, **kw):
        super().__init__(dg_dtype=-1)
        for k, v in kw.items():
            setattr(self, k, v)


def ckpt_rows_flag(rows):
    """The NAJU_CKPT_ROWS(rows) flag bits (rows a multiple of 16 below 4096;
    0 or None = the default interval)."""
    rows = int(rows or 0)
    if rows < 0 or rows % 16 or rows >= 4096:
        raise ValueError(f"checkpoint interval must be a multiple of 16 below 4096, got {rows}")
    return (rows // 16) << CKPT_SHIFT

EXPORTED = (
    "naju_scan_version",
    "naju_scan_last_error",
    "naju_scan_ckpt_elems",
    "naju_scan_workspace_bytes",
    "naju_scan_ckpt_elems_ex",
    "naju_scan_workspace_bytes_ex",
    "naju_scan_fwd",
    "naju_scan_bwd",
    "naju_scan_fwd_strided",
    "naju_scan_bwd_strided",
    "naju_scan_bwd_ex",
    "naju_scan_workspace_status",
    "naju_scan_fwd_noalloc",
    "naju_scan_noalloc_status",
    "naju_mixer_last_error",
    "naju_dwconv_fwd",
    "naju_dwconv_workspace_bytes",
    "naju_dwconv_bwd",
    "naju_readout_fwd",
    "naju_readout_workspace_bytes",
    "naju_readout_bwd",
    "naju_rmsnorm_fwd",
    "naju_rmsnorm_workspace_bytes",
    "naju_rmsnorm_bwd",
    "naju_rmsnorm_bwd_add",
    "naju_residual_dropout_fwd",
    "naju_dropout_bwd",
    "naju_sum_parts",
    "naju_embedding_bwd_add",
    "naju_dwconv_pair_fwd",
    "naju_dwconv_pair_workspace_bytes",
    "naju_dwconv_pair_bwd",
    "naju_loss_last_error",
    "naju_xent_workspace_bytes",
    "naju_xent_fwd",
    "naju_xent_bwd",
    "naju_xent_fwd_grad",
    "naju_xent_bwd_if_scaled",
    "naju_optim_last_error",
    "naju_grad_norm_workspace_bytes",
    "naju_grad_norm",
    "naju_adamw_step",
    "naju_cast_multi",
)

_lib = None


class NajuScanError(RuntimeError):
    """A C-ABI call returned a nonzero code."""

    def __init__(self, code, msg):
        super().__init__(f"naju_scan error {code}: {msg}")
        self.code = code


def lib():
    """Load (once) and return the ctypes handle; raises if not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -m naju_amd.build, or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, I64, I, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    L.naju_scan_version.argtypes = []
    L.naju_scan_version.restype = I
    L.naju_scan_last_error.argtypes = []
    L.naju_scan_last_error.restype = ctypes.c_char_p
    L.naju_scan_ckpt_elems.argtypes = [I64] * 4 + [I] * 3
    L.naju_scan_ckpt_elems.restype = I64
    L.naju_scan_workspace_bytes.argtypes = [I64] * 4 + [I] * 3
    L.naju_scan_workspace_bytes.restype = SZ
    L.naju_scan_ckpt_elems_ex.argtypes = [I64] * 4 + [I] * 4
    L.naju_scan_ckpt_elems_ex.restype = I64
    L.naju_scan_workspace_bytes_ex.argtypes = [I64] * 4 + [I] * 4
    L.naju_scan_workspace_bytes_ex.restype = SZ
    # u, fl, il, B, C, D_skip, h0, y, ckpt, hT, batch, T, D, N, x_dt, g_dt, bc_dt, flags, ws, ws_bytes,
    # stream
    L.naju_scan_fwd.argtypes = [P] * 10 + [I64] * 4 + [I] * 4 + [P, SZ, P]
    L.naju_scan_fwd.restype = I
    # u, fl, il, B, C, D_skip, ckpt, dy, du, dfl, dil, dB, dC, dD, dh0, batch, T, D, N, dts, flags, ws,
    # ws_bytes, stream
    L.naju_scan_bwd.argtypes = [P] * 15 + [I64] * 4 + [I] * 4 + [P, SZ, P]
    L.naju_scan_bwd.restype = I
    # the same with the B / C row stride after N (and the dB / dC one after it)
    L.naju_scan_fwd_strided.argtypes = [P] * 10 + [I64] * 5 + [I] * 4 + [P, SZ, P]
    L.naju_scan_fwd_strided.restype = I
    L.naju_scan_bwd_strided.argtypes = [P] * 15 + [I64] * 6 + [I] * 4 + [P, SZ, P]
    L.naju_scan_bwd_strided.restype = I
    # naju_scan_bwd's arguments with a naju_scan_bwd_layout pointer after the flags
    L.naju_scan_bwd_ex.argtypes = [P] * 15 + [I64] * 4 + [I] * 4 + [P, P, SZ, P]
    L.naju_scan_bwd_ex.restype = I
    # u, fl, il, B, C, D_skip, h0, y, ckpt, hT, batch, T, D, N, x_dt, g_dt, bc_dt, flags, stream
    L.naju_scan_fwd_noalloc.argtypes = [P] * 10 + [I64] * 4 + [I] * 4 + [P]
    L.naju_scan_fwd_noalloc.restype = I
    L.naju_scan_workspace_status.argtypes = [P, P, ctypes.POINTER(ctypes.c_uint32)]
    L.naju_scan_workspace_status.restype = I
    L.naju_scan_noalloc_status.argtypes = [P, ctypes.POINTER(ctypes.c_uint32)]
    L.naju_scan_noalloc_status.restype = I
    L.naju_mixer_last_error.argtypes = []
    L.naju_mixer_last_error.restype = ctypes.c_char_p
    # x, x_ld, w, bias, add, add_ld, y, batch, T, C, K, act, x_dt, add_dt, y_dt, stream
    L.naju_dwconv_fwd.argtypes = [P, I64] + [P] * 3 + [I64, P] + [I64] * 3 + [I] * 5 + [P]
    L.naju_dwconv_fwd.restype = I
    L.naju_dwconv_workspace_bytes.argtypes = [I64] * 3 + [I]
    L.naju_dwconv_workspace_bytes.restype = SZ
    # x, x_ld, w, bias, dy, dx, dx_ld, dw, dbias, dadd, dadd_ld, batch, T, C, K, act, x_dt, dy_dt, dx_dt,
    # dadd_dt, ws, ws_bytes, stream
    L.naju_dwconv_bwd.argtypes = [P, I64] + [P] * 4 + [I64] + [P] * 3 + [I64] * 4 + [I] * 6 + [P, SZ, P]
    L.naju_dwconv_bwd.restype = I
    F = ctypes.c_float
    # cx, h, z, z_ld, Dv, scale, y, n_rows, C, cx_dt, h_dt, z_dt, y_dt, stream
    L.naju_readout_fwd.argtypes = [P, P, P, I64, P, F, P, I64, I64] + [I] * 4 + [P]
    L.naju_readout_fwd.restype = I
    L.naju_readout_workspace_bytes.argtypes = [I64, I64]
    L.naju_readout_workspace_bytes.restype = SZ
    # cx, h, z, z_ld, Dv, scale, dy, dcx, dh, dz, dz_ld, dD, n_rows, C, 7 dtypes, ws, ws_bytes, stream
    L.naju_readout_bwd.argtypes = [P, P, P, I64, P, F] + [P] * 4 + [I64, P, I64, I64] + [I] * 7 + [P, SZ, P]
    L.naju_readout_bwd.restype = I
    # x, w, eps, y, rstd, n_rows, d, x_dt, y_dt, stream
    L.naju_rmsnorm_fwd.argtypes = [P, P, F, P, P, I64, I64, I, I, P]
    L.naju_rmsnorm_fwd.restype = I
    L.naju_rmsnorm_workspace_bytes.argtypes = [I64, I64]
    L.naju_rmsnorm_workspace_bytes.restype = SZ
    # x, w, rstd, dy, dx, dw, n_rows, d, x_dt, dy_dt, dx_dt, ws, ws_bytes, stream
    L.naju_rmsnorm_bwd.argtypes = [P] * 6 + [I64, I64, I, I, I, P, SZ, P]
    L.naju_rmsnorm_bwd.restype = I
    L.naju_rmsnorm_bwd_add.argtypes = [P] * 7 + [I64, I64, I, I, I, P, SZ, P]
    L.naju_rmsnorm_bwd_add.restype = I
    L.naju_residual_dropout_fwd.argtypes = [P, P, P, F, P, I64, I, P]
    L.naju_residual_dropout_fwd.restype = I
    L.naju_dropout_bwd.argtypes = [P, P, F, P, I64, I, P]
    L.naju_dropout_bwd.restype = I
    L.naju_sum_parts.argtypes = [P, I, I64, P, P]
    L.naju_sum_parts.restype = I
    # sorted_ids, order, dy, n, d, dw, V, stream
    L.naju_embedding_bwd_add.argtypes = [P, P, P, I64, I64, P, I64, P]
    L.naju_embedding_bwd_add.restype = I
    # x, x_ld, w0, bias0, add0, w1, bias1, add1, add_ld, y0, y1, batch, T, C, K, x_dt, y_dt, stream
    L.naju_dwconv_pair_fwd.argtypes = [P, I64] + [P] * 6 + [I64, P, P] + [I64] * 3 + [I] * 3 + [P]
    L.naju_dwconv_pair_fwd.restype = I
    L.naju_dwconv_pair_workspace_bytes.argtypes = [I64] * 3 + [I]
    L.naju_dwconv_pair_workspace_bytes.restype = SZ
    # x, x_ld, w0, w1, dy0, dy1, dx, dx_ld, dw0, db0, dw1, db1, dadd0, dadd1, dadd_ld, batch, T, C, K,
    # accumulate, x_dt, dy_dt, ws, ws_bytes, stream
    L.naju_dwconv_pair_bwd.argtypes = ([P, I64] + [P] * 4 + [I64, P, I64] + [P] * 6 + [I64] * 4 + [I] * 4
                                       + [P, SZ, P])
    L.naju_dwconv_pair_bwd.restype = I
    L.naju_loss_last_error.argtypes = []
    L.naju_loss_last_error.restype = ctypes.c_char_p
    L.naju_xent_workspace_bytes.argtypes = [I64]
    L.naju_xent_workspace_bytes.restype = SZ
    # x, x_ld, target, n_rows, n_cols, x_dt, ignore_index, lse, loss, scale, ws, ws_bytes, stream
    L.naju_xent_fwd.argtypes = [P, I64, P, I64, I64, I, I64, P, P, P, P, SZ, P]
    L.naju_xent_fwd.restype = I
    # x, x_ld, target, n_rows, n_cols, x_dt, ignore_index, lse, scale, dloss, dx, dx_ld, dx_dt, stream
    L.naju_xent_bwd.argtypes = [P, I64, P, I64, I64, I, I64, P, P, P, P, I64, I, P]
    L.naju_xent_bwd.restype = I
    # x, x_ld, target, n_rows, n_cols, x_dt, ignore_index, lse, loss, scale, dx, dx_ld, dx_dt, ws, ws_bytes, stream
    L.naju_xent_fwd_grad.argtypes = [P, I64, P, I64, I64, I, I64, P, P, P, P, I64, I, P, SZ, P]
    L.naju_xent_fwd_grad.restype = I
    L.naju_xent_bwd_if_scaled.argtypes = [P, I64, P, I64, I64, I, I64, P, P, P, P, I64, I, P]
    L.naju_xent_bwd_if_scaled.restype = I
    L.naju_optim_last_error.argtypes = []
    L.naju_optim_last_error.restype = ctypes.c_char_p
    L.naju_grad_norm_workspace_bytes.argtypes = [I64]
    L.naju_grad_norm_workspace_bytes.restype = SZ
    # tensors, chunk_tensor, n_tensors, n_chunks, max_norm, norm, coef, ws, ws_bytes, stream
    L.naju_grad_norm.argtypes = [P, P, I, I64, ctypes.c_float, P, P, P, SZ, P]
    L.naju_grad_norm.restype = I
    # tensors, chunk_tensor, n_tensors, n_chunks, groups (host), n_groups, grad_coef, stream
    L.naju_adamw_step.argtypes = [P, P, I, I64, P, I, P, P]
    L.naju_adamw_step.restype = I
    # tensors, chunk_tensor, n_tensors, n_chunks, dst, dst_dtype, stream
    L.naju_cast_multi.argtypes = [P, P, I, I64, P, I, P]
    L.naju_cast_multi.restype = I
    _lib = L
    return _lib


def last_error():
    """naju_scan_last_error() as str."""
    return lib().naju_scan_last_error().decode(errors="replace")


def check(rc):
    if rc != OK:
        raise NajuScanError(rc, lib().naju_scan_last_error().decode(errors="replace"))
    return rc


def check_mixer(rc):
    """check() for the calls of include/naju_mixer.h."""
    if rc != OK:
        raise NajuScanError(rc, lib().naju_mixer_last_error().decode(errors="replace"))
    return rc


def check_optim(rc):
    """check() for the calls of include/naju_optim.h."""
    if rc != OK:
        raise NajuScanError(rc, lib().naju_optim_last_error().decode(errors="replace"))
    return rc


def check_loss(rc):
    """check() for the calls of include/naju_loss.h."""
    if rc != OK:
        raise NajuScanError(rc, lib().naju_loss_last_error().decode(errors="replace"))
    return rc
