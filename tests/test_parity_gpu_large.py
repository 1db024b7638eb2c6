"""GPU parity at the full sizes of benchmark configurations c2-c4
(naju_amd.workloads.CONFIGS) at N = 1 and at the mixer's N = 64, and of one
c5 scan layer, against the fp64 oracle run over channel slices on the
host's cores.

Config 3 (B=1, T=131072, D=2048, fp32, retention near 1): EVERY output is
checked against the oracle. The oracle runs on 64-channel slices; y, du, dfl,
dil and dD are per-channel, and dB, dC (sums over the channels) are the sums
of the slices' partial dB, dC, added in slice order.

Config 4 (B=32, T=8192, D=4096, bf16, 10% of the gates exactly 0 and 10%
exactly 1): batch row 0 in full (every output except dD depends only on its
own batch row, dB and dC included), dD against sum(dy*u) over the whole batch.

Tolerances are those of every parity test (tests/_helpers.tol_for), applied to
the whole output: the max-abs error over max|oracle| and the l2 ratio are
assembled from the slices' sums.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from tests._helpers import run_hip, tol_for

pytestmark = pytest.mark.gpu

_WORKERS = max(1, min(16, os.cpu_count() or 1))


class _Err:
    """Running max-abs error, max |ref|, sum err^2 and sum ref^2 of one output."""

    def __init__(self):
        self.emax = self.rmax = self.e2 = self.r2 = 0.0

    def add(self, out, ref):
        err = np.asarray(out, np.float64) - ref
        assert np.all(np.isfinite(out))
        self.emax = max(self.emax, float(np.abs(err).max()))
        self.rmax = max(self.rmax, float(np.abs(ref).max()))
        self.e2 += float((err * err).sum())
        self.r2 += float((ref * ref).sum())

    def check(self, name, dtype):
        mx = self.emax / max(self.rmax, 1e-30)
        l2 = (self.e2 ** 0.5) / max(self.r2 ** 0.5, 1e-30)
        tmx, tl2 = tol_for(dtype)
        assert mx <= tmx and l2 <= tl2, f"{name}: rel err max {mx:.3e} l2 {l2:.3e} > tol ({tmx:.2e}, {tl2:.1e})"


def _host(t):
    return t.detach().float().cpu().numpy()


def _slices_vs_oracle(inp, out, width):
    """Oracle over channel slices of one batch row set (inp / out: host float32
    arrays [b, T, D] of u, f_logit, i_logit, dy and y, du, dfl, dil; B, C
    [b, T, N]; D_skip [D]; optional h0 [b, D, N] in inp and dh0 in out).
    Returns the per-output error accumulators and the oracle's dB, dC (summed
    over the slices in slice order) and dD."""
    from oracle.scan_ref import oracle_bwd, oracle_fwd
    D = inp["u"].shape[2]
    starts = list(range(0, D, width))
    h0 = inp.get("h0")

    def one(d0):
        sl = slice(d0, min(D, d0 + width))
        a = [np.ascontiguousarray(inp[k][:, :, sl]) for k in ("u", "f_logit", "i_logit")]
        a += [inp["B"], inp["C"], np.ascontiguousarray(inp["D_skip"][sl])]
        hs = np.ascontiguousarray(h0[:, sl]) if h0 is not None else None
        ry = oracle_fwd(*a, h0=hs)
        rg = oracle_bwd(*a, dy=np.ascontiguousarray(inp["dy"][:, :, sl]), h0=hs)
        errs = {}
        pairs = [("y", ry), ("du", rg["du"]), ("dfl", rg["dfl"]), ("dil", rg["dil"])]
        for k, ref in pairs:
            e = _Err()
            e.add(out[k][:, :, sl], ref)
            errs[k] = e
        if h0 is not None:
            e = _Err()
            e.add(out["dh0"][:, sl], rg["dh0"])
            errs["dh0"] = e
        return errs, rg["dB"], rg["dC"], rg["dD"]

    with ThreadPoolExecutor(_WORKERS) as ex:
        res = list(ex.map(one, starts))
    tot = {k: _Err() for k in ("y", "du", "dfl", "dil") + (("dh0",) if h0 is not None else ())}
    for errs, _, _, _ in res:
        for k, e in errs.items():
            t = tot[k]
            t.emax, t.rmax = max(t.emax, e.emax), max(t.rmax, e.rmax)
            t.e2, t.r2 = t.e2 + e.e2, t.r2 + e.r2
    dB = sum(r[1] for r in res)
    dC = sum(r[2] for r in res)
    dD = np.concatenate([r[3] for r in res])
    return tot, dB, dC, dD


def test_full_size_c3_every_output(gpu):
    """1 x 131072 x 2048 fp32 with retention near 1 (2048 chunks per channel
    tile carried in sequence): every element of every output."""
    from naju_amd.workloads import config_inputs
    ins = config_inputs("c3", N=1, seed=3, device=gpu)
    y, g = run_hip(ins, gpu)
    inp = {k: _host(ins[k]) for k in ("u", "f_logit", "i_logit", "dy", "B", "C", "D_skip")}
    out = {"y": _host(y), "du": _host(g["du"]), "dfl": _host(g["dfl"]), "dil": _host(g["dil"])}
    del ins
    tot, dB, dC, dD = _slices_vs_oracle(inp, out, 64)
    for k in ("y", "du", "dfl", "dil"):
        tot[k].check(k, torch.float32)
    for k, ref in (("dB", dB), ("dC", dC)):
        e = _Err()
        e.add(_host(g[k]), ref)
        e.check(k, torch.float32)
    e = _Err()
    e.add(_host(g["dD"]), dD)
    e.check("dD", torch.float32)


def test_full_size_c4_batch_row(gpu):
    """32 x 8192 x 4096 bf16 with hard resets and pure retention (f_logit
    = -inf / +inf on 10% of the entries each): batch row 0 in full, dD over
    the whole batch."""
    from naju_amd.workloads import config_inputs
    ins = config_inputs("c4", N=1, seed=4, device=gpu)
    assert bool(torch.isinf(ins["f_logit"][0]).any())
    y, g = run_hip(ins, gpu)
    inp = {k: _host(ins[k][:1]) for k in ("u", "f_logit", "i_logit", "dy", "B", "C")}
    inp["D_skip"] = _host(ins["D_skip"])
    out = {"y": _host(y[:1]), "du": _host(g["du"][:1]), "dfl": _host(g["dfl"][:1]), "dil": _host(g["dil"][:1])}
    tot, dB, dC, _ = _slices_vs_oracle(inp, out, 256)
    for k in ("y", "du", "dfl", "dil"):
        tot[k].check(k, y.dtype)
    for k, ref in (("dB", dB), ("dC", dC)):
        e = _Err()
        e.add(_host(g[k][:1]), ref)
        e.check(k, g[k].dtype)
    ref_dD = torch.zeros(ins["u"].shape[2], dtype=torch.float64, device=gpu)
    for b in range(ins["u"].shape[0]):
        ref_dD += (ins["dy"][b].double() * ins["u"][b].double()).sum(0)
    ref_dD = ref_dD.cpu().numpy()
    assert np.max(np.abs(g["dD"].double().cpu().numpy() - ref_dD)) <= 1e-4 * max(1.0, np.abs(ref_dD).max())


def _check_row0(ins, y, g, width, n_rows=1):
    """Batch rows [0, n_rows) of every output against the oracle over channel
    slices (dB, dC included); dD against sum(dy*u) over the whole batch."""
    rows = slice(0, n_rows)
    inp = {k: _host(ins[k][rows]) for k in ("u", "f_logit", "i_logit", "dy", "B", "C")}
    inp["D_skip"] = _host(ins["D_skip"])
    out = {k: _host(v[rows]) for k, v in (("y", y), ("du", g["du"]), ("dfl", g["dfl"]), ("dil", g["dil"]))}
    if ins.get("h0") is not None:
        inp["h0"] = _host(ins["h0"][rows])
        out["dh0"] = _host(g["dh0"][rows])
    tot, dB, dC, _ = _slices_vs_oracle(inp, out, width)
    for k in ("y", "du", "dfl", "dil"):
        tot[k].check(k, (y if k == "y" else g[k]).dtype)
    if "dh0" in tot:
        tot["dh0"].check("dh0", torch.float32)
    for k, ref in (("dB", dB), ("dC", dC)):
        e = _Err()
        e.add(_host(g[k][rows]), ref)
        e.check(k, g[k].dtype)
    ref_dD = (ins["dy"].double() * ins["u"].double()).sum((0, 1)).cpu().numpy()
    assert np.max(np.abs(g["dD"].double().cpu().numpy() - ref_dD)) <= 1e-4 * max(1.0, np.abs(ref_dD).max())


def test_full_size_c2_n64_batch_row(gpu):
    """Benchmark configuration c2 at the mixer's N = 64 (8 x 4096 x 1024, bf16
    streams, h0), full size on the GPU: batch row 0 of every output in full,
    dB and dC (sums over all 1024 channels) and dh0 included."""
    from naju_amd.workloads import config_inputs
    ins = config_inputs("c2", N=64, seed=12, device=gpu)
    y, g = run_hip(ins, gpu)
    _check_row0(ins, y, g, 64)


def test_full_size_c4_n64_exact_decay_batch_row(gpu):
    """Benchmark configuration c4's recipe at the mixer's N = 64 (32 x 8192 x
    4096, bf16, 10% of the gates exactly 0 and 10% exactly 1), full size.
    Nearly every 16-row x 16-channel block then holds a hard reset, so the
    matrix-core kernels take their exact-decay (Horner) path at NP = 64
    almost everywhere. Batch row 0 of every output in full, dB and dC (sums
    over all 4096 channels) included; dD over the whole batch."""
    from naju_amd.workloads import config_inputs
    print("c4 N=64 full size, seed 44", flush=True)
    ins = config_inputs("c4", N=64, seed=44, device=gpu)
    # share of (16 rows x 16 channels) blocks of batch row 0 with a zero gate
    z = torch.isneginf(ins["f_logit"][0]).view(8192 // 16, 16, 4096 // 16, 16).any(dim=3).any(dim=1)
    assert float(z.float().mean()) > 0.999
    y, g = run_hip(ins, gpu)
    _check_row0(ins, y, g, 256)


def test_full_size_c3_n64_every_output(gpu):
    """Benchmark configuration c3 at N = 64 (1 x 131072 x 2048 fp32,
    retention near 1: the state carries over the whole 131072 rows), full
    size: every element of every output against the oracle over 64-channel
    slices, dB and dC as the slice-ordered sums of the slices' partial sums."""
    from naju_amd.workloads import config_inputs
    print("c3 N=64 full size, seed 33", flush=True)
    ins = config_inputs("c3", N=64, seed=33, device=gpu)
    y, g = run_hip(ins, gpu)
    inp = {k: _host(ins[k]) for k in ("u", "f_logit", "i_logit", "dy", "B", "C", "D_skip")}
    out = {"y": _host(y), "du": _host(g["du"]), "dfl": _host(g["dfl"]), "dil": _host(g["dil"])}
    del ins
    tot, dB, dC, dD = _slices_vs_oracle(inp, out, 64)
    for k in ("y", "du", "dfl", "dil"):
        tot[k].check(k, torch.float32)
    for k, ref in (("dB", dB), ("dC", dC)):
        e = _Err()
        e.add(_host(g[k]), ref)
        e.check(k, torch.float32)
    e = _Err()
    e.add(_host(g["dD"]), dD)
    e.check("dD", torch.float32)


def test_full_size_c5_scan_layer(gpu):
    """The scan call of one layer of the c5 LM step at full size: 8 x 2048 x
    1536 channels, N = 64, with the mixer's autocast dtypes (u, B, C bf16;
    gate logits f32, the gate biases' +5 / -2 initial offsets): batch row 0
    of every output in full, dB and dC included."""
    from tests._helpers import rand_inputs
    ins = rand_inputs(8, 2048, 1536, 64, seed=55, dtype=torch.bfloat16, gate_dtype=torch.float32,
                      bc_dtype=torch.bfloat16, f_shift=5.0, i_shift=-2.0, d_scale=0.0)
    y, g = run_hip(ins, gpu)
    assert y.dtype == torch.bfloat16 and g["dfl"].dtype == torch.float32
    _check_row0(ins, y, g, 96)
