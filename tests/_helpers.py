"""Shared helpers of the parity tests: run the HIP scan through autograd and
compare every output with the fp64 oracle at the stated tolerance."""
import numpy as np
import torch

from oracle.scan_ref import oracle_bwd, oracle_fwd, rel_err

NAMES = ("u", "f_logit", "i_logit", "B", "C", "D_skip")
GRAD_KEYS = {"u": "du", "f_logit": "dfl", "i_logit": "dil", "B": "dB", "C": "dC", "D_skip": "dD", "h0": "dh0"}


def tol_for(dtype):
    """Tolerance (max-abs error / max|oracle| and ||err||/||oracle||):
    float32 1e-5; bfloat16/float16 in with float32 accumulation 2e-3."""
    return 1e-5 if dtype in (torch.float32, torch.float64) else 2e-3


def rand_inputs(batch, T, D, N, seed=0, dtype=torch.float32, f_shift=2.0, i_shift=-1.0,
                bc_scale=None, d_scale=0.01, h0_std=0.0, gate_dtype=None, bc_dtype=None):
    """The reference tests' recipe (naju/tests/test_affine_chunk.py:34-44):
    u~N(0,1), f_logit~N(0,1)+2, i_logit~N(0,1)-1, B,C~N(0,1)/sqrt(N),
    D_skip~0.01 N(0,1); plus optional h0 and an upstream gradient dy."""
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    sc = (1.0 / N ** 0.5) if bc_scale is None else bc_scale
    gd = gate_dtype or dtype
    bd = bc_dtype or dtype
    ins = dict(
        u=r(batch, T, D).to(dtype),
        f_logit=(r(batch, T, D) + f_shift).to(gd),
        i_logit=(r(batch, T, D) + i_shift).to(gd),
        B=(r(batch, T, N) * sc).to(bd),
        C=(r(batch, T, N) * sc).to(bd),
        D_skip=r(D) * d_scale,
    )
    ins["h0"] = (r(batch, D, N) * h0_std) if h0_std > 0 else None
    ins["dy"] = r(batch, T, D).to(dtype)
    return ins


def run_hip(ins, device, grad=True, grad_names=None):
    """Forward (+ backward with ins['dy']) through naju_scan_hip on `device`.
    Returns (y, {grad_key: tensor})."""
    from naju_amd import naju_scan_hip
    names = list(NAMES) + (["h0"] if ins.get("h0") is not None else [])
    want = set(grad_names) if grad_names is not None else set(names)
    xs = {}
    for k in names:
        t = ins[k].to(device)
        if grad and k in want:
            t = t.detach().requires_grad_(True)
        xs[k] = t
    if grad:
        y = naju_scan_hip(*[xs[k] for k in NAMES], xs.get("h0"))
        y.backward(ins["dy"].to(device))
        grads = {GRAD_KEYS[k]: xs[k].grad for k in names if k in want}
    else:
        with torch.no_grad():
            y = naju_scan_hip(*[xs[k] for k in NAMES], xs.get("h0"))
        grads = {}
    torch.cuda.synchronize()
    return y, grads


def oracle_all(ins):
    args = [ins[k] for k in NAMES]
    y = oracle_fwd(*args, h0=ins.get("h0"))
    g = oracle_bwd(*args, dy=ins["dy"], h0=ins.get("h0"))
    return y, g


def check(name, out, ref, tol):
    out = out.detach().float().cpu().numpy().astype(np.float64) if hasattr(out, "detach") else out
    assert np.all(np.isfinite(out)), f"{name}: non-finite output"
    mx, l2 = rel_err(out, ref)
    assert mx <= tol and l2 <= tol, f"{name}: rel err max {mx:.3e} l2 {l2:.3e} > tol {tol:.1e}"
    return mx, l2


def check_all(y, grads, ref_y, ref_g, skip=()):
    """Every output against the oracle at the tolerance of its own dtype."""
    res = {"y": check("y", y, ref_y, tol_for(y.dtype))}
    for k, v in grads.items():
        if k in skip or v is None:
            continue
        res[k] = check(k, v, ref_g[k], tol_for(v.dtype))
    return res
