"""Shared helpers of the parity tests: run the HIP scan through autograd and
compare every output with the fp64 oracle at the stated tolerance."""
import numpy as np
import torch

from oracle.scan_ref import oracle_bwd, oracle_fwd, rel_err

NAMES = ("u", "f_logit", "i_logit", "B", "C", "D_skip")
GRAD_KEYS = {"u": "du", "f_logit": "dfl", "i_logit": "dil", "B": "dB", "C": "dC", "D_skip": "dD", "h0": "dh0"}


def tol_for(dtype):
    """(max_tol, l2_tol) on max-abs error / max|oracle| and ||err||/||oracle||.

    float32 outputs: 1e-5 both -- this covers bf16/fp16 INPUTS with float32
    outputs too, since the oracle runs on the same quantized inputs.
    bfloat16 outputs: 2e-3 norm-wise; the max-norm bound is the storage
    rounding itself, 2^-8 relative (bf16 keeps 8 significant bits), plus
    float32-level slack. float16 outputs: 2e-3 both (rounding 2^-11)."""
    if dtype in (torch.float32, torch.float64):
        return 1e-5, 1e-5
    if dtype == torch.bfloat16:
        return 2.0 ** -8 + 2e-5, 2e-3
    return 2e-3, 2e-3


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
    tmx, tl2 = tol
    assert mx <= tmx and l2 <= tl2, f"{name}: rel err max {mx:.3e} l2 {l2:.3e} > tol ({tmx:.2e}, {tl2:.1e})"
    return mx, l2


def check_all(y, grads, ref_y, ref_g, skip=()):
    """Every output against the oracle at the tolerance of its own dtype."""
    res = {"y": check("y", y, ref_y, tol_for(y.dtype))}
    for k, v in grads.items():
        if k in skip or v is None:
            continue
        res[k] = check(k, v, ref_g[k], tol_for(v.dtype))
    return res


_DTC = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def run_abi(ins, device, out_f32=True, deterministic=False):
    """Forward + backward through the C ABI directly (naju_scan_fwd/_bwd), with
    every output in float32 when out_f32 and fixed-order carries when
    deterministic. Returns (y, grads) like run_hip."""
    from naju_amd import _lib
    L = _lib.lib()
    t = {k: (v.to(device).contiguous() if v is not None else None) for k, v in ins.items()}
    u, fl, il, Bm, Cm = t["u"], t["f_logit"], t["i_logit"], t["B"], t["C"]
    Dk = t["D_skip"].float().contiguous()
    h0 = t.get("h0")
    dy = t["dy"]
    Bsz, T, D = u.shape
    N = Bm.shape[-1]
    dts = (_DTC[u.dtype], _DTC[fl.dtype], _DTC[Bm.dtype])
    od = lambda x: torch.float32 if out_f32 else x.dtype  # noqa: E731
    flags = (_lib.FLAG_OUT_F32 if out_f32 else 0) | (_lib.FLAG_DETERMINISTIC if deterministic else 0)
    y = torch.empty(u.shape, dtype=od(u), device=device)
    ck = torch.empty(max(1, L.naju_scan_ckpt_elems(Bsz, T, D, N, *dts)), dtype=torch.float32, device=device)
    nb = L.naju_scan_workspace_bytes(Bsz, T, D, N, *dts)
    ws = torch.zeros(max(nb, 256), dtype=torch.uint8, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    p = lambda x: None if x is None else x.data_ptr()  # noqa: E731
    _lib.check(L.naju_scan_fwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(h0), p(y), p(ck), None,
                               Bsz, T, D, N, *dts, flags, p(ws), ws.numel(), st))
    g = {"du": torch.empty(u.shape, dtype=od(u), device=device),
         "dfl": torch.empty(u.shape, dtype=od(fl), device=device),
         "dil": torch.empty(u.shape, dtype=od(il), device=device),
         "dB": torch.empty(Bm.shape, dtype=od(Bm), device=device),
         "dC": torch.empty(Bm.shape, dtype=od(Cm), device=device),
         "dD": torch.empty(D, dtype=torch.float32, device=device)}
    if h0 is not None:
        g["dh0"] = torch.empty(h0.shape, dtype=torch.float32, device=device)
    _lib.check(L.naju_scan_bwd(p(u), p(fl), p(il), p(Bm), p(Cm), p(Dk), p(ck), p(dy), p(g["du"]),
                               p(g["dfl"]), p(g["dil"]), p(g["dB"]), p(g["dC"]), p(g["dD"]), p(g.get("dh0")),
                               Bsz, T, D, N, *dts, flags, p(ws), ws.numel(), st))
    torch.cuda.synchronize()
    return y, g
