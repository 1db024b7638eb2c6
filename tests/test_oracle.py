"""CPU pins of the oracle (oracle/scan_ref.c and oracle/scan_ref.py).

Each check is chosen so that a plausible mistake in the oracle (a dropped
term, a wrong sign or index, f_{t} where f_{t+1} belongs) fails one of them:

* closed forms computed independently with numpy: constant gates (geometric
  series), f == 0 (no memory), f == 1 (prefix sum), i == 0 (pure decay of h0);
* the explicit C adjoint against torch autograd of the independent torch-loop
  restatement (fp64), and that loop against finite differences (gradcheck);
* invariants: causality, linearity in (u, h0), channel independence,
  dD == sum(dy*u), dfl == 0 exactly where f is exactly 0 or 1;
* the h0 extension reduced to the reference's zero-init 6-argument scan
  (prepending N "load" tokens);
* the chunked affine decomposition the HIP kernels compute (restated here in
  numpy) equals the sequential scan -- the identity of reference
  naju/tests/test_affine_chunk.py:47-78.
"""
import math

import numpy as np
import pytest
import torch

from oracle.scan_ref import (oracle_bwd, oracle_bwd_channels, oracle_fwd, oracle_fwd_channels, rel_err,
                             scan_loop_torch)

NAMES = ("u", "f_logit", "i_logit", "B", "C", "D_skip")


def rand(batch, T, D, N, seed=0, f_shift=2.0, h0=False):
    g = np.random.default_rng(seed)
    ins = dict(u=g.standard_normal((batch, T, D)), f_logit=g.standard_normal((batch, T, D)) + f_shift,
               i_logit=g.standard_normal((batch, T, D)) - 1.0,
               B=g.standard_normal((batch, T, N)) / math.sqrt(N), C=g.standard_normal((batch, T, N)) / math.sqrt(N),
               D_skip=g.standard_normal(D) * 0.1)
    ins = {k: v.astype(np.float32) for k, v in ins.items()}
    ins["h0"] = g.standard_normal((batch, D, N)).astype(np.float32) if h0 else None
    ins["dy"] = g.standard_normal((batch, T, D)).astype(np.float32)
    return ins


def sig(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


# ----------------------------------------------------------- closed forms

def test_geometric_series_constant_gates():
    """N=1, B=C=1, constant f, i, u: x_t = f^(t+1) h0 + i u (1-f^(t+1))/(1-f)."""
    batch, T, D = 2, 50, 3
    # the oracle takes float32 inputs: evaluate the closed form at the
    # float32-rounded values
    fl, il, uu = (float(np.float32(v)) for v in (1.3, -0.4, 0.7))
    f, i = sig(fl), sig(il)
    ins = dict(u=np.full((batch, T, D), uu, np.float32), f_logit=np.full((batch, T, D), fl, np.float32),
               i_logit=np.full((batch, T, D), il, np.float32), B=np.ones((batch, T, 1), np.float32),
               C=np.ones((batch, T, 1), np.float32), D_skip=np.zeros(D, np.float32))
    h0 = np.full((batch, D, 1), -0.25, np.float32)
    y = oracle_fwd(*[ins[k] for k in NAMES], h0=h0)
    t = np.arange(T, dtype=np.float64)[None, :, None]
    expect = f ** (t + 1) * (-0.25) + i * uu * (1 - f ** (t + 1)) / (1 - f)
    np.testing.assert_allclose(y, np.broadcast_to(expect, y.shape), rtol=1e-12, atol=1e-12)


def test_f_zero_no_memory():
    """f == 0 (f_logit = -inf): y_t = (C_t . B_t) i_t u_t + D u_t."""
    ins = rand(2, 40, 5, 4, seed=1)
    ins["f_logit"][:] = -np.inf
    y = oracle_fwd(*[ins[k] for k in NAMES])
    i = sig(ins["i_logit"])
    cb = (ins["C"].astype(np.float64) * ins["B"]).sum(-1)[..., None]
    expect = cb * i * ins["u"] + ins["D_skip"] * ins["u"].astype(np.float64)
    np.testing.assert_allclose(y, expect, rtol=1e-12, atol=1e-12)


def test_f_one_prefix_sum():
    """f == 1 (f_logit = +inf): x_t = h0 + cumsum_s(i_s B_s u_s)."""
    ins = rand(2, 60, 4, 3, seed=2, h0=True)
    ins["f_logit"][:] = np.inf
    y = oracle_fwd(*[ins[k] for k in NAMES], h0=ins["h0"])
    i = sig(ins["i_logit"])[..., None]                                      # [B,T,D,1]
    w = i * ins["u"][..., None].astype(np.float64) * ins["B"][:, :, None, :]  # [B,T,D,N]
    x = ins["h0"][:, None].astype(np.float64) + np.cumsum(w, axis=1)
    expect = (x * ins["C"][:, :, None, :]).sum(-1) + ins["D_skip"] * ins["u"].astype(np.float64)
    np.testing.assert_allclose(y, expect, rtol=1e-11, atol=1e-11)


def test_i_zero_pure_decay():
    """i == 0 (i_logit = -inf): y_t = (prod_{s<=t} f_s) (C_t . h0)."""
    ins = rand(2, 30, 4, 3, seed=3, h0=True)
    ins["i_logit"][:] = -np.inf
    ins["D_skip"][:] = 0
    y = oracle_fwd(*[ins[k] for k in NAMES], h0=ins["h0"])
    decay = np.cumprod(sig(ins["f_logit"]), axis=1)                         # [B,T,D]
    ch0 = np.einsum("btn,bdn->btd", ins["C"].astype(np.float64), ins["h0"].astype(np.float64))
    np.testing.assert_allclose(y, decay * ch0, rtol=1e-11, atol=1e-13)


# ----------------------------------------------- the two restatements agree

@pytest.mark.parametrize("N,h0", [(1, False), (4, True), (16, False)])
def test_c_oracle_matches_torch_loop(N, h0):
    ins = rand(2, 37, 6, N, seed=4 + N, h0=h0)
    t = {k: torch.tensor(v, dtype=torch.float64) for k, v in ins.items() if v is not None}
    y_t = scan_loop_torch(*[t[k] for k in NAMES], h0=t.get("h0")).numpy()
    y_c = oracle_fwd(*[ins[k] for k in NAMES], h0=ins["h0"])
    np.testing.assert_allclose(y_c, y_t, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("N,h0", [(1, True), (3, False), (8, True)])
def test_explicit_adjoint_matches_autograd(N, h0):
    """The C oracle's hand-written backward (naju_cuda.cu:104-141 restated)
    against torch autograd of the torch-loop forward, in fp64."""
    ins = rand(2, 29, 5, N, seed=10 + N, h0=h0)
    xs = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in ins.items()
          if v is not None and k != "dy"}
    y = scan_loop_torch(*[xs[k] for k in NAMES], h0=xs.get("h0"))
    y.backward(torch.tensor(ins["dy"], dtype=torch.float64))
    g = oracle_bwd(*[ins[k] for k in NAMES], dy=ins["dy"], h0=ins["h0"])
    pairs = {"u": "du", "f_logit": "dfl", "i_logit": "dil", "B": "dB", "C": "dC", "D_skip": "dD", "h0": "dh0"}
    for k, gk in pairs.items():
        if k not in xs:
            continue
        np.testing.assert_allclose(g[gk], xs[k].grad.numpy(), rtol=1e-9, atol=1e-11, err_msg=gk)


def test_torch_loop_gradcheck():
    """Finite differences (torch.autograd.gradcheck, fp64) on the torch loop,
    including h0."""
    ins = rand(1, 7, 3, 2, seed=5, h0=True)
    xs = tuple(torch.tensor(ins[k], dtype=torch.float64, requires_grad=True) for k in NAMES + ("h0",))

    def fn(u, fl, il, B, C, Dk, h0):
        return scan_loop_torch(u, fl, il, B, C, Dk, h0=h0)

    assert torch.autograd.gradcheck(fn, xs, eps=1e-6, atol=1e-7, rtol=1e-5)


# ------------------------------------------------------------- invariants

def test_causality():
    ins = rand(2, 40, 4, 3, seed=6)
    y1 = oracle_fwd(*[ins[k] for k in NAMES])
    t0 = 23
    for k in ("u", "f_logit", "i_logit"):
        ins[k][:, t0] += 1.0
    ins["B"][:, t0] *= -2.0
    y2 = oracle_fwd(*[ins[k] for k in NAMES])
    np.testing.assert_array_equal(y1[:, :t0], y2[:, :t0])
    assert np.abs(y1[:, t0:] - y2[:, t0:]).max() > 1e-3


def test_linearity_in_u_and_h0():
    a1, a2 = 0.75, -1.5
    i1 = rand(2, 33, 5, 3, seed=7, h0=True)
    i2 = rand(2, 33, 5, 3, seed=8, h0=True)
    mix = dict(i1)
    mix["u"] = (a1 * i1["u"].astype(np.float64) + a2 * i2["u"]).astype(np.float32)
    mix["h0"] = (a1 * i1["h0"].astype(np.float64) + a2 * i2["h0"]).astype(np.float32)
    args = lambda u: [u, i1["f_logit"], i1["i_logit"], i1["B"], i1["C"], i1["D_skip"]]  # noqa: E731
    y1 = oracle_fwd(*args(i1["u"]), h0=i1["h0"])
    y2 = oracle_fwd(*args(i2["u"]), h0=i2["h0"])
    ym = oracle_fwd(*args(mix["u"]), h0=mix["h0"])
    # inputs were rounded to fp32 once; compare to the fp64 mix of the
    # separately-run outputs with a tolerance covering that rounding
    np.testing.assert_allclose(ym, a1 * y1 + a2 * y2, rtol=1e-6, atol=1e-6)


def test_channel_independence_and_channel_slices():
    """Permuting channels permutes y (no cross-channel coupling), and the
    per-channel oracle functions agree with the full ones."""
    ins = rand(2, 45, 7, 4, seed=12, h0=True)
    y = oracle_fwd(*[ins[k] for k in NAMES], h0=ins["h0"])
    perm = np.random.default_rng(0).permutation(7)
    p = dict(ins)
    for k in ("u", "f_logit", "i_logit", "dy"):
        p[k] = np.ascontiguousarray(ins[k][..., perm])
    p["D_skip"] = np.ascontiguousarray(ins["D_skip"][perm])
    p["h0"] = np.ascontiguousarray(ins["h0"][:, perm])
    yp = oracle_fwd(*[p[k] for k in NAMES], h0=p["h0"])
    np.testing.assert_array_equal(yp, y[..., perm])
    chans = np.array([0, 5, 7 + 2, 7 + 6])
    ys = oracle_fwd_channels(*[ins[k] for k in NAMES], chans=chans, h0=ins["h0"])
    g = oracle_bwd(*[ins[k] for k in NAMES], dy=ins["dy"], h0=ins["h0"])
    gs = oracle_bwd_channels(*[ins[k] for k in NAMES], dy=ins["dy"], chans=chans, h0=ins["h0"])
    for n, c in enumerate(chans):
        b, d = divmod(int(c), 7)
        np.testing.assert_array_equal(ys[n], y[b, :, d])
        for k in ("du", "dfl", "dil"):
            np.testing.assert_array_equal(gs[k][n], g[k][b, :, d])
        np.testing.assert_array_equal(gs["dh0"][n], g["dh0"][b, d])


def test_dD_and_hard_gate_zeros():
    ins = rand(2, 50, 6, 2, seed=13)
    sel = np.random.default_rng(1).random(ins["f_logit"].shape)
    ins["f_logit"][sel < 0.1] = -np.inf
    ins["f_logit"][sel > 0.9] = np.inf
    g = oracle_bwd(*[ins[k] for k in NAMES], dy=ins["dy"])
    np.testing.assert_allclose(g["dD"], (ins["dy"].astype(np.float64) * ins["u"]).sum((0, 1)), rtol=1e-12)
    assert np.all(g["dfl"][(sel < 0.1) | (sel > 0.9)] == 0.0)
    assert np.all(np.isfinite(g["du"])) and np.all(np.isfinite(g["dB"]))


# -------------------------------- h0 reduced to the zero-init reference API

def test_h0_by_prepended_tokens():
    """Prepend N tokens with f = i = 1 (logits +inf), u_t = h0[..., n_t],
    B_t = e_{n_t}, C_t = 0, dy = 0: after them the zero-init state equals h0,
    so y[N:] == scan(..., h0) and du at prepended token n == dh0[..., n]."""
    batch, T, D, N = 2, 20, 3, 4
    ins = rand(batch, T, D, N, seed=14, h0=True)
    h0 = ins["h0"]
    pre = dict(
        u=np.concatenate([np.transpose(h0, (0, 2, 1)), ins["u"]], 1),
        f_logit=np.concatenate([np.full((batch, N, D), np.inf, np.float32), ins["f_logit"]], 1),
        i_logit=np.concatenate([np.full((batch, N, D), np.inf, np.float32), ins["i_logit"]], 1),
        B=np.concatenate([np.broadcast_to(np.eye(N, dtype=np.float32), (batch, N, N)), ins["B"]], 1),
        C=np.concatenate([np.zeros((batch, N, N), np.float32), ins["C"]], 1),
        D_skip=np.zeros(D, np.float32))
    ins["D_skip"][:] = 0
    dy_pre = np.concatenate([np.zeros((batch, N, D), np.float32), ins["dy"]], 1)
    y_pre = oracle_fwd(*[pre[k] for k in NAMES])
    y = oracle_fwd(*[ins[k] for k in NAMES], h0=h0)
    np.testing.assert_allclose(y_pre[:, N:], y, rtol=1e-12, atol=1e-12)
    g_pre = oracle_bwd(*[pre[k] for k in NAMES], dy=dy_pre)
    g = oracle_bwd(*[ins[k] for k in NAMES], dy=ins["dy"], h0=h0)
    np.testing.assert_allclose(np.transpose(g_pre["du"][:, :N], (0, 2, 1)), g["dh0"], rtol=1e-11, atol=1e-12)
    for k in ("du", "dfl", "dil", "dB", "dC"):
        np.testing.assert_allclose(g_pre[k][:, N:], g[k], rtol=1e-11, atol=1e-12, err_msg=k)


# ------------------- the decomposition the HIP kernels compute, restated

def _affine_chunked(f, w, h0, L, W):
    """Chunks of L rows, each made of W sub-chunks (waves): every sub-chunk
    scans from zero to a map s -> F s + Z; maps are composed to the chunk's
    map; chunk carries are composed in order from h0; each sub-chunk's exact
    states are z_t + P_t * s_in. f, w: [T, C]; h0: [C]."""
    T, Cn = f.shape
    x = np.empty((T, Cn))
    s = h0.astype(np.float64).copy()
    R = L // W
    for c0 in range(0, T, L):
        maps = []
        for w0 in range(c0, min(c0 + L, T), R):
            F = np.ones(Cn)
            Z = np.zeros(Cn)
            for t in range(w0, min(w0 + R, T)):
                Z = f[t] * Z + w[t]
                F = F * f[t]
            maps.append((w0, F, Z))
        carry = s
        for (w0, F, Z) in maps:           # per-sub-chunk carry from the chunk's
            P = np.ones(Cn)               # carry and the earlier sub-chunks' maps
            z = np.zeros(Cn)
            for t in range(w0, min(w0 + R, T)):
                z = f[t] * z + w[t]
                P = P * f[t]
                x[t] = z + P * carry
            carry = F * carry + Z
        s = carry
    return x


def test_chunk_decomposition_equals_sequential():
    g = np.random.default_rng(15)
    T, Cn = 203, 9
    f = sig(g.standard_normal((T, Cn)) + 2)
    f[g.random((T, Cn)) < 0.05] = 0.0
    f[g.random((T, Cn)) < 0.05] = 1.0
    w = g.standard_normal((T, Cn))
    h0 = g.standard_normal(Cn)
    xs = np.empty((T, Cn))
    x = h0.copy()
    for t in range(T):
        x = f[t] * x + w[t]
        xs[t] = x
    for L, W in [(64, 8), (32, 4), (16, 16), (7, 7)]:
        np.testing.assert_allclose(_affine_chunked(f, w, h0, L, W), xs, rtol=1e-12, atol=1e-12)


def test_rel_err_measure():
    ref = np.array([1.0, -2.0, 4.0])
    mx, l2 = rel_err(ref + np.array([0.0, 0.04, 0.0]), ref)
    assert abs(mx - 0.01) < 1e-12 and abs(l2 - 0.04 / np.linalg.norm(ref)) < 1e-12
