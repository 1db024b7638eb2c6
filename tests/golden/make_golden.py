"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

The reference ships no golden vectors for its scan (its tests are
differential against naju_scan_reference recomputed at run time), and its
package is not run here. The fixtures are therefore of two kinds:

* closed-form cases -- inputs plus expected outputs computed directly from
  the closed forms (numpy, float64), independent of any scan code:
    geometric : constant gates and input, N=1, B=C=1, with h0
    f_zero    : f_logit = -inf (no memory)
    f_one     : f_logit = +inf (prefix sum), with h0
    i_zero    : i_logit = -inf (pure decay of h0)
* oracle_n1 / oracle_n4 -- seeded inputs (the reference tests' recipe,
  naju/tests/test_affine_chunk.py:34-44) with y and all gradients from the
  fp64 C oracle (oracle/scan_ref.c), whose pins live in tests/test_oracle.py.

Inputs are stored, not seeds (RNG streams are not stable across versions).
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.scan_ref import oracle_bwd, oracle_fwd  # noqa: E402

NAMES = ("u", "f_logit", "i_logit", "B", "C", "D_skip")


def sig(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def closed_forms():
    g = np.random.default_rng(2024)
    out = {}
    # geometric series: x_t = f^(t+1) h0 + i u (1 - f^(t+1)) / (1 - f)
    b, T, D = 2, 300, 96
    fl, il, uu, hh = (float(np.float32(v)) for v in (1.7, -0.3, 0.9, 0.4))
    f, i = sig(fl), sig(il)
    t = np.arange(T, dtype=np.float64)[None, :, None]
    y = np.broadcast_to(f ** (t + 1) * hh + i * uu * (1 - f ** (t + 1)) / (1 - f), (b, T, D))
    out["geometric"] = dict(u=f32(np.full((b, T, D), uu)), f_logit=f32(np.full((b, T, D), fl)),
                            i_logit=f32(np.full((b, T, D), il)), B=f32(np.ones((b, T, 1))),
                            C=f32(np.ones((b, T, 1))), D_skip=f32(np.zeros(D)), h0=f32(np.full((b, D, 1), hh)),
                            y=np.ascontiguousarray(y))
    # f == 0: y_t = (C_t . B_t) i_t u_t + D u_t
    b, T, D, N = 2, 120, 48, 1
    u = f32(g.standard_normal((b, T, D)))
    il = f32(g.standard_normal((b, T, D)))
    Bm = f32(g.standard_normal((b, T, N)))
    Cm = f32(g.standard_normal((b, T, N)))
    Dk = f32(g.standard_normal(D) * 0.1)
    y = (Cm.astype(np.float64) * Bm).sum(-1)[..., None] * sig(il) * u + Dk * u.astype(np.float64)
    out["f_zero"] = dict(u=u, f_logit=f32(np.full((b, T, D), -np.inf)), i_logit=il, B=Bm, C=Cm, D_skip=Dk, y=y)
    # f == 1: x_t = h0 + cumsum(i B u)
    b, T, D, N = 2, 150, 48, 1
    u = f32(g.standard_normal((b, T, D)))
    il = f32(g.standard_normal((b, T, D)))
    Bm = f32(g.standard_normal((b, T, N)))
    Cm = f32(g.standard_normal((b, T, N)))
    h0 = f32(g.standard_normal((b, D, N)))
    w = sig(il)[..., None] * u[..., None].astype(np.float64) * Bm[:, :, None, :]
    x = h0[:, None].astype(np.float64) + np.cumsum(w, axis=1)
    y = (x * Cm[:, :, None, :]).sum(-1)
    out["f_one"] = dict(u=u, f_logit=f32(np.full((b, T, D), np.inf)), i_logit=il, B=Bm, C=Cm,
                        D_skip=f32(np.zeros(D)), h0=h0, y=y)
    # i == 0: y_t = prod_{s<=t} f_s * (C_t . h0)
    b, T, D, N = 2, 120, 40, 1
    fl = f32(g.standard_normal((b, T, D)) + 2)
    Cm = f32(g.standard_normal((b, T, N)))
    h0 = f32(g.standard_normal((b, D, N)))
    y = np.cumprod(sig(fl), axis=1) * np.einsum("btn,bdn->btd", Cm.astype(np.float64), h0.astype(np.float64))
    out["i_zero"] = dict(u=f32(g.standard_normal((b, T, D))), f_logit=fl,
                         i_logit=f32(np.full((b, T, D), -np.inf)), B=f32(g.standard_normal((b, T, N))), C=Cm,
                         D_skip=f32(np.zeros(D)), h0=h0, y=y)
    return out


def oracle_case(b, T, D, N, seed):
    g = np.random.default_rng(seed)
    ins = dict(u=f32(g.standard_normal((b, T, D))), f_logit=f32(g.standard_normal((b, T, D)) + 2.0),
               i_logit=f32(g.standard_normal((b, T, D)) - 1.0),
               B=f32(g.standard_normal((b, T, N)) / math.sqrt(N)), C=f32(g.standard_normal((b, T, N)) / math.sqrt(N)),
               D_skip=f32(g.standard_normal(D) * 0.01), h0=f32(g.standard_normal((b, D, N)) * 0.3),
               dy=f32(g.standard_normal((b, T, D))))
    ins["y"] = oracle_fwd(*[ins[k] for k in NAMES], h0=ins["h0"])
    for k, v in oracle_bwd(*[ins[k] for k in NAMES], dy=ins["dy"], h0=ins["h0"]).items():
        ins[k] = v
    return ins


def main():
    cases = closed_forms()
    cases["oracle_n1"] = oracle_case(2, 160, 48, 1, seed=7)
    cases["oracle_n4"] = oracle_case(2, 64, 24, 4, seed=8)
    for name, arrs in cases.items():
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **arrs)
        print(name, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
