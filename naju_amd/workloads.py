"""Synthetic scan inputs for the configurations the benchmark and tests use.

Each configuration of the headline benchmark is described in terms of gate
values: retention a = sigmoid(f_logit), write gate w = sigmoid(i_logit),
input x = u, initial state h0. The reference takes logits (naju/scan.py:17),
so a = sigmoid(N(0,1)+2) means f_logit = N(0,1)+2, and
a = exp(-softplus(z)) = sigmoid(-z) means f_logit = -z.

B and C (the [B,T,N] write/read vectors) are ones at N = 1, which makes the
scan the plain per-channel gated recurrence h_t = a_t h_{t-1} + w_t x_t; at
N > 1 they are N(0,1)/sqrt(N), as in reference naju/tests/bench_scan.py:30-31.
D_skip is zero, as NajuMixer passes it (naju/mixer.py:121).
"""
import math

import torch

CONFIGS = {
    # name: (batch, T, D, stream dtype, gate recipe, h0 std)
    "c1": dict(batch=2, T=1024, D=256, dtype=torch.float32, gate="shift2", h0_std=0.0),
    "c2": dict(batch=8, T=4096, D=1024, dtype=torch.bfloat16, gate="shift2", h0_std=0.1),
    "c3": dict(batch=1, T=131072, D=2048, dtype=torch.float32, gate="near_one", h0_std=0.0),
    "c4": dict(batch=32, T=8192, D=4096, dtype=torch.bfloat16, gate="edge", h0_std=0.0),
}


def make_inputs(batch, T, D, N=1, dtype=torch.float32, gate="shift2", h0_std=0.0, seed=0,
                device="cpu", with_dy=True):
    """Seeded inputs. Returns dict u, f_logit, i_logit, B, C, D_skip, h0, dy.
    Generated in float32 on `device` with its own generator, then cast."""
    g = torch.Generator(device=device).manual_seed(seed)

    def rn(*shape):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32)

    u = rn(batch, T, D)
    if gate == "shift2":          # a = sigmoid(N(0,1) + 2)
        fl = rn(batch, T, D) + 2.0
    elif gate == "near_one":      # a = exp(-softplus(N(-4,1))) = sigmoid(N(4,1))
        fl = rn(batch, T, D) + 4.0
    elif gate == "edge":          # sigmoid(N(0,2^2)); 10% exactly 0, 10% exactly 1
        fl = rn(batch, T, D) * 2.0
        sel = torch.rand(batch, T, D, generator=g, device=device)
        fl = torch.where(sel < 0.1, torch.full_like(fl, -math.inf), fl)
        fl = torch.where(sel >= 0.9, torch.full_like(fl, math.inf), fl)
    elif gate == "deep":          # f ~ sigmoid(-12): the reference's deep-gate stress
        fl = rn(batch, T, D) - 12.0
    else:
        raise ValueError(gate)
    il = rn(batch, T, D)
    if N == 1:
        Bm = torch.ones(batch, T, 1, device=device)
        Cm = torch.ones(batch, T, 1, device=device)
    else:
        Bm = rn(batch, T, N) / math.sqrt(N)
        Cm = rn(batch, T, N) / math.sqrt(N)
    D_skip = torch.zeros(D, device=device)
    h0 = rn(batch, D, N) * h0_std if h0_std > 0 else None
    dy = rn(batch, T, D) if with_dy else None
    out = dict(u=u.to(dtype), f_logit=fl.to(dtype), i_logit=il.to(dtype), B=Bm.to(dtype),
               C=Cm.to(dtype), D_skip=D_skip, h0=h0, dy=None if dy is None else dy.to(dtype))
    return out


def config_inputs(name, N=1, seed=0, device="cuda", with_dy=True):
    c = CONFIGS[name]
    return make_inputs(c["batch"], c["T"], c["D"], N=N, dtype=c["dtype"], gate=c["gate"],
                       h0_std=c["h0_std"], seed=seed, device=device, with_dy=with_dy)


def algorithmic_bytes(batch, T, D, N, s_x, s_g, s_bc, has_h0, fwd=True, bwd=True):
    """HBM bytes the fused fwd+bwd must move at minimum (per call pair):
    fwd reads u, fl, il, B, C and h0, writes y; bwd reads u, fl, il, dy, B, C
    and h0, writes du, dfl, dil, dB, dC and dh0 (h0/dh0 float32)."""
    E = batch * T * D
    BTN = batch * T * N
    tot = 0
    if fwd:
        tot += E * (s_x + 2 * s_g + s_x) + BTN * 2 * s_bc + (batch * D * N * 4 if has_h0 else 0)
    if bwd:
        tot += E * (2 * s_x + 2 * s_g) + E * (s_x + 2 * s_g) + BTN * 4 * s_bc \
            + (batch * D * N * 8 if has_h0 else 0)
    return tot
