"""The memory-light checkpoint interval (NAJU_CKPT_ROWS, naju_scan_hip's
ckpt_rows): the forward keeps the state every r rows instead of every 16, and
the backward recomputes the states between from it -- the role of the
reference's recompute backend (naju/cuda/__init__.py:9-12, CK = 32 in
naju/cuda/naju_cuda.cu:25). Every output must be bitwise the default
interval's (the recompute repeats the forward's arithmetic exactly), and
the default itself is pinned against the fp64 oracle by the parity tests;
one case here is also checked against the oracle directly."""
import pytest
import torch

from tests._helpers import GRAD_KEYS, NAMES, check_all, oracle_all, rand_inputs, tol_for

pytestmark = pytest.mark.gpu


def _run(ins, dev, rows):
    from naju_amd import naju_scan_hip
    names = list(NAMES) + (["h0"] if ins.get("h0") is not None else [])
    xs = {k: ins[k].to(dev).detach().requires_grad_(True) for k in names}
    y = naju_scan_hip(*[xs[k] for k in NAMES], xs.get("h0"), ckpt_rows=rows)
    y.backward(ins["dy"].to(dev))
    torch.cuda.synchronize()
    return y.detach(), {GRAD_KEYS[k]: xs[k].grad for k in names}


CASES = [
    # (batch, T, D, N), dtype, h0_std, intervals
    ((2, 300, 96, 16), torch.float32, 0.5, (32, 64, 128)),
    ((2, 300, 70, 33), torch.float32, 0.0, (32, 64)),
    ((1, 1000, 128, 64), torch.float32, 0.3, (32, 64, 128)),
    ((2, 129, 200, 64), torch.bfloat16, 0.0, (64, 128)),
    ((3, 77, 64, 9), torch.float16, 0.2, (32, 128)),
    # long enough for several time segments of the forward (and of the
    # backward) with their carries
    ((2, 2500, 192, 64), torch.bfloat16, 0.3, (32, 128)),
]


@pytest.mark.parametrize("shape,dtype,h0_std,intervals", CASES)
def test_interval_is_bitwise_the_default(shape, dtype, h0_std, intervals):
    dev = torch.device("cuda:0")
    print(f"ckpt interval case {shape} {dtype} h0={h0_std} rows={intervals}", flush=True)
    ins = rand_inputs(*shape, seed=sum(shape), dtype=dtype, h0_std=h0_std)
    y0, g0 = _run(ins, dev, None)
    for rows in intervals:
        y, g = _run(ins, dev, rows)
        assert torch.equal(y, y0), rows
        for k in g0:
            assert torch.equal(g[k], g0[k]), (rows, k)


def test_interval_against_oracle():
    """A long interval on a ragged shape, directly against the fp64 oracle."""
    dev = torch.device("cuda:0")
    ins = rand_inputs(2, 211, 72, 40, seed=5, h0_std=0.4)
    y, g = _run(ins, dev, 64)
    ref_y, ref_g = oracle_all(ins)
    check_all(y.cpu(), {k: v.cpu() for k, v in g.items()}, ref_y, ref_g)


def test_interval_rejected_where_not_served():
    from naju_amd import naju_scan_hip
    from naju_amd._lib import NajuScanError
    dev = torch.device("cuda:0")
    ins = rand_inputs(1, 40, 32, 4, seed=1)
    xs = [ins[k].to(dev).requires_grad_(True) for k in NAMES]
    with pytest.raises(NajuScanError, match="interval"):
        naju_scan_hip(*xs, None, ckpt_rows=64)
    ins = rand_inputs(1, 40, 32, 16, seed=1)
    xs = [ins[k].to(dev).requires_grad_(True) for k in NAMES]
    with pytest.raises(NajuScanError, match="interval"):
        naju_scan_hip(*xs, None, ckpt_rows=256)
