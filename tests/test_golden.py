"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py):
the oracle on the CPU, and the HIP scan on the GPU, against stored expected
outputs. Closed-form fixtures pin both independently of any scan code."""
import os

import numpy as np
import pytest

from oracle.scan_ref import oracle_bwd, oracle_fwd, rel_err

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
NAMES = ("u", "f_logit", "i_logit", "B", "C", "D_skip")
CLOSED = ("geometric", "f_zero", "f_one", "i_zero")
GRADS = ("du", "dfl", "dil", "dB", "dC", "dD", "dh0")


def load(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", CLOSED + ("oracle_n1", "oracle_n4"))
def test_oracle_matches_fixture(name):
    fx = load(name)
    y = oracle_fwd(*[fx[k] for k in NAMES], h0=fx.get("h0"))
    mx, _ = rel_err(y, fx["y"])
    assert mx <= 1e-12, (name, mx)
    if "dy" in fx:
        g = oracle_bwd(*[fx[k] for k in NAMES], dy=fx["dy"], h0=fx.get("h0"))
        for k in GRADS:
            assert rel_err(g[k], fx[k])[0] <= 1e-12, (name, k)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CLOSED + ("oracle_n1",))
def test_hip_matches_fixture(gpu, name):
    """float32 HIP scan against the stored expected outputs (1e-5)."""
    import torch
    from tests._helpers import check, run_hip, tol_for
    fx = load(name)
    ins = {k: torch.from_numpy(fx[k]) for k in NAMES}
    ins["h0"] = torch.from_numpy(fx["h0"]) if "h0" in fx else None
    ins["dy"] = torch.from_numpy(fx["dy"]) if "dy" in fx else torch.zeros_like(ins["u"])
    y, g = run_hip(ins, gpu, grad="dy" in fx)
    check("y", y, fx["y"], tol_for(torch.float32))
    if "dy" in fx:
        for k in GRADS:
            check(k, g[k], fx[k], tol_for(torch.float32))
