"""The final state hT = x_{T-1} [B, D, N] (the state a streaming decoder
resumes from) and the forward without a checkpoint (the no_grad / inference
path, the role of reference naju/cuda/bw.py:36-38 -> naju_cuda_bw.cu:282-309),
against the fp64 oracle, for N = 1 and for both general-N forwards: the
segmented one (small batch x channel grids, several time segments) and the
unsegmented one with four states per lane (grids that fill the GPU)."""
import numpy as np
import pytest
import torch

from oracle.scan_ref import oracle_fwd
from tests._helpers import NAMES, check, check_all, oracle_all, rand_inputs, tol_for

pytestmark = pytest.mark.gpu


def _hip(ins, dev, grad):
    from naju_amd import naju_scan_hip
    xs = {k: ins[k].to(dev) for k in NAMES}
    h0 = ins["h0"].to(dev) if ins.get("h0") is not None else None
    if grad:
        xs = {k: v.detach().requires_grad_(True) for k, v in xs.items()}
        y, hT = naju_scan_hip(*[xs[k] for k in NAMES], h0, return_final_state=True)
        assert not hT.requires_grad
        y.backward(ins["dy"].to(dev))
    else:
        with torch.no_grad():
            y, hT = naju_scan_hip(*[xs[k] for k in NAMES], h0, return_final_state=True)
    torch.cuda.synchronize()
    return y, hT


def _oracle_y_hT(ins):
    return oracle_fwd(*[ins[k] for k in NAMES], h0=ins.get("h0"), want_hT=True)


N1_CASES = [((2, 300, 96), torch.float32, 0.0), ((2, 300, 96), torch.float32, 0.5),
            ((3, 1000, 130), torch.bfloat16, 0.3), ((1, 37, 64), torch.float32, 0.5),
            ((2, 64, 256), torch.float32, 0.0), ((2, 65, 256), torch.bfloat16, 0.0),
            ((1, 4100, 200), torch.float16, 0.2)]


@pytest.mark.parametrize("grad", [False, True])
@pytest.mark.parametrize("shape,dtype,h0_std", N1_CASES)
def test_final_state_n1(gpu, shape, dtype, h0_std, grad):
    ins = rand_inputs(*shape, 1, seed=sum(shape), dtype=dtype, h0_std=h0_std)
    y, hT = _hip(ins, gpu, grad)
    ry, rT = _oracle_y_hT(ins)
    assert hT.shape == (shape[0], shape[2], 1) and hT.dtype == torch.float32
    check("hT", hT, rT, tol_for(torch.float32))
    check("y", y, ry, tol_for(y.dtype))


# (batch, T, D, N): small grids take the segmented forward (T split into
# time segments, the final state written by the last one); 8 x 1536 at
# N = 64 and 8 x 6144 at N = 16 take the unsegmented four-states-per-lane one
GN_CASES = [(2, 300, 96, 16), (2, 300, 96, 64), (1, 1000, 64, 48), (2, 77, 70, 3), (1, 100, 64, 128),
            (8, 70, 1536, 64), (8, 45, 6144, 16)]


@pytest.mark.parametrize("grad", [False, True])
@pytest.mark.parametrize("shape", GN_CASES)
def test_final_state_and_no_grad_forward_general_n(gpu, shape, grad):
    b, T, D, N = shape
    wide = b * D >= 8 * 1536
    ins = rand_inputs(b, T, D, N, seed=T + D + N, h0_std=0.4,
                      **(dict(dtype=torch.bfloat16, gate_dtype=torch.float32, bc_dtype=torch.bfloat16)
                         if wide else {}))
    y, hT = _hip(ins, gpu, grad)
    ry, rT = _oracle_y_hT(ins)
    assert hT.shape == (b, D, N)
    check("hT", hT, rT, tol_for(torch.float32))
    check("y", y, ry, tol_for(y.dtype))


@pytest.mark.parametrize("N", [1, 16, 64])
def test_streaming_resume_from_final_state(gpu, N):
    """Scanning T in two pieces, the second from the first's final state,
    gives the one-piece result: the decode-time use of hT and h0."""
    from naju_amd import naju_scan_hip
    ins = rand_inputs(2, 500, 128, N, seed=N + 3, h0_std=0.3)
    x = {k: ins[k].to(gpu) for k in NAMES}
    h0 = ins["h0"].to(gpu)
    cut = 213
    with torch.no_grad():
        y_all, hT_all = naju_scan_hip(*[x[k] for k in NAMES], h0, return_final_state=True)
        part = lambda k, sl: x[k][:, sl] if x[k].dim() == 3 else x[k]  # noqa: E731
        y1, h1 = naju_scan_hip(*[part(k, slice(0, cut)) for k in NAMES], h0, return_final_state=True)
        y2, h2 = naju_scan_hip(*[part(k, slice(cut, None)) for k in NAMES], h1, return_final_state=True)
    ry, rT = _oracle_y_hT(ins)
    check("y_pieces", torch.cat([y1, y2], 1), ry, tol_for(torch.float32))
    check("hT_pieces", h2, rT, tol_for(torch.float32))
    check("hT_all", hT_all, rT, tol_for(torch.float32))
    assert torch.allclose(torch.cat([y1, y2], 1), y_all, rtol=0, atol=1e-5 * float(y_all.abs().max()))


def test_final_state_of_empty_sequence_is_h0(gpu):
    from naju_amd import naju_scan_hip
    h0 = torch.randn(2, 8, 4, device=gpu)
    z = lambda *s: torch.zeros(*s, device=gpu)  # noqa: E731
    y, hT = naju_scan_hip(z(2, 0, 8), z(2, 0, 8), z(2, 0, 8), z(2, 0, 4), z(2, 0, 4), z(8), h0,
                          return_final_state=True)
    torch.cuda.synchronize()
    assert y.shape == (2, 0, 8)
    assert torch.equal(hT, h0)


@pytest.mark.parametrize("N", [1, 64])
def test_no_grad_forward_matches_training_forward(gpu, N):
    """The forward without a checkpoint (no_grad) gives the training
    forward's y bit for bit (general N) or to float32 rounding (N = 1, whose
    chunk carries compose in arrival order)."""
    from naju_amd import naju_scan_hip
    ins = rand_inputs(2, 700, 192, N, seed=N + 11, h0_std=0.2)
    x = {k: ins[k].to(gpu).requires_grad_(True) for k in NAMES}
    h0 = ins["h0"].to(gpu)
    y_train = naju_scan_hip(*[x[k] for k in NAMES], h0)
    with torch.no_grad():
        y_inf = naju_scan_hip(*[x[k].detach() for k in NAMES], h0)
    torch.cuda.synchronize()
    if N > 1:
        assert torch.equal(y_train.detach(), y_inf)
    ry, _ = oracle_all(ins)
    check_all(y_inf, {}, ry, {})
    d = (y_train.detach() - y_inf).abs().max().item()
    assert d <= 1e-6 * max(1.0, float(np.abs(ry).max()))
