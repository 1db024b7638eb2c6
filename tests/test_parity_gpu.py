"""GPU parity of the HIP scan (through the C ABI) against the fp64 oracle.

Tolerances (tests/_helpers.tol_for), on max-abs error / max|oracle| and
||err||_2 / ||oracle||_2: float32 outputs 1e-5 (also for bf16/fp16 inputs
with float32 outputs); bf16 outputs 2e-3 norm-wise with the max-norm bounded
by bf16 storage rounding (2^-8); fp16 outputs 2e-3. The oracle runs on the
same (already quantized) inputs, upcast -- the practice of reference
naju/tests/test_affine_chunk.py:149-153.
"""
import math

import numpy as np
import pytest
import torch

from tests._helpers import GRAD_KEYS, check_all, oracle_all, rand_inputs, run_abi, run_hip

pytestmark = pytest.mark.gpu

# (batch, T, D): single chunk, ragged T, D not a multiple of the lane width,
# several tiles, long-ish T -- the reference's shape matrix style
# (naju/tests/test_affine_chunk.py:84-86).
SHAPES_N1 = [(1, 7, 32), (2, 64, 64), (2, 65, 96), (1, 129, 96), (3, 200, 40),
             (2, 33, 1000), (2, 1024, 256), (8, 256, 512)]


@pytest.mark.parametrize("shape", SHAPES_N1)
def test_fp32_n1_shapes(gpu, shape):
    b, T, D = shape
    ins = rand_inputs(b, T, D, 1, seed=T + D)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("dtype,gate_dtype", [(torch.bfloat16, None), (torch.float16, None),
                                              (torch.bfloat16, torch.float32),
                                              (torch.float16, torch.float32)])
def test_half_n1(gpu, dtype, gate_dtype):
    ins = rand_inputs(4, 512, 128, 1, seed=5, dtype=dtype, gate_dtype=gate_dtype)
    y, g = run_hip(ins, gpu)
    assert y.dtype == dtype
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("dtype,gate_dtype", [(torch.bfloat16, None), (torch.float16, None),
                                              (torch.bfloat16, torch.float32)])
def test_half_inputs_f32_outputs(gpu, dtype, gate_dtype):
    """bf16/fp16 inputs, float32 outputs through the C ABI (out_f32=1): with
    storage rounding out of the way, every output matches the oracle on the
    same quantized inputs to the float32 tolerance 1e-5."""
    ins = rand_inputs(4, 512, 128, 1, seed=5, dtype=dtype, gate_dtype=gate_dtype, h0_std=0.2)
    y, g = run_abi(ins, gpu, out_f32=True)
    assert y.dtype == torch.float32 and all(v.dtype == torch.float32 for v in g.values())
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


def test_bf16_u_bc_f32_gates_mixer_dtypes(gpu):
    """Autocast dtypes at the mixer's call (u, B, C bf16; logits fp32;
    D_skip fp32)."""
    ins = rand_inputs(2, 300, 192, 1, seed=21, dtype=torch.bfloat16, gate_dtype=torch.float32)
    y, g = run_hip(ins, gpu)
    assert g["dfl"].dtype == torch.float32 and g["du"].dtype == torch.bfloat16
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_h0(gpu, dtype):
    ins = rand_inputs(3, 257, 192, 1, seed=3, dtype=dtype, h0_std=0.5)
    y, g = run_hip(ins, gpu)
    assert "dh0" in g and g["dh0"].shape == (3, 192, 1)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


# Odd D: a lane's two channels are not a whole vector, so both directions
# take the element-wise load / store path (every channel checked against D);
# with ragged T, h0 and partial channel tiles.
@pytest.mark.parametrize("shape", [(2, 70, 33), (1, 129, 7), (3, 65, 131)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_n1_odd_channels_elementwise_path(gpu, shape, dtype):
    b, T, D = shape
    ins = rand_inputs(b, T, D, 1, seed=T * D, dtype=dtype, h0_std=0.3)
    if dtype == torch.float32:
        y, g = run_hip(ins, gpu)
    else:
        # bf16 inputs with float32 outputs: the kernels' arithmetic at the
        # float32 bound. (With bf16 outputs, the storage rounding of the few
        # dB / dC entries of these small shapes alone comes close to the bf16
        # norm-wise tolerance.)
        y, g = run_abi(ins, gpu, out_f32=True)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


# Even D but streams that start one element past an aligned address: the
# vector path needs every stream aligned to its vector width, so this also
# runs element-wise (and the outputs, freshly allocated, are aligned).
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_n1_misaligned_streams(gpu, dtype):
    from naju_amd import naju_scan_hip

    b, T, D = 2, 97, 256
    ins = rand_inputs(b, T, D, 1, seed=11, dtype=dtype, h0_std=0.2)
    names = ["u", "f_logit", "i_logit", "B", "C", "D_skip", "h0"]
    xs = {}
    for k in names:
        t = ins[k].to(gpu)
        buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=gpu)
        buf[1:].copy_(t.reshape(-1))
        xs[k] = buf[1:].view(t.shape).detach().requires_grad_(True)
    # one element past an allocation: not aligned to two elements
    assert xs["u"].data_ptr() % (2 * xs["u"].element_size()) != 0
    y = naju_scan_hip(*[xs[k] for k in names[:6]], xs["h0"])
    y.backward(ins["dy"].to(gpu))
    torch.cuda.synchronize()
    grads = {GRAD_KEYS[k]: xs[k].grad for k in names}
    ry, rg = oracle_all(ins)
    check_all(y, grads, ry, rg)


def test_edge_gates_exact_zero_one(gpu):
    """a forced to exactly 0 (f_logit=-inf) and 1 (+inf) on 10% each: the
    scan stays finite and exact, and dfl is exactly 0 there (f(1-f) = 0)."""
    ins = rand_inputs(2, 400, 256, 1, seed=11, dtype=torch.bfloat16, f_shift=0.0)
    g = torch.Generator().manual_seed(12)
    sel = torch.rand(2, 400, 256, generator=g)
    fl = ins["f_logit"].float() * 2.0
    fl[sel < 0.1] = -math.inf
    fl[sel >= 0.9] = math.inf
    ins["f_logit"] = fl.to(torch.bfloat16)
    y, gr = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, gr, ry, rg)
    hard = (sel < 0.1) | (sel >= 0.9)
    assert torch.all(gr["dfl"].float().cpu()[hard] == 0)


def test_deep_gates(gpu):
    """f ~ sigmoid(-12): the guard region of the reference chunk backend
    (naju/tests/test_affine_chunk.py:101-115, :172-194)."""
    ins = rand_inputs(2, 256, 64, 1, seed=7, f_shift=-12.0)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


def test_long_sequence_near_one(gpu):
    """Long T with retention near 1: cross-chunk carries dominate."""
    ins = rand_inputs(1, 32768, 64, 1, seed=11, f_shift=4.0)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("shape", [(4, 700, 320), (2, 4096, 1024)])
def test_deterministic_flag_bitwise(gpu, shape):
    """NAJU_FLAG_DETERMINISTIC: every chunk takes its carry from its immediate
    predecessor, so repeated runs are bitwise identical (including the full
    C2 sequence length with 64 forward / 128 backward chunks), and the
    results still match the oracle."""
    B, T, D = shape
    ins = rand_inputs(B, T, D, 1, seed=17, dtype=torch.bfloat16)
    y1, g1 = run_abi(ins, gpu, out_f32=True, deterministic=True)
    y2, g2 = run_abi(ins, gpu, out_f32=True, deterministic=True)
    assert torch.equal(y1, y2)
    for k in g1:
        assert torch.equal(g1[k], g2[k]), k
    if T <= 1024:
        ry, rg = oracle_all(ins)
        check_all(y1.cpu(), {k: v.cpu() for k, v in g1.items()}, ry, rg)


def test_torch_deterministic_mode_selects_flag(gpu):
    """torch.use_deterministic_algorithms(True) makes the Python backend pass
    NAJU_FLAG_DETERMINISTIC: two autograd runs agree bitwise."""
    ins = rand_inputs(2, 1500, 256, 1, seed=19, dtype=torch.bfloat16)
    prev = torch.are_deterministic_algorithms_enabled()
    torch.use_deterministic_algorithms(True)
    try:
        y1, g1 = run_hip(ins, gpu)
        y2, g2 = run_hip(ins, gpu)
    finally:
        torch.use_deterministic_algorithms(prev)
    assert torch.equal(y1, y2)
    for k in g1:
        if g1[k] is not None:
            assert torch.equal(g1[k], g2[k]), k


def test_repeatable_and_workspace_reusable(gpu):
    """Two identical runs agree to float32 rounding. (Chunk carries are
    composed in the order the decoupled look-back meets its predecessors,
    which depends on timing, so results are not bitwise identical; the
    channel/batch reductions dB, dC, dD use a fixed order.) The workspace
    status word stays healthy across reuse."""
    ins = rand_inputs(4, 700, 320, 1, seed=13, dtype=torch.bfloat16)
    y1, g1 = run_abi(ins, gpu, out_f32=True)
    y2, g2 = run_abi(ins, gpu, out_f32=True)
    assert (y1 - y2).abs().max().item() <= 1e-6 * y1.abs().max().item()
    for k in g1:
        assert (g1[k] - g2[k]).abs().max().item() <= 1e-6 * g1[k].abs().max().item(), k
    run_hip(ins, gpu)
    run_hip(ins, gpu)
    from naju_amd import _lib
    from naju_amd.scan import _WS
    import ctypes
    for (dev, stream), buf in _WS._bufs.items():
        st = ctypes.c_uint32(99)
        _lib.check(_lib.lib().naju_scan_workspace_status(buf.data_ptr(), stream, ctypes.byref(st)))
        assert st.value == 0


def test_workspace_shared_across_shapes(gpu):
    """One cached workspace serves shapes whose tile counts grow from call to
    call (regression: the ticket counters live in a fixed header region that
    no other part of any layout overlaps). Status stays 0 throughout."""
    import ctypes
    from naju_amd import _lib
    from naju_amd.scan import _WS
    for (b, T, D) in [(1, 40, 32), (3, 200, 40), (2, 33, 1000), (4, 130, 2000), (1, 300, 64)]:
        ins = rand_inputs(b, T, D, 1, seed=b * T + D)
        y, g = run_hip(ins, gpu)
        ry, rg = oracle_all(ins)
        check_all(y, g, ry, rg)
    for (dev, stream), buf in _WS._bufs.items():
        st = ctypes.c_uint32(99)
        _lib.check(_lib.lib().naju_scan_workspace_status(buf.data_ptr(), stream, ctypes.byref(st)))
        assert st.value == 0


def test_needs_input_grad_subset(gpu):
    ins = rand_inputs(2, 100, 64, 1, seed=17)
    y, g = run_hip(ins, gpu, grad_names=["u", "f_logit"])
    assert set(g) == {"du", "dfl"}
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


def test_no_grad_forward(gpu):
    ins = rand_inputs(2, 300, 128, 1, seed=19)
    y, _ = run_hip(ins, gpu, grad=False)
    ry, _ = oracle_all(ins)
    check_all(y, {}, ry, {})


def test_register_into_reference_style_dispatch(gpu):
    """register() inserts the backend into a scan module's _BACKEND_CACHE;
    dispatch by name then reaches the HIP kernels (scan.py:55-57, :75-76)."""
    import types
    from naju_amd import register
    fake = types.SimpleNamespace(_BACKEND_CACHE={})
    fn = register("HIP", scan_module=fake)
    assert fake._BACKEND_CACHE["hip"] is fn
    ins = rand_inputs(1, 50, 64, 1, seed=23)
    args = [ins[k].to(gpu) for k in ("u", "f_logit", "i_logit", "B", "C", "D_skip")]
    y = fake._BACKEND_CACHE["hip"](*args)
    ry, _ = oracle_all(ins)
    check_all(y, {}, ry, {})


def test_empty_time_axis(gpu):
    from naju_amd import naju_scan_hip
    u = torch.zeros(2, 0, 8, device=gpu, requires_grad=True)
    fl = torch.zeros(2, 0, 8, device=gpu, requires_grad=True)
    il = torch.zeros(2, 0, 8, device=gpu, requires_grad=True)
    B = torch.zeros(2, 0, 1, device=gpu, requires_grad=True)
    C = torch.zeros(2, 0, 1, device=gpu, requires_grad=True)
    Dk = torch.ones(8, device=gpu, requires_grad=True)
    y = naju_scan_hip(u, fl, il, B, C, Dk)
    assert y.shape == (2, 0, 8)
    y.sum().backward()
    assert torch.all(Dk.grad == 0)


@pytest.mark.parametrize("name", ["c2"])
def test_full_size_batch_row_slice(gpu, name):
    """Full benchmark size on the GPU; batch row 0 checked in full against the
    oracle (every output except dD depends only on its own batch row), dD
    checked against sum(dy*u) over the whole batch."""
    from naju_amd.workloads import config_inputs
    ins = config_inputs(name, N=1, seed=1, device=gpu)
    y, g = run_hip(ins, gpu)
    row = {k: (v[:1].cpu() if v is not None and k != "D_skip" else v) for k, v in ins.items()}
    row["D_skip"] = ins["D_skip"].cpu()
    ry, rg = oracle_all(row)
    g0 = {k: v[:1] for k, v in g.items() if k != "dD"}
    check_all(y[:1], g0, ry, rg)
    ref_dD = (ins["dy"].float() * ins["u"].float()).sum((0, 1)).double().cpu().numpy()
    out_dD = g["dD"].double().cpu().numpy()
    assert np.max(np.abs(out_dD - ref_dD)) <= 1e-4 * max(1.0, np.abs(ref_dD).max())
