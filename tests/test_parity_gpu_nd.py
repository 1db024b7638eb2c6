"""GPU parity of the general-N scan (N >= 2, lanes over the state index)
against the fp64 oracle, through the C ABI; tolerances as in
tests/_helpers.tol_for. Shapes follow the reference's own matrix
(naju/tests/test_affine_chunk.py:84-86, test_gpu_smoke.py:29): N up to 128,
ragged T, D not a multiple of the 64-channel tile, N not a power of two."""
import numpy as np
import pytest
import torch

from tests._helpers import check_all, oracle_all, rand_inputs, run_abi, run_hip

pytestmark = pytest.mark.gpu

SHAPES = [(1, 7, 32, 16), (2, 64, 64, 4), (2, 65, 96, 16), (1, 129, 96, 32), (2, 192, 128, 64),
          (1, 100, 64, 128), (2, 33, 70, 3), (2, 256, 64, 64), (1, 40, 200, 2)]


@pytest.mark.parametrize("shape", SHAPES)
def test_fp32_general_n(gpu, shape):
    b, T, D, N = shape
    ins = rand_inputs(b, T, D, N, seed=T + D + N)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("N", [8, 64])
def test_h0_general_n(gpu, N):
    ins = rand_inputs(2, 150, 96, N, seed=N, h0_std=0.5)
    y, g = run_hip(ins, gpu)
    assert g["dh0"].shape == (2, 96, N)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("dtype,gate_dtype", [(torch.bfloat16, None), (torch.bfloat16, torch.float32),
                                              (torch.float16, None)])
def test_half_general_n(gpu, dtype, gate_dtype):
    ins = rand_inputs(2, 300, 128, 64, seed=5, dtype=dtype, gate_dtype=gate_dtype)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("N", [16, 64])
def test_half_inputs_f32_outputs_general_n(gpu, N):
    ins = rand_inputs(2, 200, 96, N, seed=9, dtype=torch.bfloat16, gate_dtype=torch.float32, h0_std=0.2)
    y, g = run_abi(ins, gpu, out_f32=True)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


def test_mixer_call_shape_and_dtypes(gpu):
    """NajuMixer's call (mixer.py:121-122) under bf16 autocast: u, B, C bf16,
    logits fp32, D_skip = zeros fp32, N = 64 (mixer.py:62); forget bias +5,
    input bias -2 (mixer.py:91,95)."""
    ins = rand_inputs(2, 256, 192, 64, seed=31, dtype=torch.bfloat16, gate_dtype=torch.float32,
                      f_shift=5.0, i_shift=-2.0, d_scale=0.0)
    y, g = run_hip(ins, gpu)
    assert y.dtype == torch.bfloat16 and g["dfl"].dtype == torch.float32
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


def test_edge_gates_general_n(gpu):
    import math
    ins = rand_inputs(2, 130, 64, 16, seed=11, f_shift=0.0)
    gsel = torch.Generator().manual_seed(12)
    sel = torch.rand(2, 130, 64, generator=gsel)
    fl = ins["f_logit"] * 2.0
    fl[sel < 0.1] = -math.inf
    fl[sel >= 0.9] = math.inf
    ins["f_logit"] = fl
    y, gr = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, gr, ry, rg)
    assert torch.all(gr["dfl"].cpu()[(sel < 0.1) | (sel >= 0.9)] == 0)


def test_ratio_and_exact_decay_paths(gpu):
    """The matrix-core kernels form the in-sub-block decay terms as ratios
    of running products when every channel of a 16-channel group keeps its
    16-row decay at or above 2^-30, as exact products otherwise. Channel
    groups here sit just above the bound (1/Pf up to 2^29), just below it
    in one channel only, well inside, and far below; all against the
    oracle at the fp32 tolerance."""
    import math
    b, T, D, N = 2, 70, 64, 32
    ins = rand_inputs(b, T, D, N, seed=21, h0_std=0.3)
    logit = lambda f: math.log(f / (1.0 - f))  # noqa: E731
    fl = ins["f_logit"].clone()
    fl[:, :, 0:16] = logit(2.0 ** (-29.0 / 16.0)) + 0.001 * fl[:, :, 0:16]   # product about 2^-29
    fl[:, :, 16:32] = fl[:, :, 16:32] + 0.0                                   # the recipe's gates
    fl[:, :, 16] = logit(2.0 ** (-31.0 / 16.0))                               # one channel below 2^-30
    fl[:, :, 48:64] = logit(0.05) + 0.1 * fl[:, :, 48:64]                     # far below
    ins["f_logit"] = fl
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)


@pytest.mark.parametrize("shape", [(2, 200, 130, 64), (4, 2048, 512, 64), (2, 1024, 256, 32)])
def test_deterministic_general_n(gpu, shape):
    """No look-back and fixed-order sums: repeated runs are bitwise identical.
    With bf16 B / C the matrix-core kernels take G = C B^T and the products
    with one bf16 operand on the 16-bit MFMA; a register hazard there shows
    as run-to-run differences, so the larger shapes (many segments, every
    wave busy) run three times."""
    ins = rand_inputs(*shape, seed=13, dtype=torch.bfloat16)
    y1, g1 = run_abi(ins, gpu, out_f32=True)
    for _ in range(2):
        y2, g2 = run_abi(ins, gpu, out_f32=True)
        assert torch.equal(y1, y2)
        for k in g1:
            assert torch.equal(g1[k], g2[k]), k


def test_golden_oracle_n4(gpu):
    import os
    from tests._helpers import check, tol_for
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_n4.npz")
    with np.load(path) as z:
        fx = {k: z[k] for k in z.files}
    ins = {k: torch.from_numpy(fx[k]) for k in ("u", "f_logit", "i_logit", "B", "C", "D_skip", "h0", "dy")}
    y, g = run_hip(ins, gpu)
    check("y", y, fx["y"], tol_for(torch.float32))
    for k in ("du", "dfl", "dil", "dB", "dC", "dD", "dh0"):
        check(k, g[k], fx[k], tol_for(torch.float32))


def test_full_size_c2_n64_channel_slice(gpu):
    """Benchmark configuration c2 at the mixer's N = 64, full size on the GPU; 24
    channels checked against the per-channel oracle (y, du, dfl, dil, dh0 are
    per-channel), dD against sum(dy*u)."""
    from naju_amd.workloads import config_inputs
    from oracle.scan_ref import oracle_bwd_channels, oracle_fwd_channels
    ins = config_inputs("c2", N=64, seed=2, device=gpu)
    y, g = run_hip(ins, gpu)
    rng = np.random.default_rng(0)
    Bsz, T, D = ins["u"].shape
    chans = np.sort(rng.choice(Bsz * D, size=24, replace=False))
    cpu = {k: (v.float().cpu() if v is not None else None) for k, v in ins.items()}
    args = [cpu[k] for k in ("u", "f_logit", "i_logit", "B", "C", "D_skip")]
    ry = oracle_fwd_channels(*args, chans=chans, h0=cpu["h0"])
    rg = oracle_bwd_channels(*args, dy=cpu["dy"], chans=chans, h0=cpu["h0"])
    from tests._helpers import check, tol_for
    bb, dd = chans // D, chans % D
    check("y", y.detach().float().cpu().numpy()[bb, :, dd], ry, tol_for(y.dtype))
    for k in ("du", "dfl", "dil"):
        check(k, g[k].float().cpu().numpy()[bb, :, dd], rg[k], tol_for(g[k].dtype))
    check("dh0", g["dh0"].cpu().numpy()[bb, dd], rg["dh0"], tol_for(torch.float32))
    ref_dD = (ins["dy"].float() * ins["u"].float()).sum((0, 1)).double().cpu().numpy()
    assert np.max(np.abs(g["dD"].double().cpu().numpy() - ref_dD)) <= 1e-4 * max(1.0, np.abs(ref_dD).max())


@pytest.mark.parametrize("N,D", [(48, 1536), (32, 3072), (16, 6144)])
def test_wide_grid_forward_general_n(gpu, N, D):
    """Batch x channel grids that fill the GPU on their own take the forward
    with four states per lane and no time segments (the C5 layer is one:
    8 x 1536 channels at N = 64): ragged T, N below its power-of-two tile,
    h0, and the mixer's dtypes (bf16 u, B, C; f32 gates)."""
    ins = rand_inputs(8, 70, D, N, seed=N, dtype=torch.bfloat16, gate_dtype=torch.float32,
                      bc_dtype=torch.bfloat16, h0_std=0.3)
    y, g = run_hip(ins, gpu)
    ry, rg = oracle_all(ins)
    check_all(y, g, ry, rg)
