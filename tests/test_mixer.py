"""CPU tests of the restated mixer / block / LM (naju_amd/mixer.py).

The scan runs through a test-only backend, the oracle loop
(oracle/scan_ref.py:scan_loop_torch, the algorithm of reference
naju/scan.py:79-93), inserted into naju_amd.scan's backend cache the way the
reference's own dispatcher accepts pre-registered entries (scan.py:55-57).
"""
import math

import pytest
import torch

from naju_amd import scan as scan_mod
from naju_amd.mixer import NajuBlock, NajuLM, NajuMixer, RMSNorm, build_optimizer
from oracle.scan_ref import scan_loop_torch


@pytest.fixture(autouse=True)
def oracle_backend(monkeypatch):
    monkeypatch.setitem(scan_mod._BACKEND_CACHE, "oracle_loop", scan_loop_torch)


# Parameter names and shapes of the reference modules for d_model=8,
# d_state=4, d_conv=4, expand=2 (naju/mixer.py:73-95): checkpoints must load
# with strict=True in both directions.
MIXER_KEYS = {
    "D": (16,), "f_bias": (16,), "i_bias": (16,),
    "in_proj.weight": (32, 8),
    "conv1d.weight": (16, 1, 4), "conv1d.bias": (16,),
    "x_proj.weight": (8, 16), "out_proj.weight": (8, 16),
    "f_proj.weight": (16, 16), "f_conv.weight": (16, 1, 4),
    "i_proj.weight": (16, 16), "i_conv.weight": (16, 1, 4),
}


def test_mixer_state_dict_layout():
    m = NajuMixer(8, d_state=4)
    sd = m.state_dict()
    assert {k: tuple(v.shape) for k, v in sd.items()} == MIXER_KEYS
    assert "D_zero" not in sd  # non-persistent buffer, like the reference
    assert float(m.f_bias[0].detach()) == 5.0 and float(m.i_bias[0].detach()) == -2.0
    assert float(m.D[0].detach()) == pytest.approx(0.01)


def test_low_rank_gate_names():
    m = NajuMixer(8, d_state=4, gate_rank=3)
    sd = m.state_dict()
    assert tuple(sd["f_proj.0.weight"].shape) == (3, 16) and tuple(sd["f_proj.1.weight"].shape) == (16, 3)
    with pytest.raises(ValueError, match="incompatible"):
        NajuMixer(8, gate_rank=3, gate_reparam=True)


def test_lm_tied_head_and_names():
    lm = NajuLM(50, d_model=8, n_layers=2, d_state=4)
    assert lm.head.weight is lm.embed.weight
    names = set(lm.state_dict())
    assert "blocks.1.mixer.in_proj.weight" in names and "blocks.0.norm.weight" in names
    assert "norm.weight" in names and "embed.weight" in names


def test_rmsnorm_closed_form():
    x = torch.randn(3, 5, 7, dtype=torch.float64)
    n = RMSNorm(7).double()
    with torch.no_grad():
        n.weight.copy_(torch.linspace(0.5, 2.0, 7, dtype=torch.float64))
    ref = n.weight * x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-5)
    torch.testing.assert_close(n(x), ref, rtol=1e-12, atol=1e-12)


def test_causal_dwconv_matches_padded_conv():
    """Left-padded valid convolution == symmetric padding k-1 then the first
    T outputs (the reference's form, naju/mixer.py:108-109,115)."""
    from naju_amd.mixer import _causal_dwconv
    torch.manual_seed(0)
    conv = torch.nn.Conv1d(6, 6, 4, groups=6, bias=True).double()
    x = torch.randn(2, 11, 6, dtype=torch.float64)
    ref = torch.nn.functional.conv1d(x.transpose(1, 2), conv.weight, conv.bias, padding=3, groups=6)[..., :11]
    torch.testing.assert_close(_causal_dwconv(x, conv), ref.transpose(1, 2))


def test_lm_is_causal():
    torch.manual_seed(0)
    lm = NajuLM(40, d_model=8, n_layers=2, dropout=0.0, d_state=4, scan_backend="oracle_loop").double()
    ids = torch.randint(0, 40, (2, 12))
    ids2 = ids.clone()
    ids2[:, 7] = (ids2[:, 7] + 1) % 40
    with torch.no_grad():
        a, b = lm(ids), lm(ids2)
    torch.testing.assert_close(a[:, :7], b[:, :7], rtol=0, atol=0)
    assert not torch.allclose(a[:, 7:], b[:, 7:])


def test_gate_reparam_same_forward_at_init():
    torch.manual_seed(1)
    m0 = NajuMixer(8, d_state=4, scan_backend="oracle_loop").double()
    torch.manual_seed(1)
    m1 = NajuMixer(8, d_state=4, gate_reparam=True, scan_backend="oracle_loop").double()
    x = torch.randn(2, 9, 8, dtype=torch.float64)
    with torch.no_grad():
        torch.testing.assert_close(m0(x), m1(x), rtol=1e-12, atol=1e-12)


def test_mixer_readout_scale_and_skip():
    """With the input gate closed (i_bias = -inf, so i = 0 exactly) the scan
    adds nothing and the mixer output is exactly out_proj(D * h * SiLU(z)):
    this pins the D skip outside the scan and the z-gate."""
    torch.manual_seed(2)
    m = NajuMixer(4, d_state=4, scan_backend="oracle_loop").double()
    with torch.no_grad():
        m.i_bias.fill_(-float("inf"))
        m.D.fill_(0.5)
    u = torch.randn(1, 6, 4, dtype=torch.float64)
    x, z = m.in_proj(u).chunk(2, dim=-1)
    from naju_amd.mixer import _causal_dwconv
    h = torch.nn.functional.silu(_causal_dwconv(x, m.conv1d))
    ref = m.out_proj(0.5 * h * torch.nn.functional.silu(z))
    with torch.no_grad():
        torch.testing.assert_close(m(u), ref, rtol=1e-12, atol=1e-12)
    assert m._cx_scale == pytest.approx(1 / math.sqrt(4))


def test_lm_init_loss_near_log_vocab_and_backward():
    torch.manual_seed(3)
    V = 64
    lm = NajuLM(V, d_model=16, n_layers=2, d_state=4, scan_backend="oracle_loop")
    ids = torch.randint(0, V, (2, 16))
    logits = lm(ids)
    loss = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, V), ids[:, 1:].reshape(-1))
    assert abs(float(loss.detach()) - math.log(V)) < 0.2
    loss.backward()
    assert all(p.grad is not None and torch.isfinite(p.grad).all() for p in lm.parameters())


def test_block_checkpoint_same_grads():
    torch.manual_seed(4)
    b0 = NajuBlock(8, dropout=0.0, d_state=4, scan_backend="oracle_loop").double()
    b1 = NajuBlock(8, dropout=0.0, use_ckpt=True, d_state=4, scan_backend="oracle_loop").double()
    b1.load_state_dict(b0.state_dict())
    x = torch.randn(2, 7, 8, dtype=torch.float64, requires_grad=True)
    x1 = x.detach().clone().requires_grad_(True)
    b0(x).sum().backward()
    b1(x1).sum().backward()
    torch.testing.assert_close(x.grad, x1.grad)
    for p0, p1 in zip(b0.parameters(), b1.parameters()):
        torch.testing.assert_close(p0.grad, p1.grad)


def test_build_optimizer_groups():
    lm = NajuLM(30, d_model=8, n_layers=2, d_state=4)
    opt = build_optimizer(lm, lr=1e-3)
    assert len(opt.param_groups) == 1
    lm2 = NajuLM(30, d_model=8, n_layers=2, d_state=4, gate_reparam=True)
    opt2 = build_optimizer(lm2, lr=1e-3, weight_decay=0.1)
    g = opt2.param_groups[1]
    mult = math.sqrt(16)
    assert g["lr"] == pytest.approx(1e-3 * mult) and g["weight_decay"] == pytest.approx(0.1 / mult)
    assert g["eps"] == pytest.approx(1e-8 / mult) and len(g["params"]) == 4


def test_linear_token_parts_rule():
    """The split-K weight gradient's token parts (naju_amd.linear._parts)."""
    from naju_amd.linear import _parts
    assert _parts(16384, 768, 1536) == 8
    assert _parts(16384, 3200, 1536) == 2
    assert _parts(16384, 3072, 768) == 4
    assert _parts(666, 40, 96) == 1          # too few tokens per part
    assert _parts(16384, 50257, 768) == 1    # many output tiles already
