"""GPU tests: the restated mixer and LM (naju_amd/mixer.py) with the HIP scan
against the same modules with the oracle loop scan (oracle/scan_ref.py,
reference naju/scan.py:79-93) on identical weights and inputs."""
import pytest
import torch

from naju_amd import scan as scan_mod
from naju_amd.mixer import NajuLM, NajuMixer
from oracle.scan_ref import scan_loop_torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def oracle_backend(monkeypatch):
    monkeypatch.setitem(scan_mod._BACKEND_CACHE, "oracle_loop", scan_loop_torch)


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _twin(make, backend_a, backend_b, dev):
    torch.manual_seed(0)
    ma = make(backend_a).to(dev)
    mb = make(backend_b).to(dev)
    mb.load_state_dict(ma.state_dict())
    return ma, mb


@pytest.mark.parametrize("d_state", [1, 16, 64])
def test_mixer_fp32_hip_matches_oracle(gpu, d_state):
    dev = torch.device("cuda", 0)
    ma, mb = _twin(lambda be: NajuMixer(32, d_state=d_state, scan_backend=be), "hip", "oracle_loop", dev)
    torch.manual_seed(1)
    u = torch.randn(2, 80, 32, device=dev)
    ua, ub = u.clone().requires_grad_(True), u.clone().requires_grad_(True)
    ya, yb = ma(ua), mb(ub)
    g = torch.randn_like(ya)
    ya.backward(g)
    yb.backward(g)
    assert _rel(ya, yb) < 1e-5
    assert _rel(ua.grad, ub.grad) < 1e-5
    for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
        assert _rel(pa.grad, pb.grad) < 1e-4, n


def test_lm_bf16_autocast_hip_matches_oracle(gpu):
    """The mixer's autocast dtypes reach the kernels as they do in training
    (u, B, C bf16; gate logits f32). Both runs compute the scan in f32 from
    the same bf16 inputs; the HIP scan returns bf16 (u's dtype), so the
    comparison allows bf16 rounding."""
    dev = torch.device("cuda", 0)
    V = 128
    ma, mb = _twin(lambda be: NajuLM(V, d_model=32, n_layers=2, dropout=0.0, d_state=16, scan_backend=be),
                   "hip", "oracle_loop", dev)
    torch.manual_seed(2)
    ids = torch.randint(0, V, (2, 64), device=dev)
    losses = []
    for m in (ma, mb):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = m(ids)
            loss = torch.nn.functional.cross_entropy(logits[:, :-1].float().reshape(-1, V), ids[:, 1:].reshape(-1))
        loss.backward()
        losses.append(float(loss.detach()))
    assert abs(losses[0] - losses[1]) < 1e-3 * abs(losses[1])
    for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
        assert _rel(pa.grad, pb.grad) < 3e-2, n


def test_lm_train_step_reduces_loss(gpu):
    """A few AdamW steps on one batch with the HIP scan lower the loss."""
    dev = torch.device("cuda", 0)
    torch.manual_seed(3)
    V = 64
    lm = NajuLM(V, d_model=32, n_layers=2, dropout=0.0, d_state=16, scan_backend="hip").to(dev)
    opt = torch.optim.AdamW(lm.parameters(), lr=3e-3)
    ids = torch.randint(0, V, (4, 64), device=dev)
    first = None
    for _ in range(8):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = lm(ids)
            loss = torch.nn.functional.cross_entropy(logits[:, :-1].float().reshape(-1, V), ids[:, 1:].reshape(-1))
        opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(lm.parameters(), 1.0)
        opt.step()
        first = float(loss.detach()) if first is None else first
    assert float(loss.detach()) < first - 0.1


def test_lm_step_fused_loss_and_optimizer_match_reference_loop(gpu):
    """The C5 step's pieces: naju_amd.xent.cross_entropy on the bf16 logits
    and build_optimizer's AdamW with the clip inside its update
    (naju_amd.optim, step(max_grad_norm=1.0)) against the reference loop's
    cross_entropy on the float32 upcast, clip_grad_norm_ and torch's foreach
    AdamW (evals/lm/train.py:70-80), from the same weights and batch."""
    from naju_amd.mixer import build_optimizer
    from naju_amd.optim import AdamW as NajuAdamW
    from naju_amd.xent import cross_entropy
    dev = torch.device("cuda", 0)
    V = 97
    torch.manual_seed(5)
    ma = NajuLM(V, d_model=32, n_layers=2, dropout=0.0, d_state=8, scan_backend="hip").to(dev)
    mb = NajuLM(V, d_model=32, n_layers=2, dropout=0.0, d_state=8, scan_backend="hip").to(dev)
    mb.load_state_dict(ma.state_dict())
    oa = build_optimizer(ma, lr=1e-3)
    ob = torch.optim.AdamW(mb.parameters(), lr=1e-3, weight_decay=0.1, foreach=True)
    assert isinstance(oa, NajuAdamW)
    ids = torch.randint(0, V, (3, 40), device=dev)
    for step in range(3):
        losses = []
        for m, o, fused in ((ma, oa, True), (mb, ob, False)):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                logits = m(ids)[:, :-1].reshape(-1, V)
                tgt = ids[:, 1:].reshape(-1)
                loss = cross_entropy(logits, tgt) if fused else \
                    torch.nn.functional.cross_entropy(logits.float(), tgt)
            o.zero_grad(set_to_none=True)
            loss.backward()
            if fused:
                o.step(max_grad_norm=1.0)
            else:
                torch.nn.utils.clip_grad_norm_(m.parameters(), 1.0)
                o.step()
            losses.append(float(loss.detach()))
        assert abs(losses[0] - losses[1]) < 2e-3 * abs(losses[1]), (step, losses)
    for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
        assert _rel(pa.detach(), pb.detach()) < 1e-3, n


@pytest.mark.parametrize("gate_reparam", [False, True])
def test_block_cuda_fused_path_matches_cpu_reference_formulation(gpu, gate_reparam):
    """What the CUDA path fuses -- RMSNorm, the one GEMM for f_proj, i_proj
    and x_proj, the depthwise convolutions reading slices in place, the
    readout -- against the reference's own formulation (naju/mixer.py:51-144),
    which the CPU path keeps, on the same weights in float32; the scan is
    the float64-checked oracle loop on the CPU and the HIP kernels on the GPU."""
    import copy
    from naju_amd.mixer import NajuBlock
    torch.manual_seed(0)
    cpu = NajuBlock(32, dropout=0.0, d_state=16, gate_reparam=gate_reparam, scan_backend="oracle_loop")
    with torch.no_grad():
        for p in cpu.parameters():
            p.add_(0.05 * torch.randn_like(p))
    dev_blk = copy.deepcopy(cpu).cuda()
    dev_blk.mixer.scan_backend = "hip"
    torch.manual_seed(1)
    u = torch.randn(2, 70, 32)
    g = torch.randn(2, 70, 32)
    uc = u.clone().requires_grad_(True)
    ud = u.cuda().requires_grad_(True)
    yc, yd = cpu(uc), dev_blk(ud)
    yc.backward(g)
    yd.backward(g.cuda())
    assert _rel(yd.cpu(), yc) < 1e-5
    assert _rel(ud.grad.cpu(), uc.grad) < 1e-5
    for (n, pc), pd in zip(cpu.named_parameters(), dev_blk.parameters()):
        assert _rel(pd.grad.cpu(), pc.grad) < 1e-4, n


@pytest.mark.parametrize("d_state,dropout", [(16, 0.0), (1, 0.0), (64, 0.1)])
def test_lm_activation_checkpointing_on_hip_scan(gpu, d_state, dropout):
    """NajuBlock(use_ckpt=True) (reference naju/mixer.py:139-141) recomputes
    each block's branch, HIP scan included, in the backward: the loss and
    every gradient equal those of use_ckpt=False (bit for bit at N > 1,
    whose scan is run-to-run deterministic; to float32 rounding at N = 1;
    dropout masks are replayed from the saved RNG state)."""
    dev = torch.device("cuda", 0)
    V = 80
    ma, mb = _twin(lambda ck: NajuLM(V, d_model=32, n_layers=2, dropout=dropout, d_state=d_state,
                                     use_ckpt=ck, scan_backend="hip"), True, False, dev)
    torch.manual_seed(9)
    ids = torch.randint(0, V, (2, 96), device=dev)
    losses = []
    for m in (ma, mb):
        torch.manual_seed(10)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = m(ids)
            loss = torch.nn.functional.cross_entropy(logits[:, :-1].float().reshape(-1, V), ids[:, 1:].reshape(-1))
        loss.backward()
        losses.append(loss.detach())
    if d_state > 1:
        assert torch.equal(losses[0], losses[1])
    else:
        assert abs(float(losses[0]) - float(losses[1])) <= 1e-5 * abs(float(losses[1]))
    for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
        if d_state > 1:
            assert torch.equal(pa.grad, pb.grad), n
        else:
            assert _rel(pa.grad, pb.grad) < 1e-5, n


def test_lm_c5_full_size_training_steps(gpu):
    """Benchmark configuration c5 at full size: 12 layers, d_model 768,
    vocab 50257, N = 64, batch 8 x 2048 uniformly random token ids, bf16
    autocast, the fused cross-entropy, clip 1.0 and AdamW, every scan on the
    HIP kernels. Gradients stay finite, the fused loss equals torch's
    cross_entropy on the float32 upcast of the same logits, and three steps on
    the batch lower the loss to about ln(vocab). (At init it starts above
    ln(vocab): with the head tied to the embedding, N(0, 0.02) rows of width
    768 give each input token its own logit |e|^2 / rms(e), about 15.)"""
    import math
    from naju_amd.mixer import build_optimizer
    from naju_amd.xent import cross_entropy
    dev = torch.device("cuda", 0)
    V, T, Bsz = 50257, 2048, 8
    torch.manual_seed(0)
    lm = NajuLM(V, d_model=768, n_layers=12, dropout=0.1, scan_backend="hip").to(dev)
    assert lm.blocks[0].mixer.d_state == 64
    opt = build_optimizer(lm, lr=1e-3, weight_decay=0.1)
    ids = torch.randint(0, V, (Bsz, T + 1), device=dev)
    x, y = ids[:, :-1].contiguous(), ids[:, 1:].contiguous()
    losses = []
    for step in range(4):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = lm(x).view(-1, V)
            loss = cross_entropy(logits, y.view(-1))
        if step == 0:
            ref = torch.nn.functional.cross_entropy(logits.detach().float(), y.view(-1))
            assert abs(float(loss.detach()) - float(ref)) <= 1e-4 * float(ref)
        del logits
        opt.zero_grad(set_to_none=True)
        loss.backward()
        # the bench's step: clip at 1.0 inside the fused AdamW update
        opt.step(max_grad_norm=1.0)
        assert torch.isfinite(opt.grad_norm), "non-finite gradient norm"
        losses.append(float(loss.detach()))
    assert all(math.isfinite(v) for v in losses)
    assert math.log(V) - 0.2 < losses[0] < math.log(V) + 2.0, losses
    assert losses[-1] < losses[0] - 0.5 and abs(losses[-1] - math.log(V)) < 0.2, losses


def test_mixer_gradient_fanout_matches_autograd_sums(gpu):
    """With the HIP scan the mixer collects h's gradient (projection GEMM,
    two gate convolutions, scan, readout) in one buffer: the scan writes its
    du, which also carries the readout's D h term (du_skip = D / s), and the
    convolutions and the GEMM add into it. Against the same mixer whose
    scan is reached through another backend name (autograd then sums the
    five gradients), under bf16 autocast at the C5 layer's width: every
    gradient agrees to bf16 rounding."""
    import copy
    from naju_amd import scan as scan_mod
    from naju_amd.mixer import NajuMixer
    scan_mod._BACKEND_CACHE["hip_plain"] = lambda *a: scan_mod.naju_scan_hip(*a)
    try:
        torch.manual_seed(3)
        ma = NajuMixer(768, d_state=64, scan_backend="hip").to(gpu)
        mb = copy.deepcopy(ma)
        mb.scan_backend = "hip_plain"
        u = torch.randn(2, 512, 768, device=gpu)
        gy = torch.randn(2, 512, 768, device=gpu)
        outs = []
        for m in (ma, mb):
            ui = u.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = m(ui)
            y.float().backward(gy)
            outs.append((y.detach().float(), ui.grad))
        assert torch.equal(outs[0][0], outs[1][0])
        assert _rel(outs[0][1], outs[1][1]) < 1e-2
        for (n, pa), pb in zip(ma.named_parameters(), mb.parameters()):
            assert _rel(pa.grad, pb.grad) < 1e-2, n
    finally:
        scan_mod._BACKEND_CACHE.pop("hip_plain", None)


def test_lm_weight_copies_match_per_layer_casts(gpu, monkeypatch):
    """NajuLM's forward under bf16 autocast writes every projection's and
    the head's 16-bit weight with one naju_cast_multi launch
    (naju_amd.wcast), which the GEMMs take in place of their own casts and
    concatenations: logits, loss and every gradient are bitwise those of the
    same model without it, and every lookup hits."""
    import copy
    from naju_amd import wcast
    from naju_amd.xent import cross_entropy
    torch.manual_seed(11)
    V = 97
    ma = NajuLM(V, d_model=64, n_layers=2, dropout=0.0, d_state=16, scan_backend="hip").to(gpu)
    mb = copy.deepcopy(ma)
    monkeypatch.setattr(mb, "_cast_groups", lambda x: [])
    hits = []
    real = wcast.lookup

    def spy(weights, dtype):
        r = real(weights, dtype)
        hits.append(r is not None)
        return r

    monkeypatch.setattr(wcast, "lookup", spy)
    ids = torch.randint(0, V, (2, 65), device=gpu)
    outs = []
    for m in (ma, mb):
        hits.clear()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = m(ids[:, :-1])
            loss = cross_entropy(logits.reshape(-1, V), ids[:, 1:].reshape(-1))
        loss.backward()
        outs.append((logits.detach().clone(), loss.detach(), [p.grad for p in m.parameters()], list(hits)))
    assert outs[0][3] == [True] * (3 * 2 + 1) and not any(outs[1][3])
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    for (n, _), ga, gb in zip(ma.named_parameters(), outs[0][2], outs[1][2]):
        assert torch.equal(ga, gb), n


def test_mixer_gate_gradients_handed_over_in_place(gpu, monkeypatch):
    """With the HIP scan the mixer's gate logits' gradients go from the
    scan's backward straight into the projection gradient buffer (bf16,
    rounded once from float32, as autocast's backward rounds them) with
    their float32 sums as the biases' gradients (naju_amd.dwconv.GateGrads):
    the hand-off happens in every layer, and the gradients agree with the
    same mixer reached through another backend name (no hand-off, float32
    gate gradients into the convolutions) to bf16 rounding."""
    import copy
    from naju_amd import dwconv
    from naju_amd import scan as scan_mod
    from naju_amd.mixer import NajuMixer
    taken = []
    real = dwconv.GateGrads.take

    def spy(self, dy0, dy1):
        r = real(self, dy0, dy1)
        taken.append(r[0] is not None)
        return r

    monkeypatch.setattr(dwconv.GateGrads, "take", spy)
    scan_mod._BACKEND_CACHE["hip_plain2"] = lambda *a: scan_mod.naju_scan_hip(*a)
    try:
        torch.manual_seed(4)
        ma = NajuMixer(256, d_state=64, scan_backend="hip").to(gpu)
        mb = copy.deepcopy(ma)
        mb.scan_backend = "hip_plain2"
        u = torch.randn(2, 384, 256, device=gpu)
        gy = torch.randn(2, 384, 256, device=gpu)
        outs = []
        for m in (ma, mb):
            ui = u.clone().requires_grad_(True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                y = m(ui)
            y.float().backward(gy)
            outs.append((ui.grad, {n: p.grad for n, p in m.named_parameters()}))
        assert taken == [True], taken
        assert _rel(outs[0][0], outs[1][0]) < 1e-2
        for n, ga in outs[0][1].items():
            assert _rel(ga, outs[1][1][n]) < 2e-2, n
    finally:
        scan_mod._BACKEND_CACHE.pop("hip_plain2", None)
