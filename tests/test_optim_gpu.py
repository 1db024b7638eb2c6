"""naju_amd.optim.AdamW against the reference loop's clip_grad_norm_ +
torch.optim.AdamW (evals/lm/train.py:79-80, 165-166; naju/optim.py:30-52):
same parameters, moments and gradient norm after several steps, over tensors
of many sizes (whole and partial chunks), an unaligned one, two param groups,
a learning-rate change between steps and a parameter without a gradient."""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(3 * 8192,), (100, 333), (8192 + 5,), (7,), (512, 768), (1,)]


def _params(dev, seed):
    """Parameters of SHAPES plus one whose data starts 4 bytes into its
    storage (a view: the kernels' element path)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    ps = [torch.nn.Parameter(torch.randn(*s, generator=g, device=dev)) for s in SHAPES]
    base = torch.randn(4097, generator=g, device=dev)
    ps.append(torch.nn.Parameter(base[1:]))
    assert ps[-1].data_ptr() % 16 == 4
    return ps


def _grads(ps, dev, step, scale):
    g = torch.Generator(device=dev).manual_seed(1000 + step)
    return [torch.randn(p.shape, generator=g, device=dev) * scale for p in ps]


def _groups(ps, lr):
    return [{"params": ps[:4]}, {"params": ps[4:], "lr": lr * 3, "weight_decay": 0.02, "eps": 1e-6}]


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def _same_update(after, before, after_ref, before_ref):
    """The steps after - before and after_ref - before_ref agree to the
    float32 rounding of the parameters themselves (two ulps of |before| +
    |after|) plus 1e-5 of the largest step: far below what a wrong bias
    correction, eps placement, decay or clip coefficient would change."""
    d, d_ref = after - before, after_ref - before_ref
    tol = 2 * torch.finfo(torch.float32).eps * (before_ref.abs() + after_ref.abs()) + 1e-5 * d_ref.abs().max()
    return bool(((d - d_ref).abs() <= tol).all())


@pytest.mark.parametrize("max_norm", [None, 1e9, 0.5])
def test_adamw_matches_clip_and_torch_adamw(gpu, max_norm):
    from naju_amd.optim import AdamW
    ref, mine = _params(gpu, 1), _params(gpu, 1)
    opt_r = torch.optim.AdamW(_groups(ref, 1e-2), lr=1e-2, weight_decay=0.1)
    opt_m = AdamW(_groups(mine, 1e-2), lr=1e-2, weight_decay=0.1)
    for step in range(4):
        gs = _grads(ref, gpu, step, 0.3)
        for i, (pr, pm, g) in enumerate(zip(ref, mine, gs)):
            # parameter 2 has no gradient on step 1 (torch skips it: no state change)
            has = not (i == 2 and step == 1)
            pr.grad = g.clone() if has else None
            pm.grad = g.clone() if has else None
        if step == 2:
            for o in (opt_r, opt_m):
                for grp in o.param_groups:
                    grp["lr"] *= 0.5
        before = [p.detach().clone() for p in mine]
        before_ref = [p.detach().clone() for p in ref]
        if max_norm is not None:
            n_ref = torch.nn.utils.clip_grad_norm_(ref, max_norm)
        opt_r.step()
        opt_m.step(max_grad_norm=max_norm)
        torch.cuda.synchronize()
        if max_norm is not None:
            assert _rel(opt_m.grad_norm, n_ref) < 1e-6, step
        for i, (pr, pm, b, br) in enumerate(zip(ref, mine, before, before_ref)):
            assert _same_update(pm.detach(), b, pr.detach(), br), (step, i)
            for k in ("exp_avg", "exp_avg_sq"):
                if pr in opt_r.state:
                    assert _rel(opt_m.state[pm][k], opt_r.state[pr][k]) < 2e-6, (step, i, k)
            if pr in opt_r.state:
                assert float(opt_m.state[pm]["step"]) == float(opt_r.state[pr]["step"])


def test_adamw_deterministic_and_state_dict_interchange(gpu):
    from naju_amd.optim import AdamW
    runs = []
    for _ in range(2):
        ps = _params(gpu, 2)
        opt = AdamW(ps, lr=1e-3)
        for step in range(3):
            for p, g in zip(ps, _grads(ps, gpu, step, 1.0)):
                p.grad = g
            opt.step(max_grad_norm=1.0)
        torch.cuda.synchronize()
        runs.append(([p.detach().clone() for p in ps], opt.grad_norm.clone(), opt.state_dict()))
    for a, b in zip(runs[0][0], runs[1][0]):
        assert torch.equal(a, b)
    assert torch.equal(runs[0][1], runs[1][1])
    # torch.optim.AdamW takes the state dict and continues as this class does
    ps_t = [torch.nn.Parameter(p.clone()) for p in runs[0][0]]
    ps_m = [torch.nn.Parameter(p.clone()) for p in runs[0][0]]
    # (each takes its own copy: load_state_dict keeps the tensors it is given)
    opt_t = torch.optim.AdamW(ps_t, lr=1e-3)
    opt_t.load_state_dict(copy.deepcopy(runs[0][2]))
    opt_m = AdamW(ps_m, lr=1e-3)
    opt_m.load_state_dict(copy.deepcopy(runs[0][2]))
    gs = _grads(ps_t, gpu, 9, 1.0)
    for pt, pm, g in zip(ps_t, ps_m, gs):
        pt.grad, pm.grad = g.clone(), g.clone()
    opt_t.step()
    opt_m.step()
    torch.cuda.synchronize()
    for pt, pm, b in zip(ps_t, ps_m, runs[0][0]):
        assert _same_update(pm.detach(), b, pt.detach(), b)


def test_adamw_rejects_what_it_does_not_serve(gpu):
    from naju_amd.optim import AdamW
    p = torch.nn.Parameter(torch.zeros(10, device=gpu, dtype=torch.bfloat16))
    p.grad = torch.zeros_like(p)
    with pytest.raises(ValueError, match="float32"):
        AdamW([p]).step()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_weight_copies_are_torch_casts_bitwise(gpu, dtype):
    """naju_cast_multi through naju_amd.wcast: every group's 16-bit matrix is
    torch's .to(dtype) of its weights concatenated, bitwise (NaN as NaN),
    over whole and partial chunks, an unaligned weight (element path),
    special values (infinities, overflow, subnormals, ties of the rounding)
    and zero padding rows; a second write after the weights change reuses the
    table and shows the new values."""
    from naju_amd import wcast
    g = torch.Generator(device=gpu).manual_seed(3)
    w1 = torch.randn(300, 1536, generator=g, device=gpu) * 0.02
    bits = torch.randint(0, 1 << 31, (17, 1536), generator=g, device=gpu, dtype=torch.int64)
    # exponents in a normal range, the low 16 bits an exact bf16 tie
    bits = (bits & 0x807FFFFF) | (torch.randint(100, 150, (17, 1536), generator=g, device=gpu) << 23)
    w2 = (bits.to(torch.int32) & ~0xFFFF | 0x8000).view(torch.float32).clone()
    w2[0, :6] = torch.tensor([float("inf"), -float("inf"), 1e-40, -3.0e38, 65520.0, float("nan")], device=gpu)
    base = torch.randn(5 * 1536 + 1, generator=g, device=gpu)
    w3 = base[1:].view(5, 1536)
    assert w3.data_ptr() % 16 == 4
    w4 = torch.randn(1, 1536, generator=g, device=gpu)
    groups = [((w1, w2), 0), ((w3,), 0), ((w4,), 128)]
    copies = wcast.WeightCopies()
    for rep in range(2):
        mats = copies.write(groups, dtype)
        torch.cuda.synchronize()
        want = [torch.cat([w1, w2]).to(dtype), w3.to(dtype),
                torch.cat([w4.to(dtype), torch.zeros(127, 1536, dtype=dtype, device=gpu)])]
        for (ws, _), ref in zip(groups, want):
            got = mats[tuple(id(w) for w in ws)]
            assert got.shape == ref.shape and got.dtype == dtype
            nan = torch.isnan(ref)
            assert torch.equal(torch.isnan(got), nan)
            assert torch.equal(got.view(torch.int16)[~nan], ref.view(torch.int16)[~nan]), rep
        w1.mul_(-1.5)
        w3.add_(0.25)
