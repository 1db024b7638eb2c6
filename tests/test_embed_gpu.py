"""GPU tests: the embedding's backward added in place into the tied head's
gradient (naju_embedding_bwd_add, naju_amd/embed.py) against float32 sums in
the same order on the CPU and against autograd's two gradients of the tied
weight (naju/lm.py:13-33 ties the head to the embedding)."""
import copy

import pytest
import torch

from naju_amd import _lib, embed
from naju_amd.linear import lm_head
from naju_amd.mixer import NajuLM
from naju_amd.xent import cross_entropy

pytestmark = pytest.mark.gpu


def _sorted_sums(ids, dy, dw0):
    """dw0[id] + dy rows of id in the order of a stable sort, one float32 add
    at a time (rank k of every run added in pass k: no id twice per pass)."""
    dw = dw0.clone()
    srt, order = torch.sort(ids, stable=True)
    start = torch.ones_like(srt, dtype=torch.bool)
    start[1:] = srt[1:] != srt[:-1]
    run_start = torch.cummax(torch.where(start, torch.arange(len(srt)), 0), 0).values
    rank = torch.arange(len(srt)) - run_start
    ok = (srt >= 0) & (srt < dw.shape[0])
    for k in range(int(rank.max()) + 1 if len(srt) else 0):
        sel = (rank == k) & ok
        dw[srt[sel]] += dy[order[sel]]
    return dw


@pytest.mark.parametrize("n,V,d,hot", [(1, 5, 4, 0), (300, 50, 768, 0), (1000, 7, 36, 0), (4096, 1000, 64, 0.5),
                                       (513, 97, 13, 0)])
def test_embedding_bwd_add_is_the_sorted_order_sum(gpu, n, V, d, hot):
    """Bitwise the CPU's float32 sums in stable-sort order added to the
    existing rows; repeated ids (a hot id taking half the positions), ids
    outside [0, V) skipped, d not a multiple of 4."""
    g = torch.Generator().manual_seed(n + V + d)
    ids = torch.randint(0, V, (n,), generator=g)
    if hot:
        ids[torch.rand(n, generator=g) < hot] = 3
    if n > 100:
        ids[:3] = torch.tensor([-1, V, V + 5])
    dy = torch.randn(n, d, generator=g)
    dw0 = torch.randn(V, d, generator=g)
    want = _sorted_sums(ids, dy, dw0)
    srt, order = torch.sort(ids.to(gpu), stable=True)
    dw = dw0.to(gpu)
    dyg = dy.to(gpu)
    assert _lib.lib().naju_embedding_bwd_add(srt.data_ptr(), order.data_ptr(), dyg.data_ptr(), n, d, dw.data_ptr(), V,
                                             torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(dw.cpu(), want)


def test_embedding_bwd_add_rejects_bad_sizes(gpu):
    L = _lib.lib()
    x = torch.zeros(4, device=gpu)
    assert L.naju_embedding_bwd_add(x.data_ptr(), x.data_ptr(), x.data_ptr(), -1, 1, x.data_ptr(), 1, None) != 0
    assert L.naju_embedding_bwd_add(None, x.data_ptr(), x.data_ptr(), 1, 1, x.data_ptr(), 1, None) != 0
    assert L.naju_embedding_bwd_add(None, None, None, 0, 1, None, 1, None) == 0


def _step(m, ids, V, n_backward=1):
    for _ in range(n_backward):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            logits = m(ids[:, :-1])
            loss = cross_entropy(logits.reshape(-1, V), ids[:, 1:].reshape(-1))
        loss.backward()
    return {n: p.grad for n, p in m.named_parameters()}


@pytest.mark.parametrize("n_backward", [1, 2])
def test_lm_tied_gradient_matches_autograd_sum(gpu, monkeypatch, n_backward):
    """NajuLM's tied weight: the embedding rows added into the head's dW in
    place equal autograd's sum of the two gradients (torch's embedding
    backward) to float32 rounding, and every other gradient is bitwise the
    same; with two backward passes the gradients accumulate."""
    torch.manual_seed(5)
    V = 97
    ma = NajuLM(V, d_model=64, n_layers=2, dropout=0.0, d_state=16, scan_backend="hip").to(gpu)
    mb = copy.deepcopy(ma)
    ids = torch.randint(0, V, (2, 129), device=gpu)
    ga = _step(ma, ids, V, n_backward)
    monkeypatch.setattr(embed, "supported", lambda ids, w: False)
    gb = _step(mb, ids, V, n_backward)
    assert ma.head.weight is ma.embed.weight
    for n in ga:
        if n == "embed.weight":
            torch.testing.assert_close(ga[n], gb[n], rtol=1e-6, atol=1e-7)
        else:
            assert torch.equal(ga[n], gb[n]), n


def test_head_gradient_without_embedding_backward_reaches_grad(gpu):
    """A backward pass that reaches the head but not the embedding (the
    loss's graph starts at a leaf h): the head's dW handed to the TiedGrad is
    added to the weight's .grad when the pass ends, equal to the plain head's
    gradient."""
    torch.manual_seed(6)
    V, d = 300, 64
    w = torch.nn.Parameter(torch.randn(V, d, device=gpu) * 0.02)
    h = torch.randn(2, 33, d, device=gpu, requires_grad=True)
    grads = []
    for tied in (embed.TiedGrad(w), None):
        w.grad = None
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = lm_head(h, w, tied)
        (y.float().square().mean()).backward()
        grads.append(w.grad.clone())
    assert torch.equal(grads[0], grads[1])
