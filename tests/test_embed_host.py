"""CPU tests of the tied-gradient hand-off's host logic (naju_amd/embed.py):
a head gradient that no embedding backward takes reaches the weight's
.grad when the backward pass ends, once, and accumulates over passes; one
that is taken is not added again."""
import torch

from naju_amd import embed


class _Head(torch.autograd.Function):
    """y = x @ w.T whose backward hands dW to the TiedGrad, like the padded
    LM head's."""

    @staticmethod
    def forward(ctx, x, w, tied):
        ctx.save_for_backward(x, w)
        ctx.tied = tied
        return x @ w.t()

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        ctx.tied.put(dy.t() @ x)
        return dy @ w, None, None


class _Take(torch.autograd.Function):
    """An embedding stand-in: its backward takes the handed-over dW and
    returns it (plus nothing of its own) as the weight's gradient."""

    @staticmethod
    def forward(ctx, w, tied):
        ctx.tied = tied
        return w.sum(1, keepdim=True).t() * 0

    @staticmethod
    def backward(ctx, dy):
        dw = ctx.tied.take()
        return dw, None


def test_untaken_head_gradient_reaches_grad_and_accumulates():
    torch.manual_seed(0)
    w = torch.nn.Parameter(torch.randn(5, 3))
    x = torch.randn(4, 3)
    want = None
    for _ in range(2):
        tied = embed.TiedGrad(w)
        y = _Head.apply(x, w, tied)
        dy = torch.randn_like(y)
        y.backward(dy)
        want = dy.t() @ x if want is None else want + dy.t() @ x
        assert tied.take() is None
        torch.testing.assert_close(w.grad, want)


def test_taken_head_gradient_is_not_added_twice():
    torch.manual_seed(1)
    w = torch.nn.Parameter(torch.randn(5, 3))
    tied = embed.TiedGrad(w)
    # the head consumes the embedding stand-in's output, so the stand-in's
    # backward runs after the head's and takes its dW
    h = _Take.apply(w, tied).expand(4, 5)[:, :3].contiguous() + torch.randn(4, 3)
    y = _Head.apply(h, w, tied)
    dy = torch.randn_like(y)
    y.backward(dy)
    torch.testing.assert_close(w.grad, dy.t() @ h.detach())


def test_autograd_grad_pass_leaves_grad_alone():
    """torch.autograd.grad over the head's input: the untaken head gradient
    is dropped, as autograd drops the weight's gradient there."""
    torch.manual_seed(2)
    w = torch.nn.Parameter(torch.randn(5, 3))
    x = torch.randn(4, 3, requires_grad=True)
    y = _Head.apply(x, w, embed.TiedGrad(w))
    dy = torch.randn_like(y)
    (dx,) = torch.autograd.grad(y, [x], dy)
    torch.testing.assert_close(dx, dy @ w.detach())
    assert w.grad is None
