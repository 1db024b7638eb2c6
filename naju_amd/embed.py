"""The LM's embedding with its tied head's gradient collected in one buffer.

NajuLM ties the head to the embedding (naju/lm.py:13-33): the weight gets
two gradients, the head's dense dW and the embedding's scatter of the input
gradient's rows, which autograd adds (one more pass over the [V, d] float32
gradient after torch's sort-based embedding backward). Here the head's
backward hands its dW to a ``TiedGrad`` instead of returning it, and the
embedding's backward adds its rows into that buffer in place
(naju_embedding_bwd_add, include/naju_mixer.h: one workgroup per run of
equal ids in a stable sort, a fixed order) and returns it as the weight's
whole gradient. A head gradient that no embedding backward takes in the same
backward pass (a loss that does not reach the embedding) is added to the
weight's ``.grad`` when the pass ends, so no gradient is lost; a
torch.autograd.grad pass leaves ``.grad`` alone, as autograd does.

CUDA float32 weights and input gradients only; ``embedding`` raises for
anything else (NajuLM then keeps nn.Embedding).
"""
import torch
import torch.nn.functional as F

from naju_amd import _lib


class TiedGrad:
    """The head's weight gradient on its way to the tied embedding's
    backward (taken once), with the end-of-pass fallback."""

    def __init__(self, weight):
        self.weight = weight
        self._dw = None
        # the weight's gradient accumulator: the end-of-pass fallback adds
        # to .grad only in a pass that runs it (not torch.autograd.grad)
        self._acc = weight.view_as(weight).grad_fn.next_functions[0][0] if weight.requires_grad else None

    def put(self, dw):
        """From the head's backward (which then returns no gradient for the
        weight)."""
        self._dw = dw
        torch.autograd.Variable._execution_engine.queue_callback(self._flush)

    def take(self):
        dw, self._dw = self._dw, None
        return dw

    def _accumulates(self):
        probe = getattr(torch._C, "_will_engine_execute_node", None)
        if self._acc is None or probe is None:
            return self._acc is not None
        try:
            return bool(probe(self._acc))
        except RuntimeError:  # torch.autograd.grad with the weight among its inputs
            return False

    def _flush(self):
        dw = self.take()
        if dw is None or not self._accumulates():
            return
        w = self.weight
        with torch.no_grad():
            if w.grad is None:
                w.grad = dw
            else:
                w.grad.add_(dw)


def supported(ids, weight):
    return (weight.is_cuda and weight.dtype == torch.float32 and weight.dim() == 2 and weight.is_contiguous()
            and ids.device == weight.device and ids.dtype in (torch.int64, torch.int32))


class _Embedding(torch.autograd.Function):
    @staticmethod
    def forward(ctx, ids, weight, tied):
        ctx.save_for_backward(ids)
        ctx.shape, ctx.tied = weight.shape, tied
        return F.embedding(ids, weight)

    @staticmethod
    def backward(ctx, dy):
        (ids,) = ctx.saved_tensors
        V, d = ctx.shape
        dw = ctx.tied.take() if ctx.tied is not None else None
        if dw is None:
            dw = torch.zeros((V, d), dtype=torch.float32, device=dy.device)
        flat = ids.reshape(-1).to(torch.int64)
        srt, order = torch.sort(flat, stable=True)
        g = dy.reshape(-1, d)
        if g.dtype != torch.float32:
            g = g.float()
        g = g.contiguous()
        _lib.check_mixer(_lib.lib().naju_embedding_bwd_add(
            srt.data_ptr(), order.data_ptr(), g.data_ptr(), flat.numel(), d, dw.data_ptr(), V,
            torch.cuda.current_stream(dy.device).cuda_stream))
        return None, dw, None


def embedding(ids, weight, tied=None):
    """F.embedding(ids, weight) with the backward above; tied: the TiedGrad
    whose head gradient the backward adds its rows into."""
    if not supported(ids, weight):
        raise ValueError("naju_amd.embed.embedding serves contiguous float32 CUDA weights and int64 / int32 ids")
    return _Embedding.apply(ids, weight, tied)
