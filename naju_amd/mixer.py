"""Naju mixer, residual block and causal LM on top of the MI355X scan.

A restatement of the reference's model code (naju/mixer.py:51-144,
naju/lm.py:13-33, naju/optim.py:30-52) over this package's scan dispatch, so
the mixer and the LM training step (benchmark configuration c5) run with the HIP
scan where the reference package is absent. Module and parameter names, shapes
and initialisation follow the reference, so state dicts load in either
direction with ``strict=True``.

One layer, with u the residual stream and h the content branch:

    [x, z]   = in_proj(u)                          d_model -> 2 d_inner
    h        = SiLU(causal depthwise conv_k(x) + conv bias)
    [B, C]   = x_proj(h)                           d_inner -> 2 N
    f_logit  = f_proj(h) [/ sqrt(d_inner)] + causal dwconv_k(h) + f_bias   (f_bias init +5)
    i_logit  = i_proj(h) [/ sqrt(d_inner)] + causal dwconv_k(h) + i_bias   (i_bias init -2)
    cx       = scan(h, f_logit, i_logit, B, C, D=0) / sqrt(N)
    out      = out_proj((cx + D * h) * SiLU(z))    (D init 0.01)

The bracketed 1/sqrt(d_inner) applies with ``gate_reparam``, whose weights
start scaled up by sqrt(d_inner) (same forward at init) and whose optimizer
half is ``build_optimizer``. ``gate_rank`` factors the gate projections as
two linear maps. The scan runs through ``naju_amd.scan.naju_scan`` with the
mixer's ``scan_backend`` (default: ``NAJU_SCAN_BACKEND``, else the HIP
kernels).
"""
import math

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from naju_amd import embed, gradsink, wcast
from naju_amd.dwconv import dwconv, dwconv_pair, pair_supported
from naju_amd.linear import HEAD_ALIGN, compute_dtype, linear, linear_cat, lm_head
from naju_amd.optim import AdamW as NajuAdamW
from naju_amd.readout import readout
from naju_amd.rmsnorm import rms_norm
from naju_amd.rmsnorm import rms_norm_fork
from naju_amd.rmsnorm import supported as rmsnorm_supported
from naju_amd.residual import draw_seeds, residual_dropout
from naju_amd.residual import supported as residual_supported
from naju_amd import scan as _scan
from naju_amd.scan import naju_scan, naju_scan_hip


class RMSNorm(nn.Module):
    """weight * x / sqrt(mean(x^2) + eps) over the last axis.

    ``out_dtype`` (default: the promoted dtype of weight and x, as the
    reference's expression gives) lets a caller whose consumer is an
    autocast GEMM take y in the autocast dtype directly: the same values the
    GEMM's own cast would produce, without the float32 copy. CUDA inputs the
    fused kernels serve (naju_amd.rmsnorm.supported) run on them; others use
    the reference's expression."""

    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x, out_dtype=None):
        if out_dtype is None:
            out_dtype = torch.promote_types(self.weight.dtype, x.dtype)
        if rmsnorm_supported(x):
            return rms_norm(x, self.weight, self.eps, out_dtype)
        y = self.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)
        return y.to(out_dtype)


def _out_dtype(x):
    dev = x.device.type
    return torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev) else x.dtype


def _hip_scan(backend):
    """naju_scan_hip when `backend` resolves to it, else None."""
    fn = _scan._get(_scan.resolve_backend(backend))
    return fn if fn is naju_scan_hip else None


def _linear(x, weight):
    """F.linear(x, weight) (no bias); on CUDA in 16-bit compute with the
    split-K float32 weight gradient of naju_amd.linear."""
    if compute_dtype(x) is not None:
        return linear(x, weight)
    return F.linear(x, weight)


def _linear_cat(x, weights):
    """F.linear(x, torch.cat(weights, 0)); on CUDA in 16-bit compute one GEMM
    whose 16-bit weight may come from naju_amd.wcast, with the split-K
    float32 weight gradient."""
    if compute_dtype(x) is not None:
        return linear_cat(x, weights)
    return F.linear(x, torch.cat(weights, 0))


def _causal_dwconv(x, conv):
    """Depthwise causal convolution of x [B, T, C] along T with the weights of
    `conv` (an nn.Conv1d with groups = C): output t sees inputs t-k+1 .. t,

        y[:, t] = bias + sum_j w[:, j] * x[:, t - (k-1) + j].

    The formulation for CPU tensors: k shifted multiply-adds in the [B, T, C]
    layout, in float32. Under autocast the result takes the autocast dtype, as
    the library convolution would. CUDA tensors take the fused HIP kernels of
    naju_amd.dwconv instead (NajuMixer._content and _gate_logit)."""
    w = conv.weight[:, 0, :].float()  # [C, k]
    k = w.shape[1]
    T = x.shape[1]
    xp = F.pad(x, (0, 0, k - 1, 0))
    y = xp[:, k - 1:].float() * w[:, k - 1]
    for j in range(k - 1):
        y = torch.addcmul(y, xp[:, j:j + T].float(), w[:, j])
    if conv.bias is not None:
        y = y + conv.bias.float()
    return y.to(_out_dtype(x))


class NajuMixer(nn.Module):
    def __init__(self, d_model, d_state=64, d_conv=4, expand=2, gate_conv_kernel=4,
                 forget_bias_init=5.0, input_bias_init=-2.0, d_init=0.01,
                 gate_rank=None, gate_reparam=False, scan_backend=None):
        super().__init__()
        if gate_reparam and gate_rank:
            raise ValueError("gate_reparam is incompatible with gate_rank "
                             "(the rescale targets the full-rank projections)")
        di = expand * d_model
        self.d_model, self.d_state, self.d_inner = d_model, d_state, di
        self.gate_rank = gate_rank
        self.gate_reparam = bool(gate_reparam)
        self.scan_backend = scan_backend
        self._cx_scale = 1.0 / math.sqrt(d_state)

        self.in_proj = nn.Linear(d_model, 2 * di, bias=False)
        # the convolutions pad inside _causal_dwconv; the modules hold weights
        self.conv1d = nn.Conv1d(di, di, kernel_size=d_conv, groups=di, bias=True)
        self.x_proj = nn.Linear(di, 2 * d_state, bias=False)
        self.out_proj = nn.Linear(di, d_model, bias=False)
        self.D = nn.Parameter(torch.full((di,), float(d_init)))
        self.register_buffer("D_zero", torch.zeros(di), persistent=False)

        self.f_proj = self._gate_proj()
        self.f_conv = nn.Conv1d(di, di, kernel_size=gate_conv_kernel, groups=di, bias=False)
        self.f_bias = nn.Parameter(torch.full((di,), float(forget_bias_init)))
        self.i_proj = self._gate_proj()
        self.i_conv = nn.Conv1d(di, di, kernel_size=gate_conv_kernel, groups=di, bias=False)
        self.i_bias = nn.Parameter(torch.full((di,), float(input_bias_init)))
        if self.gate_reparam:
            with torch.no_grad():
                self.f_proj.weight.mul_(math.sqrt(di))
                self.i_proj.weight.mul_(math.sqrt(di))

    def _gate_proj(self):
        di = self.d_inner
        if self.gate_rank:
            return nn.Sequential(nn.Linear(di, self.gate_rank, bias=False),
                                 nn.Linear(self.gate_rank, di, bias=False))
        return nn.Linear(di, di, bias=False)

    def _gate_logit(self, h, proj, conv, bias, p=None):
        if p is None:
            p = proj(h)
        if self.gate_reparam:
            p = p / math.sqrt(self.d_inner)
        if h.is_cuda:
            # one kernel: projection + conv + bias, in the dtype the sum
            # promotes to (float32 under autocast: the bias is float32)
            return dwconv(h, conv.weight, bias, add=p,
                          out_dtype=torch.promote_types(_out_dtype(h), bias.dtype))
        return p + _causal_dwconv(h, conv) + bias

    def _content(self, x):
        if x.is_cuda:
            return dwconv(x, self.conv1d.weight, self.conv1d.bias, silu=True, out_dtype=_out_dtype(x))
        return F.silu(_causal_dwconv(x, self.conv1d))

    def cast_groups(self):
        """The weight groups this mixer's GEMMs look up in naju_amd.wcast
        (on CUDA in 16-bit compute): in_proj, the fused f / i / x projection
        (without gate_rank) and out_proj."""
        g = [((self.in_proj.weight,), 0)]
        if not self.gate_rank:
            g.append(((self.f_proj.weight, self.i_proj.weight, self.x_proj.weight), 0))
        g.append(((self.out_proj.weight,), 0))
        return g

    def forward(self, u):
        xz = _linear(u, self.in_proj.weight)
        if xz.is_cuda:
            # x feeds the content convolution and z the readout; both write
            # their gradients straight into one buffer for in_proj
            x, z = gradsink.split(xz, [self.d_inner, self.d_inner])
        else:
            x, z = xz.chunk(2, dim=-1)
        h = self._content(x)
        # h feeds five consumers (projection GEMM, two gate convolutions,
        # scan, readout). With the HIP scan, their gradients collect in one
        # buffer instead of four additions: the scan's du comes first and
        # also carries the readout's D h term (du_skip = D / s), and the
        # convolutions and the GEMM add into it in place
        fold = (h.is_cuda and not self.gate_rank and torch.is_grad_enabled() and h.requires_grad
                and _hip_scan(self.scan_backend) is not None)
        # the two gate convolutions as one pass over h each way (their logits
        # take the projection slices in place; not with gate_reparam, whose
        # rescaled projection is a new tensor)
        pair = (h.is_cuda and not self.gate_rank and not self.gate_reparam and self.d_inner % 8 == 0
                and self.f_conv.weight.shape[-1] == 4 and self.i_conv.weight.shape[-1] == 4)
        if fold and pair:
            h_g, h_f, h_s, h_r = gradsink.fanout(h, 4)
            h_i = h_f
        elif fold:
            h_g, h_f, h_i, h_s, h_r = gradsink.fanout(h, 5)
        else:
            h_g = h_f = h_i = h_s = h_r = h
        gate_grads = None
        if h.is_cuda and not self.gate_rank:
            # f_proj, i_proj and x_proj in one GEMM over h (the same weights:
            # each output column is the same product), so h's gradient from
            # the three comes back as one GEMM instead of three plus two adds;
            # the convolutions read their slices in place
            di, N = self.d_inner, self.d_state
            w = (self.f_proj.weight, self.i_proj.weight, self.x_proj.weight)
            p_f, p_i, Bm, Cm = gradsink.split(_linear_cat(h_g, w), [di, di, N, N])
            if pair and pair_supported(h_f, self.f_conv.weight, p_f, self.i_conv.weight, p_i):
                # with the HIP scan, the logits' gradients come back through
                # gate_grads (written in place by the scan's backward)
                f_logit, i_logit, *gg = dwconv_pair(
                    h_f, self.f_conv.weight, self.f_bias, p_f, self.i_conv.weight, self.i_bias, p_i,
                    out_dtype=torch.promote_types(_out_dtype(h), self.f_bias.dtype), gate_grads=fold)
                gate_grads = gg[0] if gg else None
            else:
                f_logit = self._gate_logit(h_f, None, self.f_conv, self.f_bias, p=p_f)
                i_logit = self._gate_logit(h_i, None, self.i_conv, self.i_bias, p=p_i)
        else:
            Bm, Cm = self.x_proj(h).split(self.d_state, dim=-1)
            f_logit = self._gate_logit(h, self.f_proj, self.f_conv, self.f_bias)
            i_logit = self._gate_logit(h, self.i_proj, self.i_conv, self.i_bias)
        # the scan reads out the state only; the D skip is applied here
        if fold:
            # D / s: formed for all layers in one launch by NajuLM.forward
            # when it runs this mixer, else here
            du_skip = self.__dict__.pop("_du_skip", None)
            if du_skip is None:
                du_skip = self.D.detach() * (1.0 / self._cx_scale)
            cx = naju_scan_hip(h_s, f_logit, i_logit, Bm, Cm, self.D_zero, du_skip=du_skip, gate_grads=gate_grads)
        else:
            cx = naju_scan(h, f_logit, i_logit, Bm, Cm, self.D_zero, backend=self.scan_backend)
        if h.is_cuda:
            # one kernel each way; the output takes the autocast dtype the
            # out_proj GEMM consumes
            y = readout(cx, h_r, z, self.D, self._cx_scale, out_dtype=_out_dtype(h), dh_elsewhere=fold)
        else:
            y = (cx * self._cx_scale + self.D * h) * F.silu(z)
        return _linear(y, self.out_proj.weight)


class NajuBlock(nn.Module):
    """Pre-norm residual block u + Dropout(Mixer(RMSNorm(u)))."""

    def __init__(self, d_model, dropout=0.1, use_ckpt=False, **mixer_kw):
        super().__init__()
        self.norm = RMSNorm(d_model)
        self.mixer = NajuMixer(d_model, **mixer_kw)
        self.drop = nn.Dropout(dropout)
        self.use_ckpt = use_ckpt

    def _branch(self, u):
        # the norm's output feeds in_proj only: take it in that GEMM's dtype
        return self.drop(self.mixer(self.norm(u, out_dtype=_out_dtype(u))))

    def _fused(self, u, seed=None):
        # the norm and the residual read u; their gradients meet in the
        # norm's backward pass, and the residual add and the dropout are one
        # pass each way (naju_amd.residual)
        u_res, h = rms_norm_fork(u, self.norm.weight, self.norm.eps, out_dtype=_out_dtype(u))
        mix = self.mixer(h)
        if not residual_supported(u_res, mix):
            return u_res + self.drop(mix)
        return residual_dropout(u_res, mix, self.drop.p if self.training else 0.0, seed=seed)

    def fused_path(self, u):
        """Whether forward(u) runs the fused norm / residual / dropout kernels
        (CUDA float32 residual streams they serve)."""
        return u.is_cuda and u.dtype == torch.float32 and rmsnorm_supported(u)

    def forward(self, u, seed=None):
        """seed: the fused path's dropout seed (a one-element int64 CUDA
        tensor; NajuLM draws all its blocks' seeds at once), else drawn here."""
        fused = self.fused_path(u)
        if self.use_ckpt and torch.is_grad_enabled():
            if fused:
                return checkpoint(self._fused, u, seed, use_reentrant=False)
            return u + checkpoint(self._branch, u, use_reentrant=False)
        if fused:
            return self._fused(u, seed)
        return u + self._branch(u)


class NajuLM(nn.Module):
    """Embedding, n_layers NajuBlocks, final RMSNorm, LM head (tied to the
    embedding by default); embedding and head start N(0, 0.02)."""

    def __init__(self, vocab_size, d_model=256, n_layers=6, dropout=0.1,
                 tie_weights=True, use_ckpt=False, **mixer_kw):
        super().__init__()
        self.embed = nn.Embedding(vocab_size, d_model)
        self.blocks = nn.ModuleList(
            NajuBlock(d_model, dropout=dropout, use_ckpt=use_ckpt, **mixer_kw) for _ in range(n_layers))
        self.norm = RMSNorm(d_model)
        self.head = nn.Linear(d_model, vocab_size, bias=False)
        nn.init.normal_(self.embed.weight, std=0.02)
        nn.init.normal_(self.head.weight, std=0.02)
        if tie_weights:
            self.head.weight = self.embed.weight

    def _cast_groups(self, x):
        """Every weight the forward's GEMMs take in 16-bit compute on CUDA
        (the blocks' projections, the head padded to HEAD_ALIGN rows), for one
        naju_cast_multi launch per forward; none otherwise."""
        if not (x.is_cuda and torch.is_autocast_enabled("cuda")):
            return []
        groups = [g for blk in self.blocks for g in blk.mixer.cast_groups()]
        return groups + [((self.head.weight,), HEAD_ALIGN)]

    def forward(self, ids):
        # tied weights under 16-bit autocast on the GPU: the head's gradient
        # goes to the embedding's backward, which adds its rows in place
        w = self.embed.weight
        tied = None
        if (self.head.weight is w and torch.is_grad_enabled() and w.requires_grad
                and torch.is_autocast_enabled("cuda") and embed.supported(ids, w)):
            tied = embed.TiedGrad(w)
        x = embed.embedding(ids, w, tied) if tied is not None else self.embed(ids)
        groups = self._cast_groups(x)
        if groups and getattr(self, "_wcopies", None) is None:
            self._wcopies = wcast.WeightCopies()
        with wcast.active(getattr(self, "_wcopies", None), groups,
                          torch.get_autocast_dtype("cuda") if groups else None):
            # every mixer's D / s (its scan's du_skip) in one multi-tensor
            # launch; a mixer takes its own once during this forward, and what
            # is not taken is dropped at its end (a recompute under
            # activation checkpointing forms its own)
            mixers = [blk.mixer for blk in self.blocks]
            if x.is_cuda and mixers and all(m.D.is_cuda and m._cx_scale == mixers[0]._cx_scale for m in mixers):
                for m, v in zip(mixers, torch._foreach_mul([m.D.detach() for m in mixers],
                                                           1.0 / mixers[0]._cx_scale)):
                    m.__dict__["_du_skip"] = v
            try:
                # the blocks' dropout seeds in one draw (one kernel, not one each)
                seeds = None
                if (self.training and self.blocks and self.blocks[0].drop.p > 0.0
                        and self.blocks[0].fused_path(x)):
                    seeds = draw_seeds(len(self.blocks), x.device)
                for i, blk in enumerate(self.blocks):
                    x = blk(x) if seeds is None else blk(x, seeds[i:i + 1])
            finally:
                for m in mixers:
                    m.__dict__.pop("_du_skip", None)
            h = self.norm(x, out_dtype=_out_dtype(x))
            if compute_dtype(h) is not None:
                # padded vocabulary rows: aligned GEMMs (logits: a strided view)
                return lm_head(h, self.head.weight, tied)
            return self.head(h)


def build_optimizer(model, lr, weight_decay=0.1, fused=None):
    """AdamW; with gate_reparam mixers, their f_proj / i_proj weights get
    lr * sqrt(d_inner), weight_decay / sqrt(d_inner) and eps 1e-8 / sqrt(d_inner)
    (reference naju/optim.py:30-52).

    ``fused`` (default: True when every parameter is a CUDA tensor) selects a
    single-pass update: naju_amd.optim.AdamW (the HIP multi-tensor kernels,
    whose ``step(max_grad_norm=...)`` also clips) when every parameter is
    float32, else torch's fused AdamW. The same update rule as the
    reference's torch.optim.AdamW either way."""
    if fused is None:
        fused = all(p.is_cuda for p in model.parameters())
    opt_cls, kw = torch.optim.AdamW, {"fused": fused}
    if fused and all(p.dtype == torch.float32 for p in model.parameters()):
        opt_cls, kw = NajuAdamW, {}
    mixers = [m for m in model.modules() if isinstance(m, NajuMixer) and m.gate_reparam]
    if not mixers:
        return opt_cls(model.parameters(), lr=lr, weight_decay=weight_decay, **kw)
    widths = {m.d_inner for m in mixers}
    if len(widths) != 1:
        raise ValueError(f"mixed d_inner across gate_reparam mixers: {widths}")
    mult = math.sqrt(widths.pop())
    gate = {id(p) for m in mixers for p in (m.f_proj.weight, m.i_proj.weight)}
    rest = [p for p in model.parameters() if id(p) not in gate]
    gate_params = [p for p in model.parameters() if id(p) in gate]
    return opt_cls(
        [{"params": rest},
         {"params": gate_params, "lr": lr * mult, "weight_decay": weight_decay / mult, "eps": 1e-8 / mult}],
        lr=lr, weight_decay=weight_decay, **kw)
