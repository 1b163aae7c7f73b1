"""Fused ``selective_log_softmax`` (per-token log-probabilities of chosen
tokens) backed by the gfx950 kernels.

The reference's RLHF experiment (experiment_rlhf_logsumexp/run_rlhf.py:28,
143-158) times ``trl.trainer.utils.selective_log_softmax`` (trl 1.0.0) with
its ``torch.logsumexp`` replaced by the LSE kernels.  For fp32 logits that
function gathers the target logits, calls ``torch.logsumexp`` once per
leading row, and subtracts: three passes and B launches.  Here the whole
thing is one pass over the logits (forward) and one read + one write
(backward).

``make_selective_log_softmax(ext, original=None, robust=True)`` returns
``selective_log_softmax(logits, index)`` with trl's signature: logits
[..., V], index [...] (integer), result [...] fp32.  CUDA fp32 logits take
the kernels, with autograd through the fused backward.  Other inputs go to
``original`` (for instance trl's own function), or, when it is None, to
trl's published algorithm in torch ops (``_trl_algorithm``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _trl_algorithm(logits: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """trl 1.0.0 selective_log_softmax: fp32/fp64 gather minus a per-row
    logsumexp loop; other dtypes per-row log_softmax then gather."""
    if logits.dtype in (torch.float32, torch.float64):
        selected = torch.gather(logits, dim=-1, index=index.unsqueeze(-1)).squeeze(-1)
        lse = torch.stack([torch.logsumexp(lg, dim=-1) for lg in logits])
        return selected - lse
    rows = []
    for row_logits, row_labels in zip(logits, index):
        row_logps = F.log_softmax(row_logits, dim=-1)
        rows.append(row_logps.gather(dim=-1, index=row_labels.unsqueeze(-1)).squeeze(-1))
    return torch.stack(rows)


def make_selective_log_softmax(ext, original=None, robust: bool = True):
    fwd = ext.selective_log_softmax_float
    bwd = ext.selective_log_softmax_float_backward
    fallback = original if original is not None else _trl_algorithm

    class _SelectiveLogSoftmax(torch.autograd.Function):
        @staticmethod
        def forward(ctx, logits, index):
            n = logits.shape[-1]
            rows = logits.reshape(-1, n).contiguous()
            idx = index.reshape(-1).to(torch.int64).contiguous()
            logp, lse = fwd(rows, idx, robust)
            ctx.save_for_backward(rows, idx, lse)
            ctx.in_shape = tuple(logits.shape)
            ctx.mark_non_differentiable(lse)
            return logp.reshape(index.shape)

        @staticmethod
        def backward(ctx, grad_out):
            rows, idx, lse = ctx.saved_tensors
            g = bwd(grad_out.reshape(-1).to(torch.float32).contiguous(), rows, idx, lse)
            return g.reshape(ctx.in_shape), None

    def selective_log_softmax(logits, index):
        ok = (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() >= 1
              and index.device == logits.device and not torch.is_floating_point(index)
              and tuple(index.shape) == tuple(logits.shape[:-1]) and logits.shape[-1] >= 1)
        if not ok:
            return fallback(logits, index)
        if torch.is_grad_enabled() and logits.requires_grad:
            return _SelectiveLogSoftmax.apply(logits, index)
        n = logits.shape[-1]
        logp, _ = fwd(logits.reshape(-1, n).contiguous(), index.reshape(-1).to(torch.int64).contiguous(), robust)
        return logp.reshape(index.shape)

    selective_log_softmax.fuselse_robust = robust
    return selective_log_softmax
