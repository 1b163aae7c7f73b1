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


# Most leading slices taken one launch each instead of copying the logits.
_MAX_SLICES = 64


def _row_slices(x: torch.Tensor):
    """Contiguous [rows, V] views covering x's rows in order, without a copy:
    x itself when it is contiguous, or x[b] for each b of a 3-D x whose rows
    are contiguous within each leading index (trl takes the logits as
    logits[:, :-1, :], whose rows skip one row at every leading index).  None
    when neither holds."""
    n = x.shape[-1]
    if x.is_contiguous():
        return [x.reshape(-1, n)]
    if x.dim() == 3 and 1 <= x.size(0) <= _MAX_SLICES and x.stride(-1) == 1 and x.stride(1) == n:
        return [x[b] for b in range(x.size(0))]
    return None


def make_selective_log_softmax(ext, original=None, robust: bool = True):
    fwd = ext.selective_log_softmax_float
    bwd = ext.selective_log_softmax_float_backward
    fallback = original if original is not None else _trl_algorithm

    def forward_rows(logits, idx):
        """(logp, lse, slices): one launch per contiguous slice of rows (a
        copy of the logits only when they have none)."""
        slices = _row_slices(logits)
        if slices is None:
            slices = [logits.reshape(-1, logits.shape[-1]).contiguous()]
        if len(slices) == 1:
            logp, lse = fwd(slices[0], idx, robust)
            return logp, lse, slices
        logp = torch.empty(idx.shape, dtype=torch.float32, device=logits.device)
        lse = torch.empty(idx.shape, dtype=torch.float32, device=logits.device)
        r0 = 0
        for sl in slices:
            r = sl.shape[0]
            fwd(sl, idx[r0:r0 + r], robust, out=(logp[r0:r0 + r], lse[r0:r0 + r]))
            r0 += r
        return logp, lse, slices

    class _SelectiveLogSoftmax(torch.autograd.Function):
        @staticmethod
        def forward(ctx, logits, index):
            idx = index.reshape(-1).to(torch.int64).contiguous()
            logp, lse, slices = forward_rows(logits, idx)
            ctx.save_for_backward(idx, lse, *slices)
            ctx.in_shape = tuple(logits.shape)
            ctx.mark_non_differentiable(lse)
            return logp.reshape(index.shape)

        @staticmethod
        def backward(ctx, grad_out):
            idx, lse, *slices = ctx.saved_tensors
            g = grad_out.reshape(-1).to(torch.float32).contiguous()
            if len(slices) == 1:
                return bwd(g, slices[0], idx, lse).reshape(ctx.in_shape), None
            grad = torch.empty(ctx.in_shape, dtype=torch.float32, device=lse.device)
            rows = grad.view(-1, ctx.in_shape[-1])
            r0 = 0
            for sl in slices:
                r = sl.shape[0]
                bwd(g[r0:r0 + r], sl, idx[r0:r0 + r], lse[r0:r0 + r], out=rows[r0:r0 + r])
                r0 += r
            return grad, None

    def selective_log_softmax(logits, index):
        ok = (logits.is_cuda and logits.dtype == torch.float32 and logits.dim() >= 1
              and index.device == logits.device and not torch.is_floating_point(index)
              and tuple(index.shape) == tuple(logits.shape[:-1]) and logits.shape[-1] >= 1)
        if not ok:
            return fallback(logits, index)
        if torch.is_grad_enabled() and logits.requires_grad:
            return _SelectiveLogSoftmax.apply(logits, index)
        logp, _, _ = forward_rows(logits, index.reshape(-1).to(torch.int64).contiguous())
        return logp.reshape(index.shape)

    selective_log_softmax.fuselse_robust = robust
    return selective_log_softmax
