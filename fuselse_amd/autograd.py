"""Drop-in ``torch.logsumexp`` replacement backed by the gfx950 kernels.

``make_fuselse_logsumexp(ext, robust=True)`` keeps the reference's factory
contract (fuselse/gpu/autograd.py:6-61):

* it reads ``ext.onepass_lse_float_robust`` (or ``ext.onepass_lse_float`` when
  ``robust`` is False) and ``ext.onepass_lse_float_backward``;
* the returned ``logsumexp(input, dim=-1, keepdim=False)`` runs the kernel only
  for a CUDA fp32 tensor reduced over its last dimension with at least two
  elements there, and calls ``torch.logsumexp`` (captured at factory time, so a
  later ``torch.logsumexp = logsumexp`` patch does not recurse) for everything
  else;
* with grad enabled and ``input.requires_grad`` it goes through an autograd
  Function whose backward is the fused ``grad * exp(x - lse)`` kernel (no
  double backward); its forward is the same kernel as without grad, as in the
  reference (autograd.py:15-34);
* a contiguous 2-D input without grad calls the kernel directly; other shapes
  are flattened to (rows, N), made contiguous, and reshaped back;
* ``keepdim`` unsqueezes the last dimension.

``half_inputs=True`` (not in the reference, whose drop-in sends fp16 to torch,
autograd.py:40) also routes CUDA fp16 / bf16 tensors to the kernels: fp32
accumulation, the result rounded to the input dtype as ``torch.logsumexp``
returns it, and a fused half backward from the fp32 LSE.

``keep=True`` (not in the reference) makes the forward under autograd call
``ext.onepass_lse_float[_robust]_keep`` (and its half twins): the same result,
with part of x left in the Infinity Cache for a backward that reads x right
after the forward.  It is off by default: the keeping forward alone is about
4% slower than the plain one, and its gain is gone once other work moves a few
hundred MB through the cache between the forward and its backward, as the rest
of a training step does.
"""

from __future__ import annotations

import torch


def make_fuselse_logsumexp(ext, robust: bool = True, half_inputs: bool = False, keep: bool = False):
    fwd = ext.onepass_lse_float_robust if robust else ext.onepass_lse_float
    # the forward whose backward follows (autograd): with keep, the keeping
    # variant where the ext provides one
    fwd_grad = fwd
    if keep:
        fwd_grad = getattr(ext, ("onepass_lse_float_robust" if robust else "onepass_lse_float") + "_keep", fwd)
    bwd = ext.onepass_lse_float_backward
    torch_logsumexp = torch.logsumexp
    half_fwd = {}
    half_fwd_grad = {}
    if half_inputs:
        half_fwd = {torch.float16: lambda x: ext.batched_logsumexp_fp16(x, robust),
                    torch.bfloat16: lambda x: ext.batched_logsumexp_bf16(x, robust)}
        f16k = getattr(ext, "batched_logsumexp_fp16_keep", ext.batched_logsumexp_fp16) if keep else \
            ext.batched_logsumexp_fp16
        bf16k = getattr(ext, "batched_logsumexp_bf16_keep", ext.batched_logsumexp_bf16) if keep else \
            ext.batched_logsumexp_bf16
        half_fwd_grad = {torch.float16: lambda x: f16k(x, robust), torch.bfloat16: lambda x: bf16k(x, robust)}
        half_bwd = ext.onepass_lse_half_backward

    class _RowLSE(torch.autograd.Function):
        @staticmethod
        def forward(ctx, inp):
            n = inp.shape[-1]
            rows = inp.reshape(-1, n).contiguous()
            lse = fwd_grad(rows)
            ctx.save_for_backward(rows, lse)
            ctx.in_shape = tuple(inp.shape)
            return lse.reshape(inp.shape[:-1])

        @staticmethod
        def backward(ctx, grad_out):
            rows, lse = ctx.saved_tensors
            g = bwd(grad_out.reshape(-1).contiguous(), rows, lse)
            return g.reshape(ctx.in_shape)

    class _HalfRowLSE(torch.autograd.Function):
        """fp16 / bf16 rows: fp32 accumulation, the output rounded to the input
        dtype (torch.logsumexp's dtype contract); the backward uses the fp32
        LSE, not the rounded output."""

        @staticmethod
        def forward(ctx, inp):
            n = inp.shape[-1]
            rows = inp.reshape(-1, n).contiguous()
            lse = half_fwd_grad[inp.dtype](rows)
            ctx.save_for_backward(rows, lse)
            ctx.in_shape = tuple(inp.shape)
            return lse.to(inp.dtype).reshape(inp.shape[:-1])

        @staticmethod
        def backward(ctx, grad_out):
            rows, lse = ctx.saved_tensors
            g = half_bwd(grad_out.reshape(-1).to(torch.float32).contiguous(), rows, lse)
            return g.reshape(ctx.in_shape)

    def logsumexp(input, dim=-1, keepdim=False):
        last = input.dim() - 1
        d = dim if dim >= 0 else input.dim() + dim
        half = input.dtype in half_fwd
        if not (input.is_cuda and (input.dtype == torch.float32 or half) and d == last and input.shape[-1] >= 2):
            return torch_logsumexp(input, dim=dim, keepdim=keepdim)
        if torch.is_grad_enabled() and input.requires_grad:
            out = (_HalfRowLSE if half else _RowLSE).apply(input)
        else:
            n = input.shape[-1]
            rows = input if (input.dim() == 2 and input.is_contiguous()) else input.reshape(-1, n).contiguous()
            out = half_fwd[input.dtype](rows).to(input.dtype) if half else fwd(rows)
            out = out.reshape(input.shape[:-1])
        return out.unsqueeze(-1) if keepdim else out

    logsumexp.fuselse_robust = robust
    logsumexp.fuselse_half_inputs = half_inputs
    logsumexp.fuselse_keep = keep
    return logsumexp
