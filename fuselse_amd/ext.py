"""The extension object: tensor-level functions under the reference's names.

Each function validates its tensors with the reference's messages (raised as
RuntimeError, like TORCH_CHECK), allocates the output with torch on the input's
device, and enqueues the gfx950 kernel on torch's current stream through the C
ABI.  Passing this module as ``ext`` to ``make_fuselse_logsumexp`` gives the
reference's drop-in (fuselse/gpu/autograd.py:6-61).
"""

from __future__ import annotations

import contextlib

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _stream(t: torch.Tensor):
    return ctypes_stream(torch.cuda.current_stream(t.device))


def ctypes_stream(s) -> int:
    return s.cuda_stream


@contextlib.contextmanager
def _on_device(t: torch.Tensor):
    idx = t.device.index
    if idx is None or idx == torch.cuda.current_device():
        yield
    else:
        with torch.cuda.device(idx):
            yield


def _fwd_f32(x: torch.Tensor, robust: bool) -> torch.Tensor:
    # fused_fp32_kernel.cu:155-158 / :176-179
    _check(x.is_cuda, "x must be CUDA")
    _check(x.dtype == torch.float32, "x must be float32")
    _check(x.dim() == 2, "x must be 2D (B, N)")
    _check(x.is_contiguous(), "x must be contiguous")
    B, N = x.shape
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    if B == 0:
        return out
    with _on_device(x):
        _lib.call("fl_lse_fwd_f32", x.data_ptr(), out.data_ptr(), B, N, int(robust), _stream(x))
    return out


def onepass_lse_float(x: torch.Tensor) -> torch.Tensor:
    """Row LSE of a contiguous fp32 (B, N) CUDA tensor, finite inputs
    (fused_fp32_kernel.cu:154-173)."""
    return _fwd_f32(x, robust=False)


def onepass_lse_float_robust(x: torch.Tensor) -> torch.Tensor:
    """Row LSE with -inf/+inf/NaN semantics (fused_fp32_kernel.cu:175-194)."""
    return _fwd_f32(x, robust=True)


def onepass_lse_float_backward(grad_output: torch.Tensor, x: torch.Tensor, lse_output: torch.Tensor) -> torch.Tensor:
    """grad_input = grad_output[:, None] * exp(x - lse_output[:, None])
    (fused_fp32_kernel.cu:196-252, same checks and messages)."""
    _check(grad_output.is_cuda, "grad_output must be CUDA")
    _check(x.is_cuda, "x must be CUDA")
    _check(lse_output.is_cuda, "lse_output must be CUDA")
    _check(x.dtype == torch.float32, "x must be float32")
    _check(grad_output.dtype == torch.float32, "grad_output must be float32")
    _check(lse_output.dtype == torch.float32, "lse_output must be float32")
    _check(x.dim() == 2, "x must be 2D (B, N)")
    _check(grad_output.dim() == 1, "grad_output must be 1D (B)")
    _check(lse_output.dim() == 1, "lse_output must be 1D (B)")
    _check(x.is_contiguous(), "x must be contiguous")
    _check(grad_output.is_contiguous(), "grad_output must be contiguous")
    _check(lse_output.is_contiguous(), "lse_output must be contiguous")
    _check(grad_output.size(0) == x.size(0), "grad_output batch dimension must match x")
    _check(lse_output.size(0) == x.size(0), "lse_output batch dimension must match x")
    B, N = x.shape
    grad_input = torch.empty_like(x)
    if B * N == 0:
        return grad_input
    with _on_device(x):
        _lib.call("fl_lse_bwd_f32", grad_output.data_ptr(), x.data_ptr(), lse_output.data_ptr(),
                  grad_input.data_ptr(), B, N, _stream(x))
    return grad_input


def _fwd_half(x: torch.Tensor, dtype: torch.dtype, entry: str, dtype_msg: str, robust: bool) -> torch.Tensor:
    # fused_fp16_kernel.cu:113-116
    _check(x.dim() == 2, "Expected 2-D tensor (B, N)")
    _check(x.is_cuda and x.dtype == dtype, dtype_msg)
    _check(x.is_contiguous(), "Input must be contiguous")
    B, N = x.shape
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    if B == 0:
        return out
    with _on_device(x):
        _lib.call(entry, x.data_ptr(), out.data_ptr(), B, N, int(robust), _stream(x))
    return out


def batched_logsumexp_fp16(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """fp16 (B, N) -> fp32 (B,) LSE with fp32 accumulation
    (fused_fp16_kernel.cu:112-132)."""
    return _fwd_half(x, torch.float16, "fl_lse_fwd_f16", "Input must be CUDA fp16", robust)


def batched_logsumexp_bf16(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """bf16 (B, N) -> fp32 (B,) LSE with fp32 accumulation (no reference
    counterpart; the fp16 entry's contract with bf16 storage)."""
    return _fwd_half(x, torch.bfloat16, "fl_lse_fwd_bf16", "Input must be CUDA bf16", robust)
