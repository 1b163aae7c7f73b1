"""The extension object: tensor-level functions under the reference's names.

Each function validates its tensors with the reference's messages (raised as
RuntimeError, like TORCH_CHECK), allocates the output with torch on the input's
device, and enqueues the gfx950 kernel on torch's current stream through the C
ABI.  Passing this module as ``ext`` to ``make_fuselse_logsumexp`` gives the
reference's drop-in (fuselse/gpu/autograd.py:6-61).
"""

from __future__ import annotations

from typing import NamedTuple, Optional

import torch

from . import _lib


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_device(ref: torch.Tensor, ref_name: str, **others) -> None:
    """Every tensor of `others` (name=tensor; None is skipped) is on ref's
    GPU: the kernels dereference every pointer on the launching device, where
    another GPU's memory is not an operand."""
    for name, t in others.items():
        if t is not None:
            _check(t.device == ref.device, f"{name} must be on the same device as {ref_name}")


# torch's raw current-stream query (what its own compiled kernels use) costs
# a fraction of building a torch.cuda.Stream object; the public form is the
# fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor):
    if _raw_stream is not None:
        idx = t.device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return ctypes_stream(torch.cuda.current_stream(t.device))


def ctypes_stream(s) -> int:
    return s.cuda_stream


class _Same:
    """The no-op device guard (the tensor is on the current device)."""

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_SAME = _Same()


def _on_device(t: torch.Tensor):
    """A guard that makes t's device current for the enclosed launch."""
    idx = t.device.index
    if idx is None or idx == torch.cuda.current_device():
        return _SAME
    return torch.cuda.device(idx)


_ws_cache = {}


def _workspace_bytes(B: int, N: int, elem_bytes: int) -> int:
    """Bytes of split-row workspace the library's plan asks for at (B, N)
    (0: the one-pass kernels).  The plan is a fixed function of the shape, so
    each shape is asked once: the query is a second foreign call, about as
    long as the launch itself."""
    key = (B, N, elem_bytes)
    nbytes = _ws_cache.get(key)
    if nbytes is None:
        if len(_ws_cache) >= 4096:
            _ws_cache.clear()
        nbytes = _ws_cache[key] = _lib.load().fl_lse_fwd_workspace_bytes(B, N, elem_bytes)
    return nbytes


def _launch_fwd(entry: str, x: torch.Tensor, out: torch.Tensor, elem_bytes: int, robust: bool,
                keep: bool = False) -> None:
    """One-pass kernels (entry + "_keep" with keep: x partly left in the
    Infinity Cache for the backward), or the split-row kernels (entry +
    "_ws") for few long rows, where the library asks for a workspace."""
    B, N = x.shape
    with _on_device(x):
        nbytes = _workspace_bytes(B, N, elem_bytes)
        if nbytes:
            # partials between the two split kernels; stream-ordered reuse by
            # torch's caching allocator keeps it valid until they have run
            ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
            _lib.call(entry + "_ws", x.data_ptr(), out.data_ptr(), B, N, int(robust), ws.data_ptr(), ws.numel(),
                      _stream(x))
        else:
            _lib.call(entry + "_keep" if keep else entry, x.data_ptr(), out.data_ptr(), B, N, int(robust),
                      _stream(x))


def _fwd_f32(x: torch.Tensor, robust: bool, keep: bool = False) -> torch.Tensor:
    # fused_fp32_kernel.cu:155-158 / :176-179
    _check(x.is_cuda, "x must be CUDA")
    _check(x.dtype == torch.float32, "x must be float32")
    _check(x.dim() == 2, "x must be 2D (B, N)")
    _check(x.is_contiguous(), "x must be contiguous")
    B, N = x.shape
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    if B == 0:
        return out
    _launch_fwd("fl_lse_fwd_f32", x, out, 4, robust, keep)
    return out


def onepass_lse_float(x: torch.Tensor) -> torch.Tensor:
    """Row LSE of a contiguous fp32 (B, N) CUDA tensor, finite inputs
    (fused_fp32_kernel.cu:154-173)."""
    return _fwd_f32(x, robust=False)


def onepass_lse_float_robust(x: torch.Tensor) -> torch.Tensor:
    """Row LSE with -inf/+inf/NaN semantics (fused_fp32_kernel.cu:175-194)."""
    return _fwd_f32(x, robust=True)


def onepass_lse_float_keep(x: torch.Tensor) -> torch.Tensor:
    """onepass_lse_float for a backward that reads x next: the same result,
    with part of x left in the Infinity Cache for that read
    (fl_lse_fwd_f32_keep; no reference counterpart)."""
    return _fwd_f32(x, robust=False, keep=True)


def onepass_lse_float_robust_keep(x: torch.Tensor) -> torch.Tensor:
    """onepass_lse_float_robust for a backward that reads x next
    (fl_lse_fwd_f32_keep; no reference counterpart)."""
    return _fwd_f32(x, robust=True, keep=True)


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
    _check_device(x, "x", grad_output=grad_output, lse_output=lse_output)
    B, N = x.shape
    grad_input = torch.empty_like(x)
    if B * N == 0:
        return grad_input
    with _on_device(x):
        _lib.call("fl_lse_bwd_f32", grad_output.data_ptr(), x.data_ptr(), lse_output.data_ptr(),
                  grad_input.data_ptr(), B, N, _stream(x))
    return grad_input


def selective_log_softmax_float(logits: torch.Tensor, index: torch.Tensor, robust: bool = True, out=None):
    """Fused selective log-softmax over fp32 (B, N) logits and int64 (B,)
    targets: returns (logp, lse) with logp[r] = logits[r, index[r]] - lse[r],
    in one pass over the logits.  It fuses the fp32 branch of
    trl.trainer.utils.selective_log_softmax (trl 1.0.0: gather, per-row
    torch.logsumexp, subtraction), which the reference's RLHF experiment
    times (experiment_rlhf_logsumexp/run_rlhf.py:28,145,155).  An index
    outside [0, N) gives NaN.  out: an optional (logp, lse) pair of
    contiguous fp32 (B,) tensors to write."""
    _check(logits.is_cuda, "logits must be CUDA")
    _check(index.is_cuda, "index must be CUDA")
    _check(logits.dtype == torch.float32, "logits must be float32")
    _check(index.dtype == torch.int64, "index must be int64")
    _check(logits.dim() == 2, "logits must be 2D (B, N)")
    _check(index.dim() == 1, "index must be 1D (B)")
    _check(logits.is_contiguous(), "logits must be contiguous")
    _check(index.is_contiguous(), "index must be contiguous")
    _check(index.size(0) == logits.size(0), "index batch dimension must match logits")
    _check_device(logits, "logits", index=index)
    B, N = logits.shape
    if out is None:
        logp = torch.empty((B,), dtype=torch.float32, device=logits.device)
        lse = torch.empty((B,), dtype=torch.float32, device=logits.device)
    else:
        logp, lse = out
        for t in (logp, lse):
            _check(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous() and tuple(t.shape) == (B,)
                   and t.device == logits.device, "out must hold two contiguous CUDA float32 (B,) tensors")
    if B == 0:
        return logp, lse
    with _on_device(logits):
        nbytes = _workspace_bytes(B, N, 4)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=logits.device) if nbytes else None
        _lib.call("fl_selective_logsoftmax_f32", logits.data_ptr(), index.data_ptr(), logp.data_ptr(),
                  lse.data_ptr(), B, N, int(robust), ws.data_ptr() if ws is not None else None, nbytes,
                  _stream(logits))
    return logp, lse


def selective_log_softmax_float_backward(grad_output: torch.Tensor, logits: torch.Tensor, index: torch.Tensor,
                                         lse: torch.Tensor, out=None) -> torch.Tensor:
    """grad_logits[r, i] = grad_output[r] * ((i == index[r]) - exp(logits[r, i] - lse[r])),
    one pass over the logits.  out: an optional contiguous fp32 (B, N) tensor
    to write."""
    for t, nm in ((grad_output, "grad_output"), (logits, "logits"), (index, "index"), (lse, "lse")):
        _check(t.is_cuda, f"{nm} must be CUDA")
        _check(t.is_contiguous(), f"{nm} must be contiguous")
    _check(logits.dtype == torch.float32 and grad_output.dtype == torch.float32 and lse.dtype == torch.float32,
           "grad_output, logits and lse must be float32")
    _check(index.dtype == torch.int64, "index must be int64")
    _check(logits.dim() == 2, "logits must be 2D (B, N)")
    _check(grad_output.dim() == 1 and index.dim() == 1 and lse.dim() == 1, "grad_output, index and lse must be 1D (B)")
    B, N = logits.shape
    _check(grad_output.size(0) == B and index.size(0) == B and lse.size(0) == B,
           "grad_output, index and lse batch dimensions must match logits")
    _check_device(logits, "logits", grad_output=grad_output, index=index, lse=lse)
    if out is None:
        grad = torch.empty_like(logits)
    else:
        grad = out
        _check(grad.is_cuda and grad.dtype == torch.float32 and grad.is_contiguous()
               and tuple(grad.shape) == (B, N) and grad.device == logits.device,
               "out must be a contiguous CUDA float32 (B, N) tensor")
    if B * N == 0:
        return grad
    with _on_device(logits):
        _lib.call("fl_selective_logsoftmax_bwd_f32", grad_output.data_ptr(), logits.data_ptr(), index.data_ptr(),
                  lse.data_ptr(), grad.data_ptr(), B, N, _stream(logits))
    return grad


def _fwd_half(x: torch.Tensor, dtype: torch.dtype, entry: str, dtype_msg: str, robust: bool,
              keep: bool = False) -> torch.Tensor:
    # fused_fp16_kernel.cu:113-116
    _check(x.dim() == 2, "Expected 2-D tensor (B, N)")
    _check(x.is_cuda and x.dtype == dtype, dtype_msg)
    _check(x.is_contiguous(), "Input must be contiguous")
    B, N = x.shape
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    if B == 0:
        return out
    _launch_fwd(entry, x, out, 2, robust, keep)
    return out


def onepass_lse_half_backward(grad_output: torch.Tensor, x: torch.Tensor, lse_output: torch.Tensor) -> torch.Tensor:
    """grad_input = grad_output[:, None] * exp(x - lse_output[:, None]) for fp16 or
    bf16 x (B, N), fp32 grad_output and lse_output (B,); the result has x's
    dtype (fp32 arithmetic, round to nearest even).  No reference
    counterpart: the fp32 backward's contract (fused_fp32_kernel.cu:196-252)
    at half storage."""
    _check(grad_output.is_cuda and x.is_cuda and lse_output.is_cuda, "grad_output, x and lse_output must be CUDA")
    _check(x.dtype in (torch.float16, torch.bfloat16), "x must be float16 or bfloat16")
    _check(grad_output.dtype == torch.float32 and lse_output.dtype == torch.float32,
           "grad_output and lse_output must be float32")
    _check(x.dim() == 2, "x must be 2D (B, N)")
    _check(grad_output.dim() == 1 and lse_output.dim() == 1, "grad_output and lse_output must be 1D (B)")
    _check(x.is_contiguous() and grad_output.is_contiguous() and lse_output.is_contiguous(),
           "inputs must be contiguous")
    _check(grad_output.size(0) == x.size(0) and lse_output.size(0) == x.size(0),
           "grad_output and lse_output batch dimensions must match x")
    _check_device(x, "x", grad_output=grad_output, lse_output=lse_output)
    B, N = x.shape
    grad_input = torch.empty_like(x)
    if B * N == 0:
        return grad_input
    entry = "fl_lse_bwd_f16" if x.dtype == torch.float16 else "fl_lse_bwd_bf16"
    with _on_device(x):
        _lib.call(entry, grad_output.data_ptr(), x.data_ptr(), lse_output.data_ptr(), grad_input.data_ptr(), B, N,
                  _stream(x))
    return grad_input


def batched_logsumexp_fp16(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """fp16 (B, N) -> fp32 (B,) LSE with fp32 accumulation
    (fused_fp16_kernel.cu:112-132)."""
    return _fwd_half(x, torch.float16, "fl_lse_fwd_f16", "Input must be CUDA fp16", robust)


def batched_logsumexp_bf16(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """bf16 (B, N) -> fp32 (B,) LSE with fp32 accumulation (no reference
    counterpart; the fp16 entry's contract with bf16 storage)."""
    return _fwd_half(x, torch.bfloat16, "fl_lse_fwd_bf16", "Input must be CUDA bf16", robust)


def batched_logsumexp_fp16_keep(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """batched_logsumexp_fp16 for a backward that reads x next
    (fl_lse_fwd_f16_keep; no reference counterpart)."""
    return _fwd_half(x, torch.float16, "fl_lse_fwd_f16", "Input must be CUDA fp16", robust, keep=True)


def batched_logsumexp_bf16_keep(x: torch.Tensor, robust: bool = False) -> torch.Tensor:
    """batched_logsumexp_bf16 for a backward that reads x next
    (fl_lse_fwd_bf16_keep; no reference counterpart)."""
    return _fwd_half(x, torch.bfloat16, "fl_lse_fwd_bf16", "Input must be CUDA bf16", robust, keep=True)


# ---------------------------------------------------------------------------
# IntLSE (fixed point)
# ---------------------------------------------------------------------------
def _acc_ptr(acc_out, input: torch.Tensor) -> int:
    """Device pointer of the optional raw-accumulator output: the kernels write
    acc_out[r] for every row r < B, so it must hold B int32 on input's GPU."""
    if acc_out is None:
        return 0
    _check(acc_out.is_cuda and acc_out.dtype == torch.int32 and acc_out.is_contiguous(),
           "acc_out must be a contiguous CUDA int32 tensor")
    _check(acc_out.device == input.device, "acc_out must be on the input's device")
    _check(acc_out.numel() >= input.shape[0], "acc_out must hold one int32 per row")
    return acc_out.data_ptr()


def _intlse_q16_f32(input: torch.Tensor, use_lut: bool, acc_out=None) -> torch.Tensor:
    # lse_kernel.cu:187-189 (the dtype/device check carries no message there)
    _check(input.dim() == 2, "Expected 2-D tensor (B, N)")
    _check(input.is_cuda and input.dtype == torch.float32,
           "Expected input.is_cuda() && input.dtype() == torch::kFloat32 to be true, but got false.")
    _check(input.is_contiguous(), "Input must be contiguous")
    B, N = input.shape
    out = torch.empty((B,), dtype=torch.float32, device=input.device)
    if B == 0:
        return out
    with _on_device(input):
        _lib.call("fl_intlse_q16_f32", input.data_ptr(), out.data_ptr(), _acc_ptr(acc_out, input), B, N, int(use_lut),
                  _stream(input))
    return out


def batched_logsumexp(input: torch.Tensor, acc_out=None) -> torch.Tensor:
    """Q16.16 IntLSE of fp32 (B, N) base-e logits -> fp32 (B,) base-e
    (intlse/gpu/lse_kernel.cu:186-193); bit-exact reference tree."""
    return _intlse_q16_f32(input, True, acc_out)


def batched_logsumexp_nolut(input: torch.Tensor, acc_out=None) -> torch.Tensor:
    """The same without the correction table (lse_kernel.cu:195-202)."""
    return _intlse_q16_f32(input, False, acc_out)


def batched_logsumexp_q16_i32(input: torch.Tensor, use_lut: bool = True, acc_out=None) -> torch.Tensor:
    """Q16.16 IntLSE of pre-quantised int32 (B, N) base-2 values -> fp32 (B,)
    base-e, with the reference's tree (no reference entry point)."""
    _check(input.dim() == 2, "Expected 2-D tensor (B, N)")
    _check(input.is_cuda, "Input must be CUDA")
    _check(input.dtype == torch.int32, "Input must be int32 (Q16.16 base-2 fixed-point)")
    _check(input.is_contiguous(), "Input must be contiguous")
    B, N = input.shape
    out = torch.empty((B,), dtype=torch.float32, device=input.device)
    if B == 0:
        return out
    with _on_device(input):
        _lib.call("fl_intlse_q16_i32", input.data_ptr(), out.data_ptr(), _acc_ptr(acc_out, input), B, N, int(use_lut),
                  _stream(input))
    return out


def batched_logsumexp_q10_6(input: torch.Tensor, acc_out=None) -> torch.Tensor:
    """Q10.6 IntLSE of int16 (B, N) base-2 values -> fp32 (B,) base-e
    (intlse/gpu/lse_kernel_q10_6.cu:144-165, same checks and messages)."""
    _check(input.dim() == 2, "Expected 2-D tensor (B, N)")
    _check(input.is_cuda, "Input must be CUDA")
    _check(input.dtype == torch.int16, "Input must be int16 (Q10.6 base-2 fixed-point)")
    _check(input.is_contiguous(), "Input must be contiguous")
    B, N = input.shape
    out = torch.empty((B,), dtype=torch.float32, device=input.device)
    if B == 0:
        return out
    with _on_device(input):
        _lib.call("fl_intlse_q10_6", input.data_ptr(), out.data_ptr(), _acc_ptr(acc_out, input), B, N, _stream(input))
    return out


# ---------------------------------------------------------------------------
# Sparse probabilistic-circuit sum layers
# ---------------------------------------------------------------------------
def _sparse_blocked(node_mars, element_mars, params, nids, cids, pids, block_size, q16, params_are_log):
    # sparse_float_kernel.cu:119-121 / sparse_q16_kernel.cu:320-322
    _check(node_mars.is_cuda, "node_mars must be CUDA")
    _check(element_mars.is_cuda, "element_mars must be CUDA")
    _check(params.is_cuda, "params must be CUDA")
    # layout checks the reference leaves to the caller (a mismatch would read
    # out of bounds on the device)
    _check(node_mars.dtype == torch.float32 and element_mars.dtype == torch.float32 and params.dtype == torch.float32,
           "node_mars, element_mars and params must be float32")
    _check(node_mars.dim() == 2 and element_mars.dim() == 2 and node_mars.size(1) == element_mars.size(1),
           "node_mars and element_mars must be 2-D [nodes, batch] with the same batch")
    _check(node_mars.is_contiguous() and element_mars.is_contiguous() and params.is_contiguous(),
           "node_mars, element_mars and params must be contiguous")
    for name, t in (("nids", nids), ("cids", cids), ("pids", pids)):
        _check(t.is_cuda and t.dtype == torch.int64 and t.is_contiguous(), f"{name} must be a contiguous CUDA int64 tensor")
    _check(cids.dim() == 2 and pids.shape == cids.shape and nids.dim() == 1 and nids.size(0) == cids.size(0),
           "nids [nblocks], cids and pids [nblocks, num_edges] shapes disagree")
    _check_device(node_mars, "node_mars", element_mars=element_mars, params=params, nids=nids, cids=cids, pids=pids)
    batch = node_mars.size(1)
    num_nblocks = nids.size(0)
    num_edges = cids.size(1)
    if batch == 0 or num_nblocks == 0 or block_size == 0:
        return None
    with _on_device(node_mars):
        _lib.call("fl_sparse_blocked_fwd", node_mars.data_ptr(), element_mars.data_ptr(), params.data_ptr(),
                  nids.data_ptr(), cids.data_ptr(), pids.data_ptr(), num_nblocks, num_edges, int(block_size), batch,
                  int(q16), int(params_are_log), _stream(node_mars))
    return None


def sparse_forward_float(node_mars, element_mars, params, nids, cids, pids, block_size, params_are_log=False):
    """pyjuice sum-layer forward in fp32, in place on node_mars
    (experiment_pyjuice/sparse_float_kernel.cu:110-167):
    node_mars[nids[j] + p, b] = LSE_e(log max(params[pids[j, e] + p], 1e-45)
    + element_mars[cids[j, e], b]).  Returns None."""
    return _sparse_blocked(node_mars, element_mars, params, nids, cids, pids, block_size, False, params_are_log)


def sparse_forward_q16(node_mars, element_mars, params, nids, cids, pids, block_size, params_are_log=False):
    """The same in IntLSE Q16.16 with the reference's edge-thread tree
    (experiment_pyjuice/sparse_q16_kernel.cu:139-202).  Returns None."""
    return _sparse_blocked(node_mars, element_mars, params, nids, cids, pids, block_size, True, params_are_log)


class BlockedPlan(NamedTuple):
    """The transposed structure of a block-layout sum layer (see
    sparse_blocked_transpose)."""
    csc_offsets: torch.Tensor   # int64 [num_elements + 1]
    csc_edges: torch.Tensor     # int32 [nblocks * num_edges]: block edges j * num_edges + e, by child
    csc_nodes: Optional[torch.Tensor]  # int32, block_size 1 only: node_mars row of each listed edge
    param_ids: Optional[torch.Tensor]  # int64 [nblocks * num_edges], block_size 1 only: pids flattened
    # no two (block, parent, edge) triples share a parameter: the ranges
    # [pids[j, e], pids[j, e] + block_size) do not overlap
    params_disjoint: bool = False


def sparse_blocked_transpose(nids, cids, pids, block_size, num_elements):
    """The transposed structure sparse_blocked_backward walks for a block-layout
    sum layer (the forward dispatcher's nids [nblocks], cids and pids
    [nblocks, num_edges], int64): for each element row c, the block edges
    j * num_edges + e with cids[j, e] = c, in increasing order.  Built with
    torch's sort on the device; it depends on the layer only, so a caller that
    runs the layer many times builds it once and passes it to
    sparse_blocked_backward."""
    for name, t in (("nids", nids), ("cids", cids), ("pids", pids)):
        _check(t.is_cuda and t.dtype == torch.int64 and t.is_contiguous(), f"{name} must be a contiguous CUDA int64 tensor")
    _check(cids.dim() == 2 and pids.shape == cids.shape and nids.dim() == 1 and nids.size(0) == cids.size(0),
           "nids [nblocks], cids and pids [nblocks, num_edges] shapes disagree")
    _check_device(cids, "cids", nids=nids, pids=pids)
    return _blocked_plan(nids, cids, pids, block_size, num_elements)


def _blocked_plan(nids, cids, pids, block_size, num_elements):
    """sparse_blocked_transpose's construction, on the tensors' own device."""
    nb, ne = cids.shape
    bs = int(block_size)
    _check(nb * ne < 2 ** 31 and nb * bs * ne < 2 ** 31 and num_elements < 2 ** 31,
           "edges and element rows must each be < 2^31")
    dev = cids.device
    child_ids = cids.reshape(-1)
    _check(child_ids.numel() == 0 or int(child_ids.min()) >= 0, "cids hold negative ids")
    order = torch.sort(child_ids, stable=True).indices
    counts = torch.bincount(child_ids, minlength=num_elements)
    _check(counts.numel() == num_elements, "cids hold ids >= element_mars rows")
    csc_off = torch.zeros(num_elements + 1, dtype=torch.int64, device=dev)
    torch.cumsum(counts, 0, out=csc_off[1:])
    nodes = qids = None
    if bs == 1:
        # one parent per block: the block edges are the layer's edges, walked by
        # the CSR flows kernel, which names each edge's node_mars row
        nodes = nids[order // ne].to(torch.int32)
        qids = pids.reshape(-1)
    # parameter ranges of the block edges, sorted: disjoint when consecutive
    # starts are at least block_size apart (then each parameter flow has one
    # writer and takes a plain add instead of an atomic one)
    starts = torch.sort(pids.reshape(-1)).values
    disjoint = bool(starts.numel() < 2 or int((starts[1:] - starts[:-1]).min()) >= bs)
    return BlockedPlan(csc_off, order.to(torch.int32), nodes, qids, disjoint)


def sparse_blocked_backward(node_flows, element_flows, node_mars, element_mars, params, param_flows, nids, cids, pids,
                            block_size, params_are_log=False, plan=None):
    """Flows of the block-layout sum layer of sparse_forward_float (pyjuice's
    layout, as the forward dispatcher passes it), in fp32, added in place:
    for block j, position p < block_size and edge e, with n = nids[j] + p,
    c = cids[j, e] and q = pids[j, e] + p,
      term[b] = node_flows[n, b] * exp(lw_q + element_mars[c, b] - node_mars[n, b])
    (lw_q = log max(params[q], 1e-45), or params[q] itself when
    params_are_log; term = 0 where node_mars is -inf),
      element_flows[c, b] += the terms of the edges into c,
      param_flows[q]      += the terms of edge (j, p, e) summed over b.
    node_mars must hold this layer's forward output.  The reference has no
    sparse backward.  block_size >= 2 runs fl_sparse_blocked_bwd (products on
    the matrix cores, a workspace of nblocks * num_edges rows); block_size 1
    runs the CSR flows kernel fl_sparse_csr_bwd over the same edges.  plan:
    the result of sparse_blocked_transpose for this layer (built here when
    None).  param_flows receives one add per (block, parent, edge), in any
    order where several of them share a parameter.  Returns None."""
    _check(node_flows.is_cuda and element_flows.is_cuda and param_flows.is_cuda, "flows must be CUDA tensors")
    for t, nm in ((node_flows, "node_flows"), (element_flows, "element_flows"), (param_flows, "param_flows")):
        _check(t.dtype == torch.float32 and t.is_contiguous(), f"{nm} must be contiguous float32")
    _check(tuple(node_flows.shape) == tuple(node_mars.shape), "node_flows must have node_mars's shape")
    _check(tuple(element_flows.shape) == tuple(element_mars.shape), "element_flows must have element_mars's shape")
    _check(param_flows.numel() == params.numel(), "param_flows must have params's size")
    # the forward's layout checks
    _check(node_mars.is_cuda and element_mars.is_cuda and params.is_cuda, "node_mars, element_mars, params must be CUDA")
    _check(node_mars.dtype == torch.float32 and element_mars.dtype == torch.float32 and params.dtype == torch.float32,
           "node_mars, element_mars and params must be float32")
    _check(node_mars.dim() == 2 and element_mars.dim() == 2 and node_mars.size(1) == element_mars.size(1),
           "node_mars and element_mars must be 2-D [nodes, batch] with the same batch")
    _check(node_mars.is_contiguous() and element_mars.is_contiguous() and params.is_contiguous(),
           "node_mars, element_mars and params must be contiguous")
    for name, t in (("nids", nids), ("cids", cids), ("pids", pids)):
        _check(t.is_cuda and t.dtype == torch.int64 and t.is_contiguous(), f"{name} must be a contiguous CUDA int64 tensor")
    _check(cids.dim() == 2 and pids.shape == cids.shape and nids.dim() == 1 and nids.size(0) == cids.size(0),
           "nids [nblocks], cids and pids [nblocks, num_edges] shapes disagree")
    _check_device(node_mars, "node_mars", node_flows=node_flows, element_flows=element_flows,
                  element_mars=element_mars, params=params, param_flows=param_flows, nids=nids, cids=cids, pids=pids)
    nb, ne = cids.shape
    bs = int(block_size)
    num_el, batch = element_mars.shape
    if nb * ne * bs == 0 or batch == 0:
        return None
    _check(nb * bs * ne < 2 ** 31 and num_el < 2 ** 31 and node_mars.size(0) < 2 ** 31,
           "edges, element rows and node rows must each be < 2^31")
    if plan is None:
        plan = sparse_blocked_transpose(nids, cids, pids, bs, num_el)
    csc_off, csc_edge, csc_node, q, disjoint = plan
    _check_device(node_mars, "node_mars", csc_offsets=csc_off, csc_edges=csc_edge, csc_nodes=csc_node, param_ids=q)
    _check(csc_off.dtype == torch.int64 and csc_off.numel() == num_el + 1 and csc_edge.dtype == torch.int32
           and csc_edge.numel() == nb * ne and (bs != 1 or (csc_node is not None and q is not None
                                                             and csc_node.numel() == nb * ne and q.numel() == nb * ne)),
           "plan does not fit this layer")
    if bs == 1:
        w = params.reshape(-1)[q]
        logp = (w if params_are_log else torch.log(torch.clamp_min(w, 1e-45))).contiguous()
        grad_el = torch.empty_like(element_mars)
        grad_lp = torch.empty_like(logp)
        with _on_device(element_mars):
            _lib.call("fl_sparse_csr_bwd", element_mars.data_ptr(), node_mars.data_ptr(), node_flows.data_ptr(),
                      logp.data_ptr(), csc_off.data_ptr(), csc_edge.data_ptr(), csc_node.data_ptr(), grad_el.data_ptr(),
                      grad_lp.data_ptr(), num_el, batch, _stream(element_mars))
        element_flows.add_(grad_el)
        param_flows.view(-1).index_add_(0, q, grad_lp)
        return None
    edge_flows = torch.empty(nb * ne, batch, dtype=torch.float32, device=element_mars.device)
    with _on_device(element_mars):
        _lib.call("fl_sparse_blocked_bwd", node_flows.data_ptr(), node_mars.data_ptr(), element_mars.data_ptr(),
                  params.data_ptr(), nids.data_ptr(), cids.data_ptr(), pids.data_ptr(), nb, ne, bs, batch,
                  int(params_are_log), int(disjoint), csc_off.data_ptr(), csc_edge.data_ptr(), num_el,
                  edge_flows.data_ptr(),
                  element_flows.data_ptr(), param_flows.data_ptr(), _stream(element_mars))
    return None


def sparse_csr_forward(child, offsets, child_ids, logparams, q16=False, out=None):
    """CSR sum layer: out[n, b] = LSE_{e in [offsets[n], offsets[n+1])}
    (logparams[e] + child[child_ids[e], b]); -inf for a node without edges.
    child: fp32 [num_children, batch]; offsets int64 [num_nodes + 1];
    child_ids int32 [nnz]; logparams fp32 [nnz].  Returns out [num_nodes, batch]."""
    _check(child.is_cuda and child.dtype == torch.float32 and child.dim() == 2 and child.is_contiguous(),
           "child must be a contiguous CUDA float32 [num_children, batch] tensor")
    _check(offsets.is_cuda and offsets.dtype == torch.int64 and offsets.dim() == 1 and offsets.is_contiguous(),
           "offsets must be a contiguous CUDA int64 [num_nodes + 1] tensor")
    _check(child_ids.is_cuda and child_ids.dtype == torch.int32 and child_ids.is_contiguous(),
           "child_ids must be a contiguous CUDA int32 tensor")
    _check(logparams.is_cuda and logparams.dtype == torch.float32 and logparams.is_contiguous()
           and logparams.numel() == child_ids.numel(), "logparams must be contiguous CUDA float32, one per edge")
    _check_device(child, "child", offsets=offsets, child_ids=child_ids, logparams=logparams, out=out)
    num_nodes = offsets.numel() - 1
    batch = child.size(1)
    if out is None:
        out = torch.empty((max(num_nodes, 0), batch), dtype=torch.float32, device=child.device)
    _check(out.is_cuda and out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == (num_nodes, batch),
           "out must be a contiguous CUDA float32 [num_nodes, batch] tensor")
    if num_nodes <= 0 or batch == 0:
        return out
    with _on_device(child):
        _lib.call("fl_sparse_csr_fwd", child.data_ptr(), offsets.data_ptr(), child_ids.data_ptr(), logparams.data_ptr(),
                  out.data_ptr(), num_nodes, batch, int(q16), _stream(child))
    return out


def sparse_csr_transpose(offsets, child_ids, num_children):
    """The transposed (CSC) edge structure fl_sparse_csr_bwd walks: returns
    (csc_offsets int64 [num_children + 1], csc_edges int32 [nnz] with the ids
    of the edges pointing at each child in increasing order, csc_nodes int32
    [nnz] with each of those edges' parent node).  Built once per layer with
    torch's sort on the device; the structure does not depend on the batch."""
    _check(offsets.is_cuda and offsets.dtype == torch.int64 and offsets.dim() == 1,
           "offsets must be a CUDA int64 [num_nodes + 1] tensor")
    _check(child_ids.is_cuda and child_ids.dtype == torch.int32, "child_ids must be a CUDA int32 tensor")
    _check_device(child_ids, "child_ids", offsets=offsets)
    nnz = child_ids.numel()
    _check(nnz < 2 ** 31 and num_children < 2 ** 31, "CSC ids are int32: nnz and num_children must be < 2^31")
    num_nodes = offsets.numel() - 1
    dev = child_ids.device
    node_of_edge = torch.repeat_interleave(torch.arange(num_nodes, device=dev), offsets.diff(), output_size=nnz)
    order = torch.sort(child_ids.long(), stable=True).indices
    counts = torch.bincount(child_ids.long(), minlength=num_children)
    _check(counts.numel() == num_children, "child_ids hold ids >= num_children")
    csc_offsets = torch.zeros(num_children + 1, dtype=torch.int64, device=dev)
    torch.cumsum(counts, 0, out=csc_offsets[1:])
    return csc_offsets, order.to(torch.int32), node_of_edge[order].to(torch.int32)


def sparse_csr_backward(child, out, grad_out, offsets, child_ids, logparams, csc=None):
    """Backward (flows) of sparse_csr_forward in fp32: returns (grad_child,
    grad_logparams) with
      term[e, b] = grad_out[n_e, b] * exp(logparams[e] + child[c_e, b] - out[n_e, b])
    summed over the edges of each child and over the batch of each edge, and
    term = 0 where out is -inf.  csc: the result of sparse_csr_transpose for
    this layer (built here when None)."""
    for t, nm in ((child, "child"), (out, "out"), (grad_out, "grad_out"), (logparams, "logparams")):
        _check(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(), f"{nm} must be contiguous CUDA float32")
    _check(child.dim() == 2 and out.dim() == 2 and tuple(grad_out.shape) == tuple(out.shape),
           "child [num_children, batch], out and grad_out [num_nodes, batch]")
    _check(out.size(1) == child.size(1), "out and child batch dimensions must match")
    _check(logparams.numel() == child_ids.numel(), "logparams must hold one value per edge")
    num_children, batch = child.shape
    _check(out.size(0) == offsets.numel() - 1, "out rows must match offsets")
    if csc is None:
        csc = sparse_csr_transpose(offsets, child_ids, num_children)
    csc_off, csc_edge, csc_node = csc
    _check_device(child, "child", out=out, grad_out=grad_out, logparams=logparams, csc_offsets=csc_off,
                  csc_edges=csc_edge, csc_nodes=csc_node)
    _check(csc_off.dtype == torch.int64 and csc_off.numel() == num_children + 1 and csc_edge.dtype == torch.int32
           and csc_node.dtype == torch.int32 and csc_edge.numel() == child_ids.numel(), "csc does not fit this layer")
    grad_child = torch.empty_like(child)
    grad_logp = torch.empty_like(logparams)
    if num_children == 0 or batch == 0:
        grad_child.zero_()
        grad_logp.zero_()
        return grad_child, grad_logp
    if child_ids.numel() == 0:
        grad_child.zero_()
        return grad_child, grad_logp
    with _on_device(child):
        _lib.call("fl_sparse_csr_bwd", child.data_ptr(), out.data_ptr(), grad_out.data_ptr(), logparams.data_ptr(),
                  csc_off.data_ptr(), csc_edge.data_ptr(), csc_node.data_ptr(), grad_child.data_ptr(),
                  grad_logp.data_ptr(), num_children, batch, _stream(child))
    return grad_child, grad_logp
