"""CPU-side checks of the C-ABI library: it loads, exports every symbol the
header declares, the Python binding types all of them, and the shim's argument
validation raises the reference's messages before any GPU call."""

import ctypes

import pytest
import torch

from fuselse_amd import _lib


def test_header_symbols_exported():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert declared, "no fl_* declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/fuselse_amd.h but not exported"
    assert sorted(_lib.SIGNATURES) == declared


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.fl_abi_version() == 1
    assert isinstance(lib.fl_last_error(), bytes)


def test_invalid_arguments_rejected_without_launch():
    """Negative shapes and NULL outputs are refused on the host (no kernel)."""
    lib = _lib.load()
    assert lib.fl_lse_fwd_f32(None, None, -1, 4, 1, None) == 1
    assert b"negative shape" in lib.fl_last_error()
    assert lib.fl_lse_fwd_f32(None, None, 3, 4, 1, None) == 1
    assert b"out is NULL" in lib.fl_last_error()
    assert lib.fl_lse_bwd_f32(None, None, None, None, 2, 3, None) == 1
    assert b"NULL" in lib.fl_last_error()
    # B == 0 is a no-op success
    assert lib.fl_lse_fwd_f32(None, None, 0, 4, 1, None) == 0
    assert lib.fl_last_error() == b""


@pytest.mark.parametrize("fn,args,msg", [
    ("onepass_lse_float", (torch.zeros(2, 3),), "x must be CUDA"),
    ("onepass_lse_float_robust", (torch.zeros(2, 3),), "x must be CUDA"),
    ("onepass_lse_float_backward", (torch.zeros(2), torch.zeros(2, 3), torch.zeros(2)), "grad_output must be CUDA"),
    ("batched_logsumexp_fp16", (torch.zeros(2, 3, dtype=torch.float16),), "Input must be CUDA fp16"),
    ("batched_logsumexp_fp16", (torch.zeros(3, dtype=torch.float16),), "Expected 2-D tensor (B, N)"),
    ("batched_logsumexp_bf16", (torch.zeros(2, 3, dtype=torch.bfloat16),), "Input must be CUDA bf16"),
])
def test_shim_messages_match_reference(fn, args, msg):
    import fuselse_amd

    with pytest.raises(RuntimeError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        getattr(fuselse_amd.ext, fn)(*args)
