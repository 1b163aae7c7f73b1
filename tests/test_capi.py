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
    assert not [n for n in declared if n.startswith("fl_diag")], "measurement kernels belong to the diag library"


def test_diag_header_symbols_exported():
    """The measurement library exports what include/fuselse_amd_diag.h
    declares, and the row-LSE library exports none of it."""
    diag = _lib.load_diag()
    declared = _lib.header_symbols(_lib.DIAG_HEADER_PATH)
    assert declared and all(n.startswith("fl_diag_") for n in declared)
    for name in declared:
        assert hasattr(diag, name), f"{name} declared in include/fuselse_amd_diag.h but not exported"
    assert sorted(_lib.DIAG_SIGNATURES) == declared
    main = _lib.load()
    for name in declared:
        with pytest.raises(AttributeError):
            getattr(main, name)


def test_abi_version_and_error_string():
    lib = _lib.load()
    assert lib.fl_abi_version() == 1
    assert isinstance(lib.fl_last_error(), bytes)


@pytest.mark.parametrize("contents", [None, b"not an ELF object"])
def test_missing_library_raises(monkeypatch, tmp_path, contents):
    """An absent or unloadable library raises NativeLibraryMissing from the
    first call: there is no CPU path to fall back on."""
    path = tmp_path / "libfuselse_amd.so"
    if contents is not None:
        path.write_bytes(contents)
    monkeypatch.setattr(_lib, "LIB_PATH", str(path))
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "_bound", {})
    with pytest.raises(_lib.NativeLibraryMissing, match="not built" if contents is None else "cannot load"):
        _lib.call("fl_lse_fwd_f32", None, None, 2, 3, 1, None)
    assert issubclass(_lib.NativeLibraryMissing, RuntimeError)


def test_invalid_arguments_rejected_without_launch():
    """Negative shapes and NULL outputs are refused on the host (no kernel)."""
    lib = _lib.load()
    assert lib.fl_lse_fwd_f32(None, None, -1, 4, 1, None) == 1
    assert b"negative shape" in lib.fl_last_error()
    assert lib.fl_lse_fwd_f32(None, None, 3, 4, 1, None) == 1
    assert b"out is NULL" in lib.fl_last_error()
    assert lib.fl_lse_bwd_f32(None, None, None, None, 2, 3, None) == 1
    assert b"NULL" in lib.fl_last_error()
    assert lib.fl_lse_fwd_f32_noalloc(None, None, -1, 4, 1, None) == 1
    assert b"negative shape" in lib.fl_last_error()
    assert lib.fl_lse_fwd_f32_noalloc(None, None, 3, 4, 1, None) == 1
    assert b"out is NULL" in lib.fl_last_error()
    # the read-ceiling kernel refuses a NULL buffer before building a resource
    # over it (the sink pointer is only checked for NULL on the host)
    diag = _lib.load_diag()
    assert diag.fl_diag_read_stream(None, 256, 4, 64, 2, ctypes.c_void_p(256), None) == 1
    assert b"x is NULL" in lib.fl_last_error()
    assert diag.fl_diag_fwd_block_times(None, None, 512, 4, None, None) == 1
    assert diag.fl_diag_intlse_phases(3, None, None, 1, 1, None, None) == 1
    assert b"kind" in lib.fl_last_error()
    assert diag.fl_diag_half_rows_cap(0, None, None, 4, 8, 9, None) == 1
    assert b"cap" in lib.fl_last_error()
    assert diag.fl_diag_lane_pairs(None, None, None) == 1
    assert b"NULL" in lib.fl_last_error()
    assert diag.fl_diag_gather_rows(None, None, None, 4, 8, 16, 1, 0, None) == 1
    assert b"NULL" in lib.fl_last_error()
    vp = ctypes.c_void_p(256)
    assert diag.fl_diag_gather_rows(vp, vp, vp, 4, 6, 16, 1, 0, None) == 1
    assert b"16-byte" in lib.fl_last_error()
    assert diag.fl_diag_gather_rows(None, None, None, 4, 8, 8, 1, 0, None) == 1
    assert b"lanes_per_row" in lib.fl_last_error()
    assert diag.fl_diag_gather_rows(vp, vp, vp, 4, 8, 16, 2, 0, None) == 1
    assert b"waves" in lib.fl_last_error()
    assert diag.fl_diag_gather_rows(vp, vp, vp, 4, 8, 16, 1, 3, None) == 1
    assert b"policy" in lib.fl_last_error()
    assert diag.fl_diag_blocked_bwd_pattern(None, None, None, None, None, None, 2, 64, 1, 0, None) == 1
    assert b"NULL" in lib.fl_last_error()
    assert diag.fl_diag_blocked_bwd_pattern(vp, vp, vp, vp, vp, vp, 2, 100, 1, 0, None) == 1
    assert b"multiple of 64" in lib.fl_last_error()
    assert diag.fl_diag_blocked_bwd_pattern(vp, vp, vp, vp, vp, vp, 2, 64, 3, 0, None) == 1
    assert b"waves" in lib.fl_last_error()
    assert diag.fl_diag_blocked_bwd_pattern(vp, vp, vp, vp, vp, vp, 2, 64, 4, 40961, None) == 1
    assert b"lds_per_wave" in lib.fl_last_error()
    assert diag.fl_diag_blocked_bwd_pattern(None, None, None, None, None, None, 0, 64, 1, 0, None) == 0
    # B == 0 is a no-op success
    assert lib.fl_lse_fwd_f32_noalloc(None, None, 0, 4, 1, None) == 0
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


def test_split_workspace_plan():
    """fl_lse_fwd_workspace_bytes: zero where the one-pass kernels cover the
    shape (many rows, or rows of at most 4096 vectors), otherwise one
    (max, sum) pair of fp32 per row segment, 2..64 segments per row."""
    lib = _lib.load()
    ws = lib.fl_lse_fwd_workspace_bytes
    assert ws(512, 128256, 4) == 0          # C2: one block per row fills the GPU
    assert ws(4096, 128256, 4) == 0
    assert ws(320, 128256, 4) == 0          # enough rows for one block per row
    assert ws(319, 128256, 4) > 0
    assert ws(257, 128256, 4) > 0           # a partial second round of one-pass blocks
    for B in (192, 200, 256):               # at most one one-pass block per CU
        assert ws(B, 128256, 4) == 0, B
    assert ws(191, 128256, 4) > 0
    assert ws(64, 16384, 4) == 0            # 4096 vectors: one-pass
    assert ws(64, 32768, 2) == 0            # 4096 half vectors
    assert ws(64, 128256, 3) == 0           # unsupported element size
    assert ws(0, 128256, 4) == 0
    for B, N, eb in [(1, 128256, 4), (64, 128256, 4), (1, 300001, 2), (7, 300001, 2)]:
        n = ws(B, N, eb)
        assert n > 0 and n % (8 * B) == 0
        S = n // (8 * B)
        assert 2 <= S <= 64, (B, N, S)


def test_split_entry_rejects_small_workspace_without_launch():
    lib = _lib.load()
    fake = ctypes.c_void_p(1 << 40)  # never dereferenced: the size check comes first
    need = lib.fl_lse_fwd_workspace_bytes(8, 128256, 4)
    assert need > 0
    assert lib.fl_lse_fwd_f32_ws(fake, fake, 8, 128256, 1, fake, need - 1, None) == 1
    assert b"workspace of" in lib.fl_last_error()
    unaligned = ctypes.c_void_p((1 << 40) + 4)
    assert lib.fl_lse_fwd_f32_ws(fake, fake, 8, 128256, 1, unaligned, need, None) == 1
    assert b"8-byte aligned" in lib.fl_last_error()


class _OnGpu(torch.Tensor):
    """A CPU tensor that reports itself CUDA on device `_idx` (set per
    subclass), so the shim's checks run without a GPU."""
    _idx = 0

    @property
    def is_cuda(self):
        return True

    @property
    def device(self):
        return torch.device("cuda", self._idx)


class _OnGpu1(_OnGpu):
    _idx = 1


def _gpu(t, idx=0):
    return t.as_subclass(_OnGpu1 if idx else _OnGpu)


@pytest.mark.parametrize("fn,make,msg", [
    ("onepass_lse_float_backward",
     lambda: (_gpu(torch.zeros(2), 1), _gpu(torch.zeros(2, 3)), _gpu(torch.zeros(2))),
     "grad_output must be on the same device as x"),
    ("onepass_lse_float_backward",
     lambda: (_gpu(torch.zeros(2)), _gpu(torch.zeros(2, 3)), _gpu(torch.zeros(2), 1)),
     "lse_output must be on the same device as x"),
    ("onepass_lse_half_backward",
     lambda: (_gpu(torch.zeros(2)), _gpu(torch.zeros(2, 3, dtype=torch.float16)), _gpu(torch.zeros(2), 1)),
     "lse_output must be on the same device as x"),
    ("selective_log_softmax_float",
     lambda: (_gpu(torch.zeros(2, 3)), _gpu(torch.zeros(2, dtype=torch.int64), 1)),
     "index must be on the same device as logits"),
    ("selective_log_softmax_float_backward",
     lambda: (_gpu(torch.zeros(2)), _gpu(torch.zeros(2, 3)), _gpu(torch.zeros(2, dtype=torch.int64)),
              _gpu(torch.zeros(2), 1)),
     "lse must be on the same device as logits"),
    ("sparse_csr_forward",
     lambda: (_gpu(torch.zeros(4, 8)), _gpu(torch.tensor([0, 1], dtype=torch.int64), 1),
              _gpu(torch.zeros(1, dtype=torch.int32)), _gpu(torch.zeros(1))),
     "offsets must be on the same device as child"),
])
def test_shim_rejects_operands_on_another_gpu(fn, make, msg):
    """Every operand of a multi-tensor entry must live on the launching GPU:
    the check raises before any launch (a pointer into another GPU's memory
    is not an operand of the kernel)."""
    import fuselse_amd

    with pytest.raises(RuntimeError, match=msg):
        getattr(fuselse_amd.ext, fn)(*make())
