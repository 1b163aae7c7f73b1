"""ctypes binding of the gfx950 C-ABI library (``libfuselse_amd.so``).

The library is loaded after ``import torch`` so it binds to the HIP runtime
torch already loaded (same soname), which makes torch's streams and device
pointers valid inside it.  A missing or unloadable library raises loudly:
there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libfuselse_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "fuselse_amd.h")
DIAG_LIB_PATH = os.path.join(PKG_DIR, "libfuselse_amd_diag.so")
DIAG_HEADER_PATH = os.path.join(os.path.dirname(PKG_DIR), "include", "fuselse_amd_diag.h")

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes); must match include/fuselse_amd.h
SIGNATURES = {
    "fl_last_error": (ctypes.c_char_p, []),
    "fl_abi_version": (_int, []),
    "fl_lse_fwd_f32": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_lse_bwd_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_lse_fwd_f16": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_lse_fwd_bf16": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_lse_fwd_f32_keep": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_lse_fwd_f16_keep": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_lse_fwd_bf16_keep": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_selective_logsoftmax_f32": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _int, _vp, ctypes.c_size_t, _vp]),
    "fl_selective_logsoftmax_bwd_f32": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_lse_bwd_f16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_lse_bwd_bf16": (_int, [_vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_lse_fwd_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _int]),
    "fl_lse_fwd_f32_ws": (_int, [_vp, _vp, _i64, _i64, _int, _vp, ctypes.c_size_t, _vp]),
    "fl_lse_fwd_f16_ws": (_int, [_vp, _vp, _i64, _i64, _int, _vp, ctypes.c_size_t, _vp]),
    "fl_lse_fwd_bf16_ws": (_int, [_vp, _vp, _i64, _i64, _int, _vp, ctypes.c_size_t, _vp]),
    "fl_lse_fwd_f32_noalloc": (_int, [_vp, _vp, _i64, _i64, _int, _vp]),
    "fl_intlse_q16_f32": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _vp]),
    "fl_intlse_q16_i32": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _vp]),
    "fl_intlse_q10_6": (_int, [_vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_sparse_csr_fwd": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _int, _vp]),
    "fl_sparse_csr_bwd": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp]),
    "fl_sparse_blocked_fwd": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp]),
    "fl_sparse_blocked_bwd": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp, _vp,
                                     _i64, _vp, _vp, _vp, _vp]),
}

# the measurement library (include/fuselse_amd_diag.h)
DIAG_SIGNATURES = {
    "fl_diag_read_stream": (_int, [_vp, _i64, _int, _int, _int, _vp, _vp]),
    "fl_diag_copy_stream": (_int, [_vp, _vp, _i64, _int, _int, _int, _vp]),
    "fl_diag_chain_latency": (_int, [_int, _int, _int, _vp, _vp]),
    "fl_diag_fwd_block_times": (_int, [_vp, _vp, _i64, _i64, _vp, _vp]),
    "fl_diag_read_rows_times": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "fl_diag_read_stream_times": (_int, [_vp, _i64, _int, _vp, _vp, _vp]),
    "fl_diag_intlse_phases": (_int, [_int, _vp, _vp, _i64, _i64, _vp, _vp]),
    "fl_diag_half_rows_cap": (_int, [_int, _vp, _vp, _i64, _i64, _int, _vp]),
    "fl_diag_lane_pairs": (_int, [_vp, _vp, _vp]),
    "fl_diag_gather_rows": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _int, _int, _vp]),
    "fl_diag_blocked_bwd_pattern": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _vp]),
}

_lib = None
_diag = None


class NativeLibraryMissing(RuntimeError):
    pass


def header_symbols(path: str = HEADER_PATH):
    """Function names declared in the C header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fl_[a-z0-9_]+)\s*\(", text)))


def load():
    """Load and type the library once; raises NativeLibraryMissing if absent."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (binds the HIP runtime torch ships before ours)

    if not os.path.exists(LIB_PATH):
        raise NativeLibraryMissing(
            f"fuselse_amd: native library {LIB_PATH} is not built; run "
            "`python -c 'import __graft_entry__ as g; g.build()'` (no CPU fallback exists)")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as e:
        raise NativeLibraryMissing(f"fuselse_amd: cannot load {LIB_PATH}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def load_diag():
    """Load and type the measurement library once (it loads the main library
    first, whose error state it shares)."""
    global _diag
    if _diag is not None:
        return _diag
    load()
    if not os.path.exists(DIAG_LIB_PATH):
        raise NativeLibraryMissing(f"fuselse_amd: measurement library {DIAG_LIB_PATH} is not built")
    try:
        lib = ctypes.CDLL(DIAG_LIB_PATH)
    except OSError as e:
        raise NativeLibraryMissing(f"fuselse_amd: cannot load {DIAG_LIB_PATH}: {e}") from e
    for name, (res, args) in DIAG_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _diag = lib
    return lib


def diag_call(name: str, *args) -> None:
    """call() for an entry point of the measurement library."""
    rc = getattr(load_diag(), name)(*args)
    if rc != 0:
        msg = load().fl_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with status {rc}")


_bound = {}


def call(name: str, *args) -> None:
    """Call entry point `name`; a nonzero status raises RuntimeError with the
    library's message.  Entry points are looked up once and kept, since the
    Python side of a call is the floor of small launches."""
    fn = _bound.get(name)
    if fn is None:
        fn = _bound[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        msg = load().fl_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"{name} failed with status {rc}")
