"""Builds the gfx950 C-ABI libraries in-tree.

* ``fuselse_amd/libfuselse_amd.so``: every HIP source directly under
  ``fuselse_amd/csrc``, compiled with hipcc for gfx950 and linked into one
  shared library exporting the entry points declared in
  ``include/fuselse_amd.h``.  It links only the HIP runtime; it has no torch
  or Python dependency.
* ``fuselse_amd/libfuselse_amd_diag.so``: the measurement kernels under
  ``fuselse_amd/csrc/diag`` (``include/fuselse_amd_diag.h``), linked against
  the first library, whose status and error functions it uses.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_obj")
LIB_PATH = os.path.join(PKG_DIR, "libfuselse_amd.so")
DIAG_DIR = os.path.join(CSRC, "diag")
DIAG_LIB_PATH = os.path.join(PKG_DIR, "libfuselse_amd_diag.so")
ARCH = os.environ.get("FUSELSE_AMD_ARCH", "gfx950")

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    f"--offload-arch={ARCH}",
    # keep hipcc from forming packed fp32 instructions (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO_DIR, "include"),
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def sources(directory=CSRC):
    out = []
    for name in sorted(os.listdir(directory)):
        if name.endswith((".hip", ".cpp")):
            out.append(os.path.join(directory, name))
    return out


def _compile(src: str, verbose: bool) -> str:
    sub = "diag_" if os.path.dirname(src) == DIAG_DIR else ""
    obj = os.path.join(OBJ_DIR, sub + os.path.basename(src) + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (r.stdout + r.stderr).splitlines() if noise not in ln and ln.strip()]
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(msgs))
    if msgs and verbose:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(objs, out_path, extra, verbose):
    tmp = out_path + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, *extra, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, out_path)


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compile every source, link libfuselse_amd.so and libfuselse_amd_diag.so;
    returns the first library's path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    diag_srcs = sources(DIAG_DIR)
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs) + len(diag_srcs)))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs + diag_srcs))
    _link(objs[:len(srcs)], LIB_PATH, [], verbose)
    _link(objs[len(srcs):], DIAG_LIB_PATH, [f"-L{PKG_DIR}", "-lfuselse_amd", "-Wl,-rpath,$ORIGIN"], verbose)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
