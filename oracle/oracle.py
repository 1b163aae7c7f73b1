"""TEST INFRASTRUCTURE ONLY: CPU oracle for the log-sum-exp hot path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or as the timed CPU
baseline).  The shipped package never imports it.

Two kinds of oracle live here:

* fp64 numpy restatements of the float paths (forward, robust forward,
  backward, selective log-softmax forward and backward, sparse gather-LSE).  They follow the mathematics the reference
  implements (``fuselse/gpu/fused_fp32_kernel.cu:27-40,135-150``,
  ``experiment_pyjuice/run_pyjuice.py:103-118``) and torch.logsumexp's
  special-value rules, which the reference's robust variant reproduces.
* ctypes bindings of ``oracle/lse_oracle.c``, the integer restatements
  (Q16.16 / Q10.6 pair ops, GPU reduction trees, CPU AVX2 block tree, sparse
  Q16 ET tree) and the FuseLSE-CPU chain used as the CPU baseline.

``ref_intlse_cpu_rows`` calls the reference's own ``intlse/cpu/lse_kernel_simd.c``
compiled into ``oracle/_ref`` (when it was built), and ``ref_fuselse_cpu`` its
``fuselse/cpu/fused_fp32_cpu.cpp``; both pin the restatements.
"""

from __future__ import annotations

import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(HERE, "liblse_oracle.so")
_REF_PATH = os.path.join(HERE, "_ref", "liblse_kernel_simd.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i16p = ctypes.POINTER(ctypes.c_int16)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_lib = None
_ref = None

GPU_NEG_INF = -0x3FFFFFFF
Q16_CONV = np.float32(np.float32(1.44269504089) * np.float32(65536.0))  # 94548.4609375
Q16_OUT = np.float32(np.float32(0.69314718056) / np.float32(65536.0))
Q10_OUT = np.float32(np.float32(0.69314718056) / np.float32(64.0))


def lib():
    """Load oracle/liblse_oracle.so (built by ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        L.or_q16_pair.restype = ctypes.c_int32
        L.or_q16_pair.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int]
        L.or_q16_pair_x86.restype = ctypes.c_int32
        L.or_q16_pair_x86.argtypes = [ctypes.c_int32, ctypes.c_int32]
        L.or_q10_6_pair.restype = ctypes.c_int32
        L.or_q10_6_pair.argtypes = [ctypes.c_int32, ctypes.c_int32]
        L.or_lut_q16.restype = ctypes.c_int32
        L.or_lut_q10_6.restype = ctypes.c_int32
        L.or_q16_pair_batch.argtypes = [_i32p, _i32p, _i64, ctypes.c_int, _i32p]
        L.or_q10_6_pair_batch.argtypes = [_i32p, _i32p, _i64, _i32p]
        L.or_q16_quant_batch.argtypes = [_f32p, _i64, ctypes.c_int, _i32p]
        L.or_intlse_cpu_rows.argtypes = [_f32p, _i64, _i64, ctypes.c_int, _f32p]
        L.or_q16_gpu_rows.argtypes = [ctypes.c_void_p, ctypes.c_int, _i64, _i64, ctypes.c_int,
                                      ctypes.c_int, _f32p, _i32p]
        L.or_q10_6_rows.argtypes = [_i16p, _i64, _i64, ctypes.c_int, _f32p, _i32p]
        L.or_to_q10_6.argtypes = [_f32p, _i64, _i16p]
        L.or_to_q16.argtypes = [_f32p, _i64, _i32p]
        L.or_edge_threads.restype = ctypes.c_int
        L.or_edge_threads.argtypes = [_i64]
        L.or_sparse_q16_csr.argtypes = [_f32p, _i64p, _i32p, _f32p, _i64, _i64, _f32p]
        L.or_sparse_q16_blocked.argtypes = [_f32p, _f32p, _f32p, _i64p, _i64p, _i64, _i64, _i64, _i64]
        L.or_fuselse_cpu_rows.argtypes = [_f32p, _i64, _i64, _f32p]
        L.or_lse_backward_rows.argtypes = [_f32p, _f32p, _f32p, _i64, _i64, _f32p]
        L.or_omp_max_threads.restype = ctypes.c_int
        L.or_omp_set_threads.argtypes = [ctypes.c_int]
        L.or_omp_set_threads.restype = None
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(_REF_PATH)


def ref():
    """The reference's CPU IntLSE compiled from its own source (oracle/_ref)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference build missing: {_REF_PATH}")
        R = ctypes.CDLL(_REF_PATH)
        for name in ("lse_q16_1d_simd", "lse_q16_1d_simd_neg_inf"):
            fn = getattr(R, name)
            fn.restype = ctypes.c_float
            fn.argtypes = [_f32p, ctypes.c_int]
        for name in ("lse_q16_2d_simd", "lse_q16_2d_simd_neg_inf"):
            fn = getattr(R, name)
            fn.restype = None
            fn.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, _f32p]
        _ref = R
    return _ref


_REF_FUSE_PATH = os.path.join(HERE, "_ref", "fused_fp32_cpu.so")
_ref_fuse = None


def ref_fuselse_available() -> bool:
    return os.path.exists(_REF_FUSE_PATH)


def ref_fuselse_cpu(x) -> np.ndarray:
    """The reference's FuseLSE-CPU (fuselse/cpu/fused_fp32_cpu.cpp:28-46)
    compiled from its own source into oracle/_ref by oracle/Makefile: its
    cpu_lse_float over rows of a 2-D fp32 array.  Present only where the
    reference tree is mounted; used to write tests/golden fixtures and to
    check the C port."""
    global _ref_fuse
    if _ref_fuse is None:
        import importlib.util

        import torch  # noqa: F401  (the module links libtorch)

        if not ref_fuselse_available():
            raise RuntimeError(f"reference build missing: {_REF_FUSE_PATH}")
        spec = importlib.util.spec_from_file_location("fused_fp32_cpu", _REF_FUSE_PATH)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _ref_fuse = mod
    import torch

    x = np.ascontiguousarray(x, np.float32)
    return _ref_fuse.cpu_lse_float(torch.from_numpy(x)).numpy()


def _p(a, t):
    return a.ctypes.data_as(t)


# ----------------------------------------------------------------------------
# fp64 float oracles
# ----------------------------------------------------------------------------
def lse_fp64(x) -> np.ndarray:
    """Row LSE over the last axis in float64 with torch.logsumexp's special
    values: all -inf -> -inf, any +inf (no NaN) -> +inf, any NaN -> NaN.
    This is what the reference's robust pair (fused_fp32_kernel.cu:34-40)
    yields row-wise."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        m = np.max(np.where(np.isnan(x), -np.inf, x), axis=-1, keepdims=True)
        m_use = np.where(np.isinf(m), 0.0, m)
        s = np.sum(np.exp(x - m_use), axis=-1, keepdims=True)
        out = (m_use + np.log(s))[..., 0]
    return out


def lse_bwd_fp64(g, x, lse) -> np.ndarray:
    """grad_in = g[r] * exp(x[r, i] - lse[r]) (fused_fp32_kernel.cu:135-150)."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        return np.asarray(g, np.float64)[..., None] * np.exp(x - np.asarray(lse, np.float64)[..., None])


def selective_logsoftmax_fp64(x, index):
    """Selective log-softmax in float64: logp[r] = x[r, index[r]] - LSE(x[r, :]),
    NaN for an index outside [0, N).  This is the fp32 branch of
    trl.trainer.utils.selective_log_softmax (trl 1.0.0, a dependency absent
    here; its published algorithm is gather, per-row torch.logsumexp,
    subtraction), which experiment_rlhf_logsumexp/run_rlhf.py:145,155 times.
    Returns (logp, lse)."""
    x = np.asarray(x, np.float64)
    idx = np.asarray(index, np.int64)
    lse = lse_fp64(x)
    ok = (idx >= 0) & (idx < x.shape[-1])
    xt = np.take_along_axis(x, np.where(ok, idx, 0)[..., None], axis=-1)[..., 0]
    with np.errstate(invalid="ignore"):
        return np.where(ok, xt - lse, np.nan), lse


def selective_logsoftmax_bwd_fp64(g, x, index, lse):
    """d logp[r] / d x[r, i] times g[r]: g[r] * ((i == index[r]) - exp(x[r, i] - lse[r]))."""
    x = np.asarray(x, np.float64)
    g = np.asarray(g, np.float64)
    out = -lse_bwd_fp64(g, x, lse)
    idx = np.asarray(index, np.int64)
    rows = np.nonzero((idx >= 0) & (idx < x.shape[-1]))[0]
    out[rows, idx[rows]] += g[rows]
    return out


def sparse_csr_bwd_fp64(child, out, gout, offsets, child_ids, logp):
    """Flows of the CSR sum layer in float64: term[e, b] = gout[n_e, b] *
    exp(logp[e] + child[c_e, b] - out[n_e, b]) (0 where out is -inf);
    returns (grad_child, grad_logp) = (per-child sum of terms, per-edge sum
    over b).  The reference has no sparse backward; this is the derivative
    of its forward (sparse_float_kernel.cu:40-105), pyjuice's element and
    parameter flows."""
    child = np.asarray(child, np.float64)
    out = np.asarray(out, np.float64)
    gout = np.asarray(gout, np.float64)
    off = np.asarray(offsets, np.int64)
    cid = np.asarray(child_ids, np.int64)
    lw = np.asarray(logp, np.float64)
    node = np.repeat(np.arange(len(off) - 1), np.diff(off))
    with np.errstate(invalid="ignore", over="ignore"):
        term = gout[node] * np.exp(lw[:, None] + child[cid] - out[node])
    term[np.isneginf(out[node])] = 0.0
    gchild = np.zeros_like(child)
    np.add.at(gchild, cid, term)
    return gchild, term.sum(axis=1)


def sparse_blocked_fp64(element_mars, params, nids, cids, pids, block_size, clamp=1e-45):
    """pyjuice block-layout weighted gather-LSE in fp64
    (sparse_float_kernel.cu:40-105; torch form run_pyjuice.py:103-118):
    out[(nids[j]+p), b] = LSE_e(log max(params[pids[j,e]+p], clamp) + element_mars[cids[j,e], b]).
    Returns (rows, values) with rows the written node ids."""
    em = np.asarray(element_mars, np.float64)
    params = np.asarray(params, np.float64)
    nb, ne = cids.shape
    rows, vals = [], []
    for j in range(nb):
        for p in range(block_size):
            lw = np.log(np.maximum(params[pids[j] + p], clamp))
            logits = em[cids[j]] + lw[:, None]  # (E, batch)
            rows.append(int(nids[j]) + p)
            vals.append(lse_fp64(logits.T))
    return np.array(rows, np.int64), np.array(vals)


def sparse_blocked_bwd_fp64(node_flows, node_mars, element_mars, params, nids, cids, pids, block_size, clamp=1e-45,
                            params_are_log=False):
    """Flows of the block-layout sum layer in float64, by loops over blocks,
    positions and edges: for block j, position p, edge e with n = nids[j]+p,
    c = cids[j,e], q = pids[j,e]+p and lw = log max(params[q], clamp) (params[q]
    when params_are_log): term[b] = node_flows[n,b] * exp(lw + em[c,b] -
    node_mars[n,b]) (0 where node_mars is -inf).  Returns the increments
    (element_flows [nelem, batch], param_flows [nparams]).  The reference has no
    sparse backward; this is the derivative of its block-layout forward
    (sparse_float_kernel.cu:40-105, pyjuice's element and parameter flows)."""
    nf = np.asarray(node_flows, np.float64)
    nm = np.asarray(node_mars, np.float64)
    em = np.asarray(element_mars, np.float64)
    params = np.asarray(params, np.float64).reshape(-1)
    nb, ne = cids.shape
    def_el = np.zeros_like(em)
    def_par = np.zeros_like(params)
    for j in range(nb):
        for p in range(block_size):
            n = int(nids[j]) + p
            live = ~np.isneginf(nm[n])
            for e in range(ne):
                c = int(cids[j, e])
                q = int(pids[j, e]) + p
                lw = params[q] if params_are_log else np.log(max(params[q], clamp))
                with np.errstate(invalid="ignore", over="ignore"):
                    t = np.where(live, nf[n] * np.exp(lw + em[c] - np.where(live, nm[n], 0.0)), 0.0)
                def_el[c] += t
                def_par[q] += t.sum()
    return def_el, def_par


def sparse_csr_fp64(child, offsets, cids, logparam):
    """CSR gather-LSE in fp64: out[n, b] = LSE_{e in node n}(logparam[e] + child[cid[e], b])."""
    child = np.asarray(child, np.float64)
    offsets = np.asarray(offsets, np.int64)
    n = len(offsets) - 1
    out = np.empty((n, child.shape[1]))
    for i in range(n):
        e0, e1 = offsets[i], offsets[i + 1]
        logits = child[cids[e0:e1]] + np.asarray(logparam[e0:e1], np.float64)[:, None]
        out[i] = lse_fp64(logits.T) if e1 > e0 else -np.inf
    return out


# ----------------------------------------------------------------------------
# integer oracles (C)
# ----------------------------------------------------------------------------
def q16_pair(a, b, mode="gpu"):
    """Elementwise Q16.16 pair LSE. mode: 'gpu' (LUT), 'nolut', 'x86'."""
    a = np.ascontiguousarray(a, np.int32)
    b = np.ascontiguousarray(b, np.int32)
    out = np.empty_like(a)
    lib().or_q16_pair_batch(_p(a, _i32p), _p(b, _i32p), a.size, {"gpu": 0, "nolut": 1, "x86": 2}[mode],
                            _p(out, _i32p))
    return out


def q10_6_pair(a, b):
    a = np.ascontiguousarray(a, np.int32)
    b = np.ascontiguousarray(b, np.int32)
    out = np.empty_like(a)
    lib().or_q10_6_pair_batch(_p(a, _i32p), _p(b, _i32p), a.size, _p(out, _i32p))
    return out


def q16_quant(x, mode="gpu"):
    """Q16.16 quantisers: 'gpu' (__float2int_rn(v*CONV)), 'sparse', 'cpu_scalar', 'cpu_simd'."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.int32)
    lib().or_q16_quant_batch(_p(x, _f32p), x.size, {"gpu": 0, "sparse": 1, "cpu_scalar": 2, "cpu_simd": 3}[mode],
                             _p(out, _i32p))
    return out


def lut_q16():
    return np.array([lib().or_lut_q16(i) for i in range(64)], np.int64)


def lut_q10_6():
    return np.array([lib().or_lut_q10_6(i) for i in range(64)], np.int64)


def to_q16(x) -> np.ndarray:
    """Q16.16 int32 input recipe: sat_int32(rne(fl32(x * 94548.4609375)))."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int32)
    lib().or_to_q16(_p(x, _f32p), x.size, _p(q, _i32p))
    return q


def to_q10_6(x) -> np.ndarray:
    """Reduced-bit harness quantiser (reduced_bit/run_bench.py:50-53,100-103)."""
    x = np.ascontiguousarray(x, np.float32)
    q = np.empty(x.shape, np.int16)
    lib().or_to_q10_6(_p(x, _f32p), x.size, _p(q, _i16p))
    return q


def q16_gpu_rows(x, base_mod=0, use_lut=True, raw=False):
    """GPU IntLSE tree (lse_kernel.cu:67-159) over rows of a 2-D fp32 or int32
    array. base_mod: byte address of row 0 modulo 16 on the device."""
    x = np.ascontiguousarray(x)
    assert x.ndim == 2 and x.dtype in (np.float32, np.int32)
    B, N = x.shape
    out = np.empty(B, np.float32)
    r = np.empty(B, np.int32)
    lib().or_q16_gpu_rows(x.ctypes.data, int(x.dtype == np.int32), B, N, int(base_mod) & 15, int(use_lut),
                          _p(out, _f32p), _p(r, _i32p))
    return (out, r) if raw else out


def q10_6_rows(q, base_mod=0, raw=False):
    """GPU Q10.6 tree (lse_kernel_q10_6.cu:55-139) over rows of a 2-D int16 array."""
    q = np.ascontiguousarray(q, np.int16)
    B, N = q.shape
    out = np.empty(B, np.float32)
    r = np.empty(B, np.int32)
    lib().or_q10_6_rows(_p(q, _i16p), B, N, int(base_mod) & 7, _p(out, _f32p), _p(r, _i32p))
    return (out, r) if raw else out


def intlse_cpu_rows(x, neg_inf_variant=False):
    """Restatement of the CPU IntLSE AVX2 rows (lse_kernel_simd.c:164-315)."""
    x = np.ascontiguousarray(x, np.float32)
    B, N = x.shape
    out = np.empty(B, np.float32)
    lib().or_intlse_cpu_rows(_p(x, _f32p), B, N, int(neg_inf_variant), _p(out, _f32p))
    return out


def ref_intlse_cpu_rows(x, neg_inf_variant=False):
    """The reference's compiled CPU IntLSE (oracle/_ref) on the same rows."""
    x = np.ascontiguousarray(x, np.float32)
    B, N = x.shape
    out = np.empty(B, np.float32)
    fn = ref().lse_q16_2d_simd_neg_inf if neg_inf_variant else ref().lse_q16_2d_simd
    fn(_p(x, _f32p), B, N, _p(out, _f32p))
    return out


def edge_threads(fan_in: int) -> int:
    return lib().or_edge_threads(int(fan_in))


def sparse_q16_csr(child, offsets, cids, logparam):
    child = np.ascontiguousarray(child, np.float32)
    offsets = np.ascontiguousarray(offsets, np.int64)
    cids = np.ascontiguousarray(cids, np.int32)
    logparam = np.ascontiguousarray(logparam, np.float32)
    n = len(offsets) - 1
    out = np.empty((n, child.shape[1]), np.float32)
    lib().or_sparse_q16_csr(_p(child, _f32p), _p(offsets, _i64p), _p(cids, _i32p), _p(logparam, _f32p), n,
                            child.shape[1], _p(out, _f32p))
    return out


def sparse_q16_blocked(node_mars, element_mars, logw, nids, cids, block_size):
    """In-place on a copy of node_mars; logw has shape (num_nblocks, block_size, num_edges)."""
    node_mars = np.array(node_mars, np.float32, copy=True, order="C")
    element_mars = np.ascontiguousarray(element_mars, np.float32)
    logw = np.ascontiguousarray(logw, np.float32)
    nids = np.ascontiguousarray(nids, np.int64)
    cids = np.ascontiguousarray(cids, np.int64)
    nb, ne = cids.shape
    lib().or_sparse_q16_blocked(_p(node_mars, _f32p), _p(element_mars, _f32p), _p(logw, _f32p), _p(nids, _i64p),
                                _p(cids, _i64p), nb, ne, block_size, node_mars.shape[1])
    return node_mars


def fuselse_cpu_rows(x):
    """FuseLSE-CPU sequential pair chain (fused_fp32_cpu.cpp:22-46), OpenMP rows."""
    x = np.ascontiguousarray(x, np.float32)
    B, N = x.shape
    if N < 1:
        raise ValueError("FuseLSE-CPU needs N >= 1")
    out = np.empty(B, np.float32)
    lib().or_fuselse_cpu_rows(_p(x, _f32p), B, N, _p(out, _f32p))
    return out


def lse_backward_rows(g, x, lse):
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(g, np.float32)
    lse = np.ascontiguousarray(lse, np.float32)
    B, N = x.shape
    gx = np.empty_like(x)
    lib().or_lse_backward_rows(_p(g, _f32p), _p(x, _f32p), _p(lse, _f32p), B, N, _p(gx, _f32p))
    return gx


def omp_threads() -> int:
    return lib().or_omp_max_threads()


def set_omp_threads(n: int) -> None:
    """Threads of the C port's OpenMP loops (the CPU baseline's 1-thread runs)."""
    lib().or_omp_set_threads(int(n))


# ----------------------------------------------------------------------------
# workload recipes shared by tests and bench (the benchmark configs)
# ----------------------------------------------------------------------------
def make_c2_input(B=512, N=128256, seed=0, spike_frac=0.001, spike=15.0):
    """fp32 logits x ~ N(0, 3^2) with spike_frac of entries set to +15."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, N), dtype=np.float32) * np.float32(3.0))
    n_spk = int(round(spike_frac * B * N))
    if n_spk:
        idx = rng.choice(B * N, size=n_spk, replace=False)
        x.reshape(-1)[idx] = np.float32(spike)
    return x


def make_robust_rows(x, seed=1):
    """Special-value rows of the robust set: 1% of rows get 10% -inf entries;
    row 0 all -inf; row 1 one +inf; row 2 one NaN; row 3 one +inf and one -inf."""
    rng = np.random.default_rng(seed)
    x = np.array(x, copy=True)
    B, N = x.shape
    k = max(1, B // 100)
    rows = rng.choice(np.arange(4, B), size=min(k, max(B - 4, 0)), replace=False) if B > 4 else []
    for r in rows:
        cols = rng.choice(N, size=max(1, N // 10), replace=False)
        x[r, cols] = -np.inf
    if B > 0:
        x[0, :] = -np.inf
    if B > 1:
        x[1, rng.integers(N)] = np.inf
    if B > 2:
        x[2, rng.integers(N)] = np.nan
    if B > 3 and N > 1:
        c = rng.choice(N, size=2, replace=False)
        x[3, c[0]] = np.inf
        x[3, c[1]] = -np.inf
    return x


def powerlaw_fanin(num_nodes, alpha=2.0, lo=2, hi=256, seed=0):
    """Fan-in k ~ p(k) proportional to k^-alpha on [lo, hi]."""
    rng = np.random.default_rng(seed)
    ks = np.arange(lo, hi + 1)
    p = ks.astype(np.float64) ** (-alpha)
    p /= p.sum()
    return rng.choice(ks, size=num_nodes, p=p).astype(np.int64)


def fp64_lse_ref(x_fp32) -> np.ndarray:
    """fp64 ground truth m + log(sum(exp(x - m))) (run_microbenchmark.py:141-146)."""
    x = np.asarray(x_fp32, np.float64)
    m = x.max(axis=-1, keepdims=True)
    return (m + np.log(np.exp(x - m).sum(axis=-1, keepdims=True)))[..., 0]


LN2 = math.log(2.0)


# ----------------------------------------------------------------------------
# The reference's CPU wrappers around the AVX2 IntLSE (test infrastructure:
# their dispatch and special-value handling, restated over either the C
# restatement of the kernel or the compiled reference in oracle/_ref).
# ----------------------------------------------------------------------------
def _cpu_rows(backend):
    return ref_intlse_cpu_rows if backend == "ref" else intlse_cpu_rows


def logsumexp_intlse(a, axis=None, keepdims=False, backend="port"):
    """lse_ctypes_wrapper.py:99-125: a NaN or +inf anywhere sends the whole call
    to np.logaddexp.reduce; otherwise the -inf-identity kernel variant runs
    over the flattened array (axis=None) or the last axis (1-D -> float,
    2-D -> float32[B], higher ranks flattened to rows); other axes raise
    NotImplementedError.  As in the reference, keepdims is ignored by the
    finite full reduction (axis=None returns a float)."""
    a = np.asarray(a, dtype=np.float32)
    rows_fn = _cpu_rows(backend)
    maximum = np.max(a) if a.size else -np.inf
    if np.isnan(maximum) or np.isposinf(maximum):
        if axis is None:
            result = np.logaddexp.reduce(a.ravel())
            if keepdims:
                return np.full((1,) * a.ndim, result, dtype=np.float32)
            return result
        return np.logaddexp.reduce(a, axis=axis, keepdims=keepdims)

    def one(v):  # lse_intlse_simd_neg_inf: a 1-D row -> Python float
        return float(rows_fn(np.ascontiguousarray(v, np.float32)[None, :], True)[0])

    if axis is None:
        return one(a.ravel())
    if axis == -1 or axis == a.ndim - 1:
        if a.ndim == 1:
            r = one(a)
            return r if not keepdims else np.array([r], dtype=np.float32)
        if a.ndim == 2:
            r = rows_fn(a, True)
            return r if not keepdims else r[..., None]
        r = rows_fn(a.reshape(-1, a.shape[-1]), True)
        out = r.reshape(a.shape[:-1])
        return out if not keepdims else out[..., None]
    raise NotImplementedError(f"axis={axis} not yet supported")


def logsumexp_intlse_torch(input_tensor, dim=-1, keepdim=False, backend="port"):
    """torch_wrapper.py:9-29: CPU fp32 tensors reduced over the last dimension
    (N >= 2, no grad) go through logsumexp_intlse; everything else to
    torch.logsumexp."""
    import torch

    normalized_dim = dim if dim >= 0 else input_tensor.dim() + dim
    supported = (input_tensor.device.type == "cpu" and input_tensor.dtype == torch.float32
                 and normalized_dim == input_tensor.dim() - 1 and input_tensor.shape[-1] >= 2
                 and not input_tensor.requires_grad)
    if not supported:
        return torch.logsumexp(input_tensor, dim=dim, keepdim=keepdim)
    output = logsumexp_intlse(input_tensor.detach().contiguous().numpy(), axis=-1, keepdims=keepdim,
                              backend=backend)
    if isinstance(output, np.ndarray):
        return torch.from_numpy(output)
    return torch.tensor(output, dtype=input_tensor.dtype)
