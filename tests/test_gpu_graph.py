"""HIP-graph capture of the hot path: the entry points a training or
serving loop runs (fp32 robust forward and fused backward, fp16 forward and
backward, IntLSE Q16.16, the fused selective log-softmax forward and
backward, the sparse CSR forward and backward) captured into one graph and
replayed several times, with eager rewrites of the inputs and eager
synchronisations between replays; every replay is checked against the eager
results of the same inputs.  None of these launches records a memset."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


def _step(ext, t):
    """One pass over every captured entry point; returns its outputs."""
    lse = ext.onepass_lse_float_robust(t["x"])
    gx = ext.onepass_lse_float_backward(t["g"], t["x"], lse)
    lse16 = ext.batched_logsumexp_fp16(t["xh"], robust=True)
    gh = ext.onepass_lse_half_backward(t["g"], t["xh"], lse16)
    q16 = ext.batched_logsumexp(t["xq"])
    logp, slse = ext.selective_log_softmax_float(t["x"], t["idx"])
    gsel = ext.selective_log_softmax_float_backward(t["g"], t["x"], t["idx"], slse)
    out = ext.sparse_csr_forward(t["child"], t["off"], t["cid"], t["lp"])
    gc, gl = ext.sparse_csr_backward(t["child"], out, t["gout"], t["off"], t["cid"], t["lp"], t["csc"])
    return [lse, gx, lse16, gh, q16, logp, slse, gsel, out, gc, gl]


def _fill(t, rng, dev):
    """Rewrites every input in place (eager, outside the graph)."""
    B, N = t["x"].shape
    t["x"].copy_(torch.from_numpy((rng.standard_normal((B, N)) * 3).astype(np.float32)))
    t["g"].copy_(torch.from_numpy(rng.standard_normal(B).astype(np.float32)))
    t["xh"].copy_(torch.from_numpy((rng.standard_normal((B, N)) * 2).astype(np.float32)).half())
    t["xq"].copy_(torch.from_numpy((rng.random((B, N)) * -50).astype(np.float32)))
    t["idx"].copy_(torch.from_numpy(rng.integers(0, N, B)))
    t["child"].copy_(torch.from_numpy(np.log(rng.random(tuple(t["child"].shape)) + 1e-12).astype(np.float32)))
    t["gout"].copy_(torch.from_numpy(rng.standard_normal(tuple(t["gout"].shape)).astype(np.float32)))


def test_hot_path_in_a_hip_graph_replays(cuda):
    print("case hot path graph replays", flush=True)
    ext = _ext()
    rng = np.random.default_rng(5)
    B, N = 48, 20000                       # long rows: block geometry; B*N*4 = 3.8 MB
    nodes, nch, batch = 300, 200, 64
    fan = rng.integers(1, 20, nodes)
    off = np.concatenate([[0], np.cumsum(fan)]).astype(np.int64)
    t = {
        "x": torch.empty(B, N, device=cuda), "g": torch.empty(B, device=cuda),
        "xh": torch.empty(B, N, dtype=torch.float16, device=cuda), "xq": torch.empty(B, N, device=cuda),
        "idx": torch.empty(B, dtype=torch.int64, device=cuda),
        "child": torch.empty(nch, batch, device=cuda), "gout": torch.empty(nodes, batch, device=cuda),
        "off": torch.from_numpy(off).to(cuda),
        "cid": torch.from_numpy(rng.integers(0, nch, off[-1]).astype(np.int32)).to(cuda),
        "lp": torch.from_numpy((rng.standard_normal(off[-1]) - 2).astype(np.float32)).to(cuda),
    }
    t["csc"] = ext.sparse_csr_transpose(t["off"], t["cid"], nch)   # built once, outside the graph
    _fill(t, rng, cuda)
    _step(ext, t)                          # warm-up: library load, workspace sizes
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _step(ext, t)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = _step(ext, t)
    for rep in range(4):
        _fill(t, rng, cuda)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = _step(ext, t)               # eager, same inputs
        torch.cuda.synchronize()
        for k, (a, b) in enumerate(zip(outs, want)):
            assert torch.equal(a, b), (rep, k)
