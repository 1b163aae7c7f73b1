"""The C5 sparse sum layer at the size the benchmark times (1M nodes,
power-law fan-in with alpha = 2 on [2, 256], batch 512; bench.py's
c5_csr_layer builds it), checked on samples against the oracle:

* the fp32 forward of 2,000 sampled nodes against float64 (1e-5 relative);
* the Q16.16 forward of the same nodes bit for bit against the oracle's
  restatement of the reference's edge-thread tree, which for a node depends
  only on its own edges in order, so a sub-layer of the sampled nodes over
  the child rows they read reproduces it;
* the fp32 backward (flows) of 300 sampled child rows and of every edge into
  them against float64.

The node sample includes the largest and smallest fan-ins.  Reference check
of the same kind: experiment_pyjuice/run_pyjuice.py:90-119,228-239."""

import importlib.util
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_c5", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _sub_layer(nodes_sel, off, cids, lp, child):
    """The CSR sub-layer of the selected nodes over the child rows they read."""
    fan = off[nodes_sel + 1] - off[nodes_sel]
    edges = np.concatenate([np.arange(off[n], off[n + 1]) for n in nodes_sel])
    sub_off = np.concatenate([[0], np.cumsum(fan)]).astype(np.int64)
    uniq, inv = np.unique(cids[edges], return_inverse=True)
    rows = child[torch.from_numpy(uniq).to(child.device).long()].cpu().numpy()
    return edges, sub_off, inv.astype(np.int32), lp[edges], rows


def test_c5_layer_sampled(cuda):
    import fuselse_amd

    ext = fuselse_amd.ext
    print("case C5 layer 1M nodes batch 512", flush=True)
    off, _, child, d_off, d_cid, d_lp = _bench().c5_csr_layer(torch, cuda)
    nodes, batch = child.shape
    cids = d_cid.cpu().numpy()
    lp = d_lp.cpu().numpy()
    fan = np.diff(off)
    rng = np.random.default_rng(5)
    sel = set(rng.choice(nodes, 2000, replace=False).tolist())
    sel.update(np.flatnonzero(fan == fan.max())[:4].tolist())
    sel.update(np.flatnonzero(fan == 2)[:4].tolist())
    sel = np.array(sorted(sel), np.int64)

    out = ext.sparse_csr_forward(child, d_off, d_cid, d_lp)
    outq = ext.sparse_csr_forward(child, d_off, d_cid, d_lp, q16=True)
    _, s_off, s_cid, s_lp, s_child = _sub_layer(sel, off, cids, lp, child)
    want = O.sparse_csr_fp64(s_child, s_off, s_cid, s_lp)
    np.testing.assert_allclose(out[torch.from_numpy(sel).to(cuda)].cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    wq = O.sparse_q16_csr(s_child, s_off, s_cid, s_lp)
    gq = outq[torch.from_numpy(sel).to(cuda)].cpu().numpy()
    np.testing.assert_array_equal(gq.view(np.int32), wq.view(np.int32))
    del outq

    # backward: 300 sampled children, every edge into them and the parents of those edges
    gen = torch.Generator(device=cuda)
    gen.manual_seed(6)
    gout = torch.rand(nodes, batch, device=cuda, generator=gen) + 0.05
    gchild, glp = ext.sparse_csr_backward(child, out, gout, d_off, d_cid, d_lp)
    kids = np.sort(rng.choice(nodes, 300, replace=False))
    into = np.flatnonzero(np.isin(cids, kids))
    parents = np.searchsorted(off, into, side="right") - 1
    par_u, par_inv = np.unique(parents, return_inverse=True)
    _, p_off, p_cid, p_lp, p_child = _sub_layer(par_u, off, cids, lp, child)
    out64 = O.sparse_csr_fp64(p_child, p_off, p_cid, p_lp)  # the parents' outputs in float64
    ch64 = child[torch.from_numpy(cids[into]).to(cuda).long()].cpu().numpy().astype(np.float64)
    g64 = gout[torch.from_numpy(par_u).to(cuda)].cpu().numpy().astype(np.float64)
    term = g64[par_inv] * np.exp(lp[into].astype(np.float64)[:, None] + ch64 - out64[par_inv])
    want_glp = term.sum(axis=1)
    np.testing.assert_allclose(glp[torch.from_numpy(into).to(cuda)].cpu().numpy(), want_glp, rtol=1e-5)
    want_gc = np.zeros((len(kids), batch))
    np.add.at(want_gc, np.searchsorted(kids, cids[into]), term)
    got_gc = gchild[torch.from_numpy(kids).to(cuda)].cpu().numpy()
    np.testing.assert_allclose(got_gc, want_gc, rtol=1e-5, atol=1e-30)


def test_c5_blocked_layer_sampled(cuda):
    """The block-layout layer the benchmark times (8192 blocks of 32 nodes,
    32 edges per block over 262144 element rows, batch 512, bench.py's C5
    block layer), checked on samples against the float64 oracle: the forward
    of 64 sampled blocks (the first and last included) over the child rows
    they read; the backward's element flows of 200 sampled element rows,
    whose every block edge comes from the blocks that reach them, and the
    parameter flows of those blocks."""
    import fuselse_amd

    ext = fuselse_amd.ext
    print("case C5 block layer 8192 blocks x 32 nodes, 32 edges, batch 512", flush=True)
    nbk, bs, ne, nel, batch = 8192, 32, 32, 262144, 512
    floor = float(np.float32(1e-45))
    gen = torch.Generator(device=cuda)
    gen.manual_seed(7)
    em = torch.log(torch.rand(nel, batch, device=cuda, generator=gen).clamp_min_(1e-30))
    nids = torch.arange(nbk, device=cuda, dtype=torch.int64) * bs
    cids = torch.randint(0, nel, (nbk, ne), device=cuda, generator=gen, dtype=torch.int64)
    pids = (torch.arange(nbk * ne, device=cuda, dtype=torch.int64) * bs).reshape(nbk, ne)
    params = torch.rand(nbk * ne * bs, device=cuda, generator=gen) + 1e-3
    nm = torch.empty(nbk * bs, batch, device=cuda)
    ext.sparse_forward_float(nm, em, params, nids, cids, pids, bs)
    c_np, p_np, par_np = cids.cpu().numpy(), pids.cpu().numpy(), params.cpu().numpy()
    rng = np.random.default_rng(8)

    def sub_blocks(blocks):
        """The blocks' child rows (compact), their child ids into them, their
        parent rows of `rows_of` tensors and compact node ids."""
        uniq, inv = np.unique(c_np[blocks], return_inverse=True)
        em_sub = em[torch.from_numpy(uniq).to(cuda)].cpu().numpy()
        node_rows = (blocks[:, None] * bs + np.arange(bs)[None, :]).reshape(-1)
        nids_sub = (np.arange(len(blocks)) * bs).astype(np.int64)
        return uniq, em_sub, inv.reshape(len(blocks), ne).astype(np.int64), node_rows, nids_sub

    blocks = np.unique(np.concatenate([[0, nbk - 1], rng.choice(nbk, 62, replace=False)]))
    _, em_sub, c_sub, node_rows, nids_sub = sub_blocks(blocks)
    rows, vals = O.sparse_blocked_fp64(em_sub, par_np, nids_sub, c_sub, p_np[blocks], bs, clamp=floor)
    got = nm[torch.from_numpy(node_rows[rows]).to(cuda)].cpu().numpy()
    np.testing.assert_allclose(got, vals, rtol=1e-5, atol=1e-6)

    nf = torch.rand(nbk * bs, batch, device=cuda, generator=gen)
    ef = torch.zeros(nel, batch, device=cuda)
    pf = torch.zeros(params.numel(), device=cuda)
    ext.sparse_blocked_backward(nf, ef, nm, em, params, pf, nids, cids, pids, bs)
    kids = np.sort(rng.choice(np.unique(c_np), 200, replace=False))
    reach = np.unique(np.flatnonzero(np.isin(c_np, kids).any(axis=1)))
    uniq, em_sub, c_sub, node_rows, nids_sub = sub_blocks(reach)
    nrows = torch.from_numpy(node_rows).to(cuda)
    nf_sub = nf[nrows].cpu().numpy()
    nm_sub = nm[nrows].cpu().numpy()
    de, dp = O.sparse_blocked_bwd_fp64(nf_sub, nm_sub, em_sub, par_np, nids_sub, c_sub, p_np[reach], bs, clamp=floor)
    # every term is positive (node_flows in [0, 1)), so 1e-5 of the sum bounds fp32 accumulation
    at = np.searchsorted(uniq, kids)
    got_e = ef[torch.from_numpy(kids).to(cuda)].cpu().numpy()
    np.testing.assert_allclose(got_e, de[at], rtol=1e-5, atol=1e-30)
    q = (p_np[reach][:, :, None] + np.arange(bs)[None, None, :]).reshape(-1)
    got_p = pf[torch.from_numpy(q).to(cuda)].cpu().numpy()
    np.testing.assert_allclose(got_p, dp[q], rtol=1e-5, atol=1e-30)


def test_c5_blocked_layer_whole_against_expansion(cuda):
    """Every output of the block-layout layer the benchmark times against an
    independent GPU computation of the same layer: the layer expanded to one
    CSR node per parent (node j*32 + p with the block's 32 edges and the
    log-weights log(params[pids[j, e] + p])), run through the per-parent CSR
    forward and flows kernels, which the oracle pins on their own.  The
    product form's forward, element flows and parameter flows must agree
    with them on all 262144 nodes, 262144 element rows and 8.4M edges at
    1e-5 relative (every term of the flows is positive: node_flows in
    [0, 1))."""
    import fuselse_amd

    ext = fuselse_amd.ext
    print("case C5 block layer whole against its CSR expansion", flush=True)
    nbk, bs, ne, nel, batch = 8192, 32, 32, 262144, 512
    gen = torch.Generator(device=cuda)
    gen.manual_seed(9)
    em = torch.log(torch.rand(nel, batch, device=cuda, generator=gen).clamp_min_(1e-30))
    nids = torch.arange(nbk, device=cuda, dtype=torch.int64) * bs
    cids = torch.randint(0, nel, (nbk, ne), device=cuda, generator=gen, dtype=torch.int64)
    pids = (torch.arange(nbk * ne, device=cuda, dtype=torch.int64) * bs).reshape(nbk, ne)
    params = torch.rand(nbk * ne * bs, device=cuda, generator=gen) + 1e-3
    pos = torch.arange(bs, device=cuda)
    qidx = (pids[:, None, :] + pos[None, :, None]).reshape(-1)  # CSR edge (j*bs + p)*ne + e
    x_cid = cids[:, None, :].expand(nbk, bs, ne).reshape(-1).to(torch.int32).contiguous()
    x_lp = torch.log(params[qidx]).contiguous()
    x_off = torch.arange(0, nbk * bs * ne + 1, ne, device=cuda, dtype=torch.int64)

    nm = torch.empty(nbk * bs, batch, device=cuda)
    ext.sparse_forward_float(nm, em, params, nids, cids, pids, bs)
    want = ext.sparse_csr_forward(em, x_off, x_cid, x_lp)
    torch.testing.assert_close(nm, want, rtol=1e-5, atol=1e-5)
    del want

    nf = torch.rand(nbk * bs, batch, device=cuda, generator=gen)
    ef = torch.zeros(nel, batch, device=cuda)
    pf = torch.zeros(params.numel(), device=cuda)
    ext.sparse_blocked_backward(nf, ef, nm, em, params, pf, nids, cids, pids, bs)
    g_child, g_lp = ext.sparse_csr_backward(em, nm, nf, x_off, x_cid, x_lp)
    torch.testing.assert_close(ef, g_child, rtol=1e-5, atol=1e-30)
    torch.testing.assert_close(pf[qidx], g_lp, rtol=1e-5, atol=1e-30)
