"""GPU parity of the sparse probabilistic-circuit sum layers.

fp32 paths are checked against the fp64 oracle (1e-5 relative); the Q16.16
paths bit-exactly against the oracle's restatement of the reference's
edge-thread tree (experiment_pyjuice/sparse_q16_kernel.cu:61-134) when the
log-weights are given; when the kernel takes the log of linear weights itself
a 1-ulp difference of that log can move one quantised logit by one LSB, so
that case is checked to the size of one LUT step.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


def _csr(rng, nodes, nch, fanin=None, seed=0):
    k = O.powerlaw_fanin(nodes, seed=seed) if fanin is None else np.asarray(fanin, np.int64)
    off = np.concatenate([[0], np.cumsum(k)]).astype(np.int64)
    cids = rng.integers(0, nch, off[-1]).astype(np.int32)
    lp = np.log(rng.random(off[-1]) + 1e-12).astype(np.float32)
    return off, cids, lp


def _to(d, *arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(d) for a in arrs]


@pytest.mark.parametrize("batch", [1, 7, 16, 130, 512, 1000])
def test_csr_float_and_q16(cuda, batch):
    print(f"case csr batch={batch}", flush=True)
    rng = np.random.default_rng(batch)
    nodes, nch = 400, 300
    fan = O.powerlaw_fanin(nodes, seed=batch)
    fan[:6] = [0, 1, 2, 8, 9, 256]  # empty, single, ET boundaries, max fan-in
    fan[6:10] = [16, 17, 32, 33]
    off, cids, lp = _csr(rng, nodes, nch, fanin=fan)
    child = np.log(rng.random((nch, batch)) + 1e-12).astype(np.float32)
    ch, offd, cid, lpd = _to(cuda, child, off, cids, lp)
    ext = _ext()
    got = ext.sparse_csr_forward(ch, offd, cid, lpd).cpu().numpy()
    want = O.sparse_csr_fp64(child, off, cids, lp)
    assert np.isneginf(got[0]).all()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    gq = ext.sparse_csr_forward(ch, offd, cid, lpd, q16=True).cpu().numpy()
    wq = O.sparse_q16_csr(child, off, cids, lp)
    np.testing.assert_array_equal(gq.view(np.int32), wq.view(np.int32))


def test_csr_q16_extreme_logits(cuda):
    """Logits below -20000 (clamped), -inf children, +-large values."""
    rng = np.random.default_rng(5)
    nodes, nch, batch = 64, 40, 64
    off, cids, lp = _csr(rng, nodes, nch, seed=5)
    child = (rng.standard_normal((nch, batch)) * 50).astype(np.float32)
    child[0, :] = -np.inf
    child[1, :] = -3e4
    child[2, :5] = 1e4
    lp[::7] = -25000.0
    ch, offd, cid, lpd = _to(cuda, child, off, cids, lp)
    gq = _ext().sparse_csr_forward(ch, offd, cid, lpd, q16=True).cpu().numpy()
    wq = O.sparse_q16_csr(child, off, cids, lp)
    np.testing.assert_array_equal(gq.view(np.int32), wq.view(np.int32))


def _blocked(rng, nb, ne, bs, batch, nelem, nparams):
    nids = (np.arange(nb) * bs).astype(np.int64)
    cids = rng.integers(0, nelem, (nb, ne)).astype(np.int64)
    pids = rng.integers(0, nparams - bs, (nb, ne)).astype(np.int64)
    params = (rng.random(nparams) + 1e-3).astype(np.float32)
    em = np.log(rng.random((nelem, batch)) + 1e-12).astype(np.float32)
    return nids, cids, pids, params, em


@pytest.mark.parametrize("ne,bs,batch", [(5, 4, 32), (12, 2, 130), (30, 3, 512), (70, 1, 64), (300, 2, 16)])
def test_blocked_float_and_q16(cuda, ne, bs, batch):
    print(f"case blocked ne={ne} bs={bs} batch={batch}", flush=True)
    rng = np.random.default_rng(ne * bs + batch)
    nb, nelem, nparams = 6, 50, 400
    nids, cids, pids, params, em = _blocked(rng, nb, ne, bs, batch, nelem, nparams)
    nm0 = np.full((nb * bs + 3, batch), 7.0, np.float32)
    ext = _ext()
    d_nids, d_cids, d_pids, d_params, d_em = _to(cuda, nids, cids, pids, params, em)

    nm = torch.from_numpy(nm0.copy()).to(cuda)
    assert ext.sparse_forward_float(nm, d_em, d_params, d_nids, d_cids, d_pids, bs) is None
    got = nm.cpu().numpy()
    rows, vals = O.sparse_blocked_fp64(em, params, nids, cids, pids, bs)
    np.testing.assert_allclose(got[rows], vals, rtol=1e-5, atol=1e-6)
    untouched = np.setdiff1d(np.arange(nm0.shape[0]), rows)
    assert (got[untouched] == 7.0).all()

    # Q16 on log-weights: bit-exact
    logw_full = np.log(params.astype(np.float64)).astype(np.float32)
    logw = np.stack([np.stack([logw_full[pids[j] + p] for p in range(bs)]) for j in range(nb)])
    nmq = torch.from_numpy(nm0.copy()).to(cuda)
    ext.sparse_forward_q16(nmq, d_em, torch.from_numpy(logw_full).to(cuda), d_nids, d_cids, d_pids, bs,
                           params_are_log=True)
    want = O.sparse_q16_blocked(nm0, em, logw, nids, cids, bs)
    np.testing.assert_array_equal(nmq.cpu().numpy().view(np.int32), want.view(np.int32))

    # Q16 on linear weights: the kernel's own log.  A 1-ulp log difference
    # moves one quantised logit by one LSB, which can cross a LUT bin (adjacent
    # bins differ by up to 571 LSB = 6e-3), so: nearly all outputs identical,
    # the rest within one bin step.
    nml = torch.from_numpy(nm0.copy()).to(cuda)
    ext.sparse_forward_q16(nml, d_em, d_params, d_nids, d_cids, d_pids, bs)
    gl = nml.cpu().numpy()
    assert (gl == want).mean() > 0.99
    np.testing.assert_allclose(gl, want, rtol=0, atol=600 * float(O.Q16_OUT))


def test_dispatcher_contract(cuda):
    """make_sparse_dispatcher applies local_ids and passes block_size
    (run_pyjuice.py:63-77)."""
    from fuselse_amd.pc import make_sparse_dispatcher

    rng = np.random.default_rng(2)
    nb, ne, bs, batch = 5, 6, 2, 16
    nids, cids, pids, params, em = _blocked(rng, nb, ne, bs, batch, 20, 80)
    d_nids, d_cids, d_pids, d_params, d_em = _to(cuda, nids, cids, pids, params, em)

    class Layer:
        block_size = bs

    fwd = make_sparse_dispatcher(_ext().sparse_forward_float)
    nm = torch.zeros(nb * bs, batch, device=cuda)
    local = torch.tensor([1, 3], device=cuda)
    fwd(Layer(), nm, d_em, d_params, d_nids, d_cids, d_pids, local_ids=local)
    got = nm.cpu().numpy()
    rows, vals = O.sparse_blocked_fp64(em, params, nids[[1, 3]], cids[[1, 3]], pids[[1, 3]], bs)
    np.testing.assert_allclose(got[rows], vals, rtol=1e-5, atol=1e-6)
    other = np.setdiff1d(np.arange(nb * bs), rows)
    assert (got[other] == 0).all()
    with pytest.raises(NotImplementedError):
        fwd(Layer(), nm, d_em, d_params, d_nids, d_cids, d_pids, propagation_alg="MPE")


# ---------------------------------------------------------------------------
# CSR backward (flows): grad_child and grad_logparams against the fp64
# oracle.  Flows are sums of positive terms when grad_out > 0 (pyjuice's node
# flows), so they are checked to 1e-5 relative; with signed grad_out the
# bound is 1e-5 of the sum of |terms|.
# ---------------------------------------------------------------------------
def _abs_terms(child, out, gout, off, cids, lp):
    return O.sparse_csr_bwd_fp64(child, out, np.abs(gout), off, cids, lp)


@pytest.mark.parametrize("batch", [1, 7, 130, 512, 600, 1100])
@pytest.mark.parametrize("signed", [False, True])
def test_csr_backward_matches_fp64(cuda, batch, signed):
    print(f"case csr_bwd batch={batch} signed={signed}", flush=True)
    rng = np.random.default_rng(batch + 100 * signed)
    nodes, nch = 300, 200
    fan = O.powerlaw_fanin(nodes, seed=batch + 7)
    fan[:4] = [0, 1, 256, 65]   # empty node, single edge, max fan-in, across a 64-edge window
    off, cids, lp = _csr(rng, nodes, nch, fanin=fan)
    cids[:300] = 5              # one child with many parents (several 64-edge windows)
    child = np.log(rng.random((nch, batch)) + 1e-12).astype(np.float32)
    child[7, :] = -np.inf       # a child of probability 0
    ext = _ext()
    ch, offd, cid, lpd = _to(cuda, child, off, cids, lp)
    out = ext.sparse_csr_forward(ch, offd, cid, lpd)
    g = rng.standard_normal((nodes, batch)).astype(np.float32)
    if not signed:
        g = np.abs(g) + 0.1
    gd = torch.from_numpy(g).to(cuda)
    gc, gl = ext.sparse_csr_backward(ch, out, gd, offd, cid, lpd)
    out64 = O.sparse_csr_fp64(child, off, cids, lp)
    wc, wl = O.sparse_csr_bwd_fp64(child, out64, g, off, cids, lp)
    ac, al = _abs_terms(child, out64, g, off, cids, lp)
    gc, gl = gc.cpu().numpy(), gl.cpu().numpy()
    assert np.isfinite(gc).all() and np.isfinite(gl).all()
    assert (np.abs(gc - wc) <= 1e-5 * ac + 1e-30).all(), np.max(np.abs(gc - wc) / (ac + 1e-30))
    assert (np.abs(gl - wl) <= 1e-5 * al + 1e-30).all(), np.max(np.abs(gl - wl) / (al + 1e-30))
    assert (gc[7] == 0).all()


def test_csr_backward_deterministic_and_transpose(cuda):
    print("case csr_bwd determinism", flush=True)
    rng = np.random.default_rng(3)
    off, cids, lp = _csr(rng, 2000, 500, seed=3)
    child = np.log(rng.random((500, 256)) + 1e-12).astype(np.float32)
    ext = _ext()
    ch, offd, cid, lpd = _to(cuda, child, off, cids, lp)
    csc = ext.sparse_csr_transpose(offd, cid, 500)
    co, ce, cn = (t.cpu().numpy() for t in csc)
    # the transpose: per child, its edge ids in increasing order and their parents
    order = np.argsort(cids, kind="stable")
    np.testing.assert_array_equal(ce, order)
    np.testing.assert_array_equal(co, np.concatenate([[0], np.cumsum(np.bincount(cids, minlength=500))]))
    np.testing.assert_array_equal(cn, np.repeat(np.arange(2000), np.diff(off))[order])
    out = ext.sparse_csr_forward(ch, offd, cid, lpd)
    g = torch.rand(2000, 256, device=cuda)
    a = ext.sparse_csr_backward(ch, out, g, offd, cid, lpd, csc)
    for _ in range(3):
        b = ext.sparse_csr_backward(ch, out, g, offd, cid, lpd, csc)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # three 512-column tiles: the edge gradients of tiles 1 and 2 are added to
    # tile 0's in tile order by the one wave that owns the edge
    child3 = np.log(rng.random((500, 1100)) + 1e-12).astype(np.float32)
    ch3 = torch.from_numpy(child3).to(cuda)
    out3 = ext.sparse_csr_forward(ch3, offd, cid, lpd)
    g3 = torch.rand(2000, 1100, device=cuda)
    a = ext.sparse_csr_backward(ch3, out3, g3, offd, cid, lpd, csc)
    for _ in range(3):
        b = ext.sparse_csr_backward(ch3, out3, g3, offd, cid, lpd, csc)
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_csr_layer_autograd(cuda):
    """pc.sparse_csr_layer: two stacked layers trained end to end; gradients
    against torch fp64 autograd of gather + logsumexp."""
    print("case csr_layer autograd", flush=True)
    from fuselse_amd.pc import sparse_csr_layer

    rng = np.random.default_rng(4)
    batch = 64
    off1, c1, l1 = _csr(rng, 50, 40, fanin=rng.integers(1, 9, 50))
    off2, c2, l2 = _csr(rng, 10, 50, fanin=rng.integers(1, 9, 10))
    x = np.log(rng.random((40, batch)) + 1e-6).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda).requires_grad_(True)
    l1d = torch.from_numpy(l1).to(cuda).requires_grad_(True)
    l2d = torch.from_numpy(l2).to(cuda).requires_grad_(True)
    o1d, c1d, o2d, c2d = _to(cuda, off1, c1, off2, c2)
    h = sparse_csr_layer(xd, o1d, c1d, l1d)
    y = sparse_csr_layer(h, o2d, c2d, l2d)
    y.sum().backward()

    def layer_t(ch, off, cid, lw):
        rows = [torch.logsumexp(lw[off[n]:off[n + 1], None] + ch[torch.from_numpy(cid[off[n]:off[n + 1]]).long()], 0)
                for n in range(len(off) - 1)]
        return torch.stack(rows)

    xt = torch.from_numpy(x).double().requires_grad_(True)
    l1t = torch.from_numpy(l1).double().requires_grad_(True)
    l2t = torch.from_numpy(l2).double().requires_grad_(True)
    yt = layer_t(layer_t(xt, off1, c1, l1t), off2, c2, l2t)
    yt.sum().backward()
    np.testing.assert_allclose(y.detach().cpu().numpy(), yt.detach().numpy(), rtol=1e-5, atol=1e-5)
    for got, want in ((xd.grad, xt.grad), (l1d.grad, l1t.grad), (l2d.grad, l2t.grad)):
        np.testing.assert_allclose(got.cpu().numpy(), want.numpy(), rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("ne,bs,batch", [(5, 4, 32), (12, 2, 130), (30, 3, 512), (70, 1, 64), (9, 2, 600)])
def test_blocked_backward_matches_fp64(cuda, ne, bs, batch):
    """ext.sparse_blocked_backward: the flows of the block-layout layer added
    into existing element and parameter flows, against the fp64 loops of the
    oracle; also with params given as log-weights."""
    print(f"case blocked_bwd ne={ne} bs={bs} batch={batch}", flush=True)
    rng = np.random.default_rng(ne * bs + batch + 1)
    nb, nelem, nparams = 7, 40, 600
    nids, cids, pids, params, em = _blocked(rng, nb, ne, bs, batch, nelem, nparams)
    cids[0, : min(3, ne)] = 2                    # a child repeated within a block
    em[5, :] = -np.inf                           # a child of probability 0
    ext = _ext()
    for log_params in (False, True):
        p_in = np.log(params).astype(np.float32) if log_params else params
        nm = torch.zeros(nb * bs, batch, device=cuda)
        d = {k: torch.from_numpy(v).to(cuda) for k, v in (("em", em), ("p", p_in), ("nids", nids), ("cids", cids),
                                                          ("pids", pids))}
        ext.sparse_forward_float(nm, d["em"], d["p"], d["nids"], d["cids"], d["pids"], bs, params_are_log=log_params)
        nf = rng.standard_normal((nb * bs, batch)).astype(np.float32)
        ef0 = rng.standard_normal((nelem, batch)).astype(np.float32)
        pf0 = rng.standard_normal(nparams).astype(np.float32)
        ef, pf = torch.from_numpy(ef0).to(cuda), torch.from_numpy(pf0).to(cuda)
        ext.sparse_blocked_backward(torch.from_numpy(nf).to(cuda), ef, nm, d["em"], d["p"], pf, d["nids"], d["cids"],
                                    d["pids"], bs, params_are_log=log_params)
        nm64 = nm.cpu().numpy()
        de, dp = O.sparse_blocked_bwd_fp64(nf, nm64, em, p_in, nids, cids, pids, bs, params_are_log=log_params)
        ae, ap = O.sparse_blocked_bwd_fp64(np.abs(nf), nm64, em, p_in, nids, cids, pids, bs,
                                           params_are_log=log_params)
        got_e, got_p = ef.cpu().numpy(), pf.cpu().numpy()
        # fp32 terms within 1e-5 of their magnitudes, plus the rounding of the final add
        assert (np.abs(got_e - (ef0 + de)) <= 1e-5 * ae + 2e-7 * np.abs(ef0 + de) + 1e-30).all()
        assert (np.abs(got_p - (pf0 + dp)) <= 1e-5 * ap + 2e-7 * np.abs(pf0 + dp) + 1e-30).all()
        assert (got_e[5] == ef0[5]).all()        # no flow into a child of probability 0


def test_blocked_backward_subset_of_blocks(cuda):
    """The backward over a subset of node blocks (as the dispatcher selects
    with local_ids) touches only those blocks' children and parameters."""
    print("case blocked_bwd subset", flush=True)
    rng = np.random.default_rng(77)
    nb, ne, bs, batch, nelem, nparams = 6, 5, 2, 16, 30, 200
    nids, cids, pids, params, em = _blocked(rng, nb, ne, bs, batch, nelem, nparams)
    sel = np.array([1, 4])
    ext = _ext()
    nm = torch.zeros(nb * bs, batch, device=cuda)
    d = {k: torch.from_numpy(v).to(cuda) for k, v in (("em", em), ("p", params), ("nids", nids[sel]),
                                                      ("cids", cids[sel]), ("pids", pids[sel]))}
    ext.sparse_forward_float(nm, d["em"], d["p"], d["nids"], d["cids"], d["pids"], bs)
    nf = rng.standard_normal((nb * bs, batch)).astype(np.float32)
    ef = torch.zeros(nelem, batch, device=cuda)
    pf = torch.zeros(nparams, device=cuda)
    ext.sparse_blocked_backward(torch.from_numpy(nf).to(cuda), ef, nm, d["em"], d["p"], pf, d["nids"], d["cids"],
                                d["pids"], bs)
    de, dp = O.sparse_blocked_bwd_fp64(nf, nm.cpu().numpy(), em, params, nids[sel], cids[sel], pids[sel], bs)
    ae, ap = O.sparse_blocked_bwd_fp64(np.abs(nf), nm.cpu().numpy(), em, params, nids[sel], cids[sel], pids[sel], bs)
    got_e, got_p = ef.cpu().numpy(), pf.cpu().numpy()
    assert (np.abs(got_e - de) <= 1e-5 * ae + 1e-30).all()
    assert (np.abs(got_p - dp) <= 1e-5 * ap + 1e-30).all()
    untouched = np.setdiff1d(np.arange(nelem), cids[sel].reshape(-1))
    assert (got_e[untouched] == 0).all()


def test_blocked_backward_with_a_reused_plan(cuda):
    """sparse_blocked_transpose built once and passed to several backward
    calls gives the same bits as the backward that builds it itself; a plan
    of another layer is refused."""
    print("case blocked_bwd plan reuse", flush=True)
    rng = np.random.default_rng(91)
    nb, ne, bs, batch, nelem, nparams = 9, 11, 3, 96, 50, 400
    nids, cids, _, params, em = _blocked(rng, nb, ne, bs, batch, nelem, nparams)
    pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)     # one parameter per expanded edge
    ext = _ext()
    d = {k: torch.from_numpy(v).to(cuda) for k, v in (("em", em), ("p", params), ("nids", nids), ("cids", cids),
                                                      ("pids", pids))}
    nm = torch.zeros(nb * bs, batch, device=cuda)
    ext.sparse_forward_float(nm, d["em"], d["p"], d["nids"], d["cids"], d["pids"], bs)
    plan = ext.sparse_blocked_transpose(d["nids"], d["cids"], d["pids"], bs, nelem)
    for rep in range(3):
        nf = torch.from_numpy(rng.standard_normal((nb * bs, batch)).astype(np.float32)).to(cuda)
        ef_a, pf_a = torch.zeros(nelem, batch, device=cuda), torch.zeros(nparams, device=cuda)
        ef_b, pf_b = torch.zeros_like(ef_a), torch.zeros_like(pf_a)
        ext.sparse_blocked_backward(nf, ef_a, nm, d["em"], d["p"], pf_a, d["nids"], d["cids"], d["pids"], bs)
        ext.sparse_blocked_backward(nf, ef_b, nm, d["em"], d["p"], pf_b, d["nids"], d["cids"], d["pids"], bs,
                                    plan=plan)
        assert torch.equal(ef_a, ef_b)
        assert torch.equal(pf_a, pf_b)
    other = ext.sparse_blocked_transpose(d["nids"][:4], d["cids"][:4], d["pids"][:4], bs, nelem)
    with pytest.raises(RuntimeError, match="plan does not fit"):
        ext.sparse_blocked_backward(nf, ef_a, nm, d["em"], d["p"], pf_a, d["nids"], d["cids"], d["pids"], bs,
                                    plan=other)


# ---------------------------------------------------------------------------
# Block layout, fp32, block_size >= 2: the product form on the matrix cores
# (node_mars = log W_p + m_b + log sum_e w'[p, e] exp(x[e, b] - m_b)), against
# the fp64 loops of the oracle.  The weight floor is the fp32 value of 1e-45
# (the smallest subnormal), which the kernels apply before the log.
# ---------------------------------------------------------------------------
F32_FLOOR = float(np.float32(1e-45))

# (32, 32, 100) and (64, 32, 200): whole tiles of whole chunks (the unmasked
# fold) and a last partial tile (the masked one) in the same launch
PRODUCT_CASES = [(8, 5, 64), (16, 32, 130), (24, 33, 512), (32, 32, 512), (48, 7, 96), (64, 100, 260),
                 (128, 16, 64), (32, 1, 3), (9, 70, 600), (16, 64, 1), (2, 40, 200), (5, 16, 129), (3, 9, 8),
                 (32, 32, 100), (64, 32, 200)]


@pytest.mark.parametrize("bs,ne,batch", PRODUCT_CASES)
@pytest.mark.parametrize("log_params", [False, True])
def test_blocked_product_form_matches_fp64(cuda, bs, ne, batch, log_params):
    print(f"case blocked product bs={bs} ne={ne} batch={batch} log={log_params}", flush=True)
    rng = np.random.default_rng(bs * 1000 + ne * 10 + batch)
    nb, nelem = 5, 90
    nparams = nb * ne * bs + 40
    nids = (np.arange(nb) * (bs + 2) + 1).astype(np.int64)     # gaps between blocks stay untouched
    cids = rng.integers(0, nelem, (nb, ne)).astype(np.int64)
    pids = rng.integers(0, nparams - bs + 1, (nb, ne)).astype(np.int64)
    params = (rng.random(nparams) + 1e-3).astype(np.float32)
    em = (np.log(rng.random((nelem, batch)) + 1e-12) * rng.choice([1.0, 5.0], (nelem, 1))).astype(np.float32)
    p_in = np.log(params).astype(np.float32) if log_params else params
    nm0 = np.full((int(nids[-1]) + bs + 3, batch), 7.0, np.float32)
    nm = torch.from_numpy(nm0.copy()).to(cuda)
    d = _to(cuda, em, p_in, nids, cids, pids)
    _ext().sparse_forward_float(nm, d[0], d[1], d[2], d[3], d[4], bs, params_are_log=log_params)
    got = nm.cpu().numpy()
    if log_params:
        rows, vals = O.sparse_blocked_fp64(em, np.exp(p_in.astype(np.float64)), nids, cids, pids, bs, clamp=0.0)
    else:
        rows, vals = O.sparse_blocked_fp64(em, params, nids, cids, pids, bs, clamp=F32_FLOOR)
    np.testing.assert_allclose(got[rows], vals, rtol=1e-5, atol=1e-6)
    untouched = np.setdiff1d(np.arange(nm0.shape[0]), rows)
    assert (got[untouched] == 7.0).all()


@pytest.mark.parametrize("ne,bs,batch", [(40, 16, 68), (32, 32, 128)])
def test_blocked_product_form_special_values_and_fallback(cuda, ne, bs, batch):
    """Entries the product cannot resolve take the exact fold: -inf children,
    columns of -inf, +inf and NaN children (a NaN among -inf children of the
    first 32-edge chunk included), zero weights, a parent whose only large
    weights meet children ~200 nats below the column maximum.  40 edges run
    the multi-chunk kernel; 32 edges of 32 parents over whole tiles the
    unmasked fold."""
    print(f"case blocked product special values ne={ne} bs={bs} batch={batch}", flush=True)
    rng = np.random.default_rng(5)
    nb, nelem = 3, 60
    nids = (np.arange(nb) * bs).astype(np.int64)
    cids = np.stack([rng.permutation(nelem)[:ne] for _ in range(nb)]).astype(np.int64)
    pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)
    params = (rng.random(nb * ne * bs) + 1e-3).astype(np.float32)
    em = np.log(rng.random((nelem, batch)) + 1e-9).astype(np.float32)
    em[cids[0, 3], :] = -np.inf                  # a child of probability 0
    em[:, 5] = -np.inf                           # a column where every child is -inf
    em[cids[1, 0], 7] = np.inf                   # +inf wins
    em[cids[2, 1], 9] = np.nan                   # NaN wins
    # block 0, column 11: the first 32-edge chunk all -inf but one NaN, the
    # last 8 edges finite: the NaN still wins
    em[cids[0, :32], 11] = -np.inf
    em[cids[0, 4], 11] = np.nan
    params[pids[0, :] + 2] = 0.0                 # parent 2 of block 0: every weight zero
    params[pids[1, 5] + 4] = 0.0                 # one zero weight
    # block 2, parent 6: weight ~1 only on edge 0, whose child sits 200 below
    # the column maximum held by edge 1, whose weight is zero
    params[pids[2, :] + 6] = 1e-36
    params[pids[2, 0] + 6] = 1.0
    params[pids[2, 1] + 6] = 0.0
    em[cids[2, 0], 20:30] = -200.0
    em[cids[2, 1], 20:30] = 0.0
    nm = torch.zeros(nb * bs, batch, device=cuda)
    d = _to(cuda, em, params, nids, cids, pids)
    _ext().sparse_forward_float(nm, d[0], d[1], d[2], d[3], d[4], bs)
    got = nm.cpu().numpy()
    rows, vals = O.sparse_blocked_fp64(em, params, nids, cids, pids, bs, clamp=F32_FLOOR)
    want = np.empty_like(got, dtype=np.float64)
    want[rows] = vals
    assert np.isneginf(got[:, 5]).all()
    assert np.isnan(got[bs * 2:, 9]).all() and np.isposinf(got[bs:2 * bs, 7]).all()
    assert np.isnan(got[:bs, 11]).all()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6, equal_nan=True)
    assert (np.abs(got[2 * bs + 6, 20:30] - want[2 * bs + 6, 20:30]) < 1e-3).all()


@pytest.mark.parametrize("offset", [1, 3])
def test_blocked_product_form_unaligned_rows(cuda, offset):
    """Rows that are not 16-byte aligned take the scalar-column loads."""
    print(f"case blocked product unaligned off={offset}", flush=True)
    rng = np.random.default_rng(offset)
    nb, ne, bs, batch, nelem = 4, 12, 16, 36, 30
    nids, cids, pids, params, em = _blocked(rng, nb, ne, bs, batch, nelem, 600)
    buf = torch.zeros(nelem * batch + offset, device=cuda)
    emd = buf[offset:].view(nelem, batch)
    emd.copy_(torch.from_numpy(em).to(cuda))
    obuf = torch.zeros(nb * bs * batch + offset, device=cuda)
    nm = obuf[offset:].view(nb * bs, batch)
    d = _to(cuda, params, nids, cids, pids)
    _ext().sparse_forward_float(nm, emd, d[0], d[1], d[2], d[3], bs)
    rows, vals = O.sparse_blocked_fp64(em, params, nids, cids, pids, bs, clamp=F32_FLOOR)
    np.testing.assert_allclose(nm.cpu().numpy()[rows], vals, rtol=1e-5, atol=1e-6)


def test_blocked_product_form_log_weights_empty_first_chunk(cuda):
    """Log-weights of -inf (structural zeros): a parent whose first 32 edges
    are all -inf and whose later edges are finite (the online row maximum
    starts from nothing), and a parent with every weight -inf (-> -inf)."""
    print("case blocked product log-weights -inf", flush=True)
    rng = np.random.default_rng(17)
    nb, ne, bs, batch, nelem = 2, 70, 32, 64, 100
    nids = (np.arange(nb) * bs).astype(np.int64)
    cids = rng.integers(0, nelem, (nb, ne)).astype(np.int64)
    pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)
    lw = np.log(rng.random(nb * ne * bs) + 1e-3).astype(np.float32)
    lw[pids[0, :32] + 5] = -np.inf
    lw[pids[1, :] + 9] = -np.inf
    em = np.log(rng.random((nelem, batch)) + 1e-9).astype(np.float32)
    nm = torch.zeros(nb * bs, batch, device=cuda)
    d = _to(cuda, em, lw, nids, cids, pids)
    _ext().sparse_forward_float(nm, d[0], d[1], d[2], d[3], d[4], bs, params_are_log=True)
    got = nm.cpu().numpy()
    with np.errstate(divide="ignore"):
        rows, vals = O.sparse_blocked_fp64(em, np.exp(lw.astype(np.float64)), nids, cids, pids, bs, clamp=0.0)
    want = np.empty_like(got, dtype=np.float64)
    want[rows] = vals
    assert np.isneginf(got[bs + 9]).all()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# Block layout backward, block_size >= 2: fl_sparse_blocked_bwd (edge flows
# and parameter flows as products on the matrix cores, element flows summed
# in a fixed order), against the fp64 loops of the oracle with the node_mars
# of the kernels' own forward.  Bound: 1e-5 of the sum of |terms| of each
# entry plus fp32 rounding of the final add.
# ---------------------------------------------------------------------------
# (32, 32, 512), (16, 64, 128), (8, 16, 64) and (4, 32, 192) have every parent,
# edge and column of the single-pass kernel's tiles in range (its variant
# without bound tests)
PRODUCT_BWD_CASES = [(2, 5, 64), (16, 16, 130), (32, 32, 512), (24, 33, 96), (48, 70, 64), (64, 7, 260),
                     (9, 40, 1), (32, 3, 3), (128, 20, 64), (16, 64, 128), (8, 16, 64), (4, 32, 192)]


def _blocked_bwd_case(cuda, rng, nb, ne, bs, batch, nelem, log_params, special=False):
    nids = (np.arange(nb) * (bs + 1)).astype(np.int64)
    cids = rng.integers(0, nelem, (nb, ne)).astype(np.int64)
    pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)
    params = (rng.random(nb * ne * bs) + 1e-3).astype(np.float32)
    em = np.log(rng.random((nelem, batch)) + 1e-9).astype(np.float32)
    return nids, cids, pids, params, em


def _check_blocked_bwd(cuda, nids, cids, pids, params, em, bs, batch, log_params, nf=None, clamp=F32_FLOOR):
    rng = np.random.default_rng(1)
    nb, ne = cids.shape
    nelem = em.shape[0]
    nrows = int(nids.max()) + bs + 2
    p_in = np.log(params).astype(np.float32) if log_params else params
    d = {k: torch.from_numpy(v).to(cuda) for k, v in (("em", em), ("p", p_in), ("nids", nids), ("cids", cids),
                                                      ("pids", pids))}
    nm = torch.full((nrows, batch), -np.inf, device=cuda)
    ext = _ext()
    ext.sparse_forward_float(nm, d["em"], d["p"], d["nids"], d["cids"], d["pids"], bs, params_are_log=log_params)
    if nf is None:
        nf = rng.standard_normal((nrows, batch)).astype(np.float32)
    ef0 = rng.standard_normal((nelem, batch)).astype(np.float32)
    pf0 = rng.standard_normal(params.size).astype(np.float32)
    ef, pf = torch.from_numpy(ef0).to(cuda), torch.from_numpy(pf0).to(cuda)
    ext.sparse_blocked_backward(torch.from_numpy(nf).to(cuda), ef, nm, d["em"], d["p"], pf, d["nids"], d["cids"],
                                d["pids"], bs, params_are_log=log_params)
    nm64 = nm.cpu().numpy()
    p_or = np.exp(p_in.astype(np.float64)) if log_params else params
    kw = dict(clamp=0.0) if log_params else dict(clamp=clamp)
    with np.errstate(divide="ignore"):
        de, dp = O.sparse_blocked_bwd_fp64(nf, nm64, em, p_in if log_params else p_or, nids, cids, pids, bs,
                                           params_are_log=log_params, **kw)
        ae, ap = O.sparse_blocked_bwd_fp64(np.abs(nf), nm64, em, p_in if log_params else p_or, nids, cids, pids, bs,
                                           params_are_log=log_params, **kw)
    got_e, got_p = ef.cpu().numpy(), pf.cpu().numpy()
    want_e, want_p = ef0 + de, pf0 + dp
    bad_e = ~(np.abs(got_e - want_e) <= 1e-5 * ae + 2e-7 * np.abs(want_e) + 1e-30)
    bad_p = ~(np.abs(got_p - want_p) <= 1e-5 * ap + 2e-7 * np.abs(want_p) + 1e-30)
    assert not bad_e.any(), (np.argwhere(bad_e)[:5], got_e[bad_e][:5], want_e[bad_e][:5])
    assert not bad_p.any(), (np.argwhere(bad_p)[:5], got_p[bad_p][:5], want_p[bad_p][:5])
    return got_e, got_p


@pytest.mark.parametrize("bs,ne,batch", [(32, 32, 128), (16, 20, 70), (4, 33, 64), (48, 10, 64)])
def test_blocked_backward_shared_parameters(cuda, bs, ne, batch):
    """Parameters shared between block edges (overlapping ranges pids[j, e] +
    [0, block_size)): the plan says so, and the single pass (at most 32
    parents) and the two kernels (48) add each (block, parent, edge) sum
    atomically, against fp64; with the layer's parameters disjoint, the plan
    says that instead (and the single pass adds them with plain writes)."""
    print(f"case blocked bwd shared params bs={bs} ne={ne} batch={batch}", flush=True)
    rng = np.random.default_rng(bs + ne)
    nb, nelem = 6, 40
    nids, cids, pids, params, em = _blocked_bwd_case(cuda, rng, nb, ne, bs, batch, nelem, False)
    ext = _ext()
    d = {k: torch.from_numpy(v).to(cuda) for k, v in (("nids", nids), ("cids", cids), ("pids", pids))}
    assert ext.sparse_blocked_transpose(d["nids"], d["cids"], d["pids"], bs, nelem).params_disjoint
    shared = rng.integers(0, 3 * bs, (nb, ne)).astype(np.int64)     # ranges overlap and repeat
    params = (rng.random(4 * bs) + 1e-3).astype(np.float32)
    d["pids"] = torch.from_numpy(shared).to(cuda)
    assert not ext.sparse_blocked_transpose(d["nids"], d["cids"], d["pids"], bs, nelem).params_disjoint
    _check_blocked_bwd(cuda, nids, cids, shared, params, em, bs, batch, False)


@pytest.mark.parametrize("bs,ne,batch", PRODUCT_BWD_CASES)
@pytest.mark.parametrize("log_params", [False, True])
def test_blocked_backward_product_form_matches_fp64(cuda, bs, ne, batch, log_params):
    print(f"case blocked bwd product bs={bs} ne={ne} batch={batch} log={log_params}", flush=True)
    rng = np.random.default_rng(bs * 100 + ne + batch)
    nb, nelem = 5, 60
    nids, cids, pids, params, em = _blocked_bwd_case(cuda, rng, nb, ne, bs, batch, nelem, log_params)
    cids[0, : min(3, ne)] = 2                    # a child repeated within a block
    em[5, :] = -np.inf                           # a child of probability 0
    _check_blocked_bwd(cuda, nids, cids, pids, params, em, bs, batch, log_params)


@pytest.mark.parametrize("bs,ne,batch", [(16, 40, 68), (32, 40, 68), (48, 40, 68), (32, 32, 64), (16, 16, 128)])
def test_blocked_backward_product_form_pairs_left_out(cuda, bs, ne, batch):
    """Pairs (parent, column) whose scale factor would pass 2^24 take the
    one-by-one terms: a parent whose only large weight meets a child ~200
    below the column maximum (held by a child of weight zero); a column where
    every child is -inf (parents of probability 0, no flow).  Block sizes 16
    and 32 run the single-pass kernel (its second pass; (32, 32, 64) and
    (16, 16, 128) its variant without bound tests), 48 the two kernels."""
    print(f"case blocked bwd product left-out pairs bs={bs} ne={ne} batch={batch}", flush=True)
    rng = np.random.default_rng(23)
    nb, nelem = 3, 90
    nids = (np.arange(nb) * bs).astype(np.int64)
    cids = np.stack([rng.permutation(nelem)[:ne] for _ in range(nb)]).astype(np.int64)
    pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)
    params = (rng.random(nb * ne * bs) + 1e-3).astype(np.float32)
    em = np.log(rng.random((nelem, batch)) + 1e-9).astype(np.float32)
    params[pids[2, :] + 6] = 1e-36
    params[pids[2, 0] + 6] = 1.0
    params[pids[2, 1] + 6] = 0.0
    em[cids[2, 0], 20:30] = -200.0
    em[cids[2, 1], 20:30] = 0.0
    em[:, 40] = -np.inf
    nf = rng.standard_normal((nb * bs + 2, batch)).astype(np.float32)
    got_e, got_p = _check_blocked_bwd(cuda, nids, cids, pids, params, em, bs, batch, False, nf=nf)
    # the left-out parent's parameter flows carry its whole flow
    assert np.isfinite(got_p).all()


@pytest.mark.parametrize("offset", [1, 3])
def test_blocked_backward_product_form_unaligned(cuda, offset):
    """Odd batch and rows off the 16-byte grid take the scalar-column loads."""
    print(f"case blocked bwd product unaligned off={offset}", flush=True)
    rng = np.random.default_rng(40 + offset)
    nb, ne, bs, batch, nelem = 4, 20, 8, 37, 30
    nids, cids, pids, params, em = _blocked_bwd_case(cuda, rng, nb, ne, bs, batch, nelem, False)
    _check_blocked_bwd(cuda, nids, cids, pids, params, em, bs, batch, False)


@pytest.mark.parametrize("bs,ne,batch", [(48, 33, 300), (12, 33, 300), (16, 32, 320)])
def test_blocked_backward_product_form_deterministic(cuda, bs, ne, batch):
    """Element and parameter flows are the same bits on every call (block
    size 48: the two product kernels, which take blocks of more than 32
    parents; 12: the single-pass kernel; (16, 32, 320): its variant without
    bound tests)."""
    print(f"case blocked bwd product determinism bs={bs} ne={ne} batch={batch}", flush=True)
    rng = np.random.default_rng(8)
    nb, nelem = 40, 20        # few elements: many block edges per element
    nids, cids, pids, params, em = _blocked_bwd_case(cuda, rng, nb, ne, bs, batch, nelem, False)
    d = _to(cuda, em, params, nids, cids, pids)
    nm = torch.zeros(nb * (bs + 1), batch, device=cuda)
    ext = _ext()
    ext.sparse_forward_float(nm, d[0], d[1], d[2], d[3], d[4], bs)
    nf = torch.from_numpy(rng.standard_normal((nb * (bs + 1), batch)).astype(np.float32)).to(cuda)
    outs = []
    for _ in range(3):
        ef = torch.zeros(nelem, batch, device=cuda)
        pf = torch.zeros(params.size, device=cuda)
        ext.sparse_blocked_backward(nf, ef, nm, d[0], d[1], pf, d[2], d[3], d[4], bs)
        outs.append((ef, pf))
    for ef, pf in outs[1:]:
        assert torch.equal(ef, outs[0][0]) and torch.equal(pf, outs[0][1])


@pytest.mark.parametrize("bs1,bs2", [(8, 4), (32, 2), (1, 16), (48, 3)])
def test_blocked_layer_autograd_two_layers(cuda, bs1, bs2):
    """pc.sparse_blocked_layer: two stacked block-layout layers with log-weights,
    outputs and gradients of the inputs and of both weight vectors against
    torch fp64 autograd of the same layers."""
    from fuselse_amd.pc import sparse_blocked_layer

    print(f"case blocked layer autograd bs={bs1},{bs2}", flush=True)
    rng = np.random.default_rng(bs1 * 10 + bs2)
    batch, nx = 70, 24

    def layer_spec(nchild, nb, ne, bs):
        nids = (np.arange(nb) * bs).astype(np.int64)
        cids = rng.integers(0, nchild, (nb, ne)).astype(np.int64)
        pids = (np.arange(nb * ne, dtype=np.int64) * bs).reshape(nb, ne)
        lw = (rng.standard_normal(nb * ne * bs) * 0.5 - 1.0).astype(np.float32)
        return nids, cids, pids, lw

    n1b, n2b = 6, 3
    L1 = layer_spec(nx, n1b, 9, bs1)
    L2 = layer_spec(n1b * bs1, n2b, 12, bs2)
    x = np.log(rng.random((nx, batch)) + 1e-6).astype(np.float32)

    def run_gpu():
        xd = torch.from_numpy(x).to(cuda).requires_grad_(True)
        w1 = torch.from_numpy(L1[3]).to(cuda).requires_grad_(True)
        w2 = torch.from_numpy(L2[3]).to(cuda).requires_grad_(True)
        i1 = [torch.from_numpy(a).to(cuda) for a in L1[:3]]
        i2 = [torch.from_numpy(a).to(cuda) for a in L2[:3]]
        h = sparse_blocked_layer(xd, w1, *i1, bs1, n1b * bs1)
        y = sparse_blocked_layer(h, w2, *i2, bs2, n2b * bs2)
        (y * torch.linspace(0.5, 1.5, batch, device=cuda)).sum().backward()
        return y.detach().cpu().numpy(), xd.grad.cpu().numpy(), w1.grad.cpu().numpy(), w2.grad.cpu().numpy()

    def layer_t(ch, spec, lw, bs):
        nids, cids, pids, _ = spec
        rows = []
        for j in range(len(nids)):
            for p in range(bs):
                q = torch.from_numpy(pids[j] + p)
                rows.append(torch.logsumexp(lw[q][:, None] + ch[torch.from_numpy(cids[j])], 0))
        return torch.stack(rows)

    xt = torch.from_numpy(x).double().requires_grad_(True)
    w1t = torch.from_numpy(L1[3]).double().requires_grad_(True)
    w2t = torch.from_numpy(L2[3]).double().requires_grad_(True)
    yt = layer_t(layer_t(xt, L1, w1t, bs1), L2, w2t, bs2)
    (yt * torch.linspace(0.5, 1.5, batch, dtype=torch.float64)).sum().backward()
    y, gx, g1, g2 = run_gpu()
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-5, atol=1e-5)
    for got, want in ((gx, xt.grad), (g1, w1t.grad), (g2, w2t.grad)):
        np.testing.assert_allclose(got, want.numpy(), rtol=1e-4, atol=1e-5)
