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
