"""Inputs past 2^31 elements and 2^32 bytes.

Every kernel computes row and element offsets in 64 bits and keeps 32-bit
offsets inside a row or a row group; these tests run each path on tensors of
4-9 GB and check the rows on either side of the 2^31- and 2^32-element and
2^32- and 2^33-byte boundaries (plus the first and last rows) against the
oracle: float paths in float64 within the stated tolerances, integer paths
bit for bit.  Inputs are generated on the GPU from a seeded generator and
only the checked rows come back to the host."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

RTOL32 = 1e-5
RTOL16 = 1e-3


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


@pytest.fixture
def big(cuda):
    """Frees the large tensors of a test before the next one allocates."""
    yield cuda
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _boundary_rows(B: int, N: int, esize: int) -> list:
    """Rows that hold or neighbour element 2^31 / 2^32 and byte 2^32 / 2^33."""
    rows = {0, 1, B - 2, B - 1}
    for limit in (1 << 31, 1 << 32):
        rows.update({limit // N - 1, limit // N, limit // N + 1})
    for limit in (1 << 32, 1 << 33):
        r = limit // (N * esize)
        rows.update({r - 1, r, r + 1})
    out = sorted(r for r in rows if 0 <= r < B)
    assert any(r * N * esize >= 1 << 32 for r in out), "the case must cross 2^32 bytes"
    return out


def _randn(shape, dtype, seed, dev, scale=2.0):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.empty(shape, dtype=dtype, device=dev)
    flat = x.view(-1)
    step = 1 << 28
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i:i + n] = (torch.randn(n, device=dev, generator=g) * scale).to(dtype)
    return x


def test_fwd_bwd_f32_past_2g_elements(big):
    """(16400, 131072) fp32, 8.6 GB: one block per row forward (robust and
    plain) and the flat fused backward."""
    B, N = 16400, 131072
    print(f"case large fwd/bwd f32 B={B} N={N}", flush=True)
    x = _randn((B, N), torch.float32, 11, big, scale=3.0)
    rows = _boundary_rows(B, N, 4)
    xr = x[rows].cpu().numpy()
    want = O.lse_fp64(xr)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(x)
    np.testing.assert_allclose(lse[rows].cpu().numpy(), want, rtol=RTOL32)
    plain = ext.onepass_lse_float(x)
    np.testing.assert_allclose(plain[rows].cpu().numpy(), want, rtol=RTOL32)
    g = torch.randn(B, device=big, generator=torch.Generator(device=big).manual_seed(12))
    gx = ext.onepass_lse_float_backward(g, x, lse)
    gw = O.lse_bwd_fp64(g[rows].cpu().numpy(), xr, want)
    np.testing.assert_allclose(gx[rows].cpu().numpy(), gw, rtol=RTOL32, atol=1e-30)


def test_selective_f32_past_2g_elements(big):
    """Fused selective log-softmax forward and backward at (16400, 131072)."""
    B, N = 16400, 131072
    print(f"case large selective f32 B={B} N={N}", flush=True)
    x = _randn((B, N), torch.float32, 13, big, scale=3.0)
    idx = torch.randint(0, N, (B,), device=big, generator=torch.Generator(device=big).manual_seed(14))
    rows = _boundary_rows(B, N, 4)
    xr = x[rows].cpu().numpy()
    ir = idx[rows].cpu().numpy()
    ext = _ext()
    logp, lse = ext.selective_log_softmax_float(x, idx)
    want, want_lse = O.selective_logsoftmax_fp64(xr, ir)
    np.testing.assert_allclose(logp[rows].cpu().numpy(), want, rtol=RTOL32, atol=1e-5)
    np.testing.assert_allclose(lse[rows].cpu().numpy(), want_lse, rtol=RTOL32)
    go = torch.randn(B, device=big, generator=torch.Generator(device=big).manual_seed(15))
    gx = ext.selective_log_softmax_float_backward(go, x, idx, lse)
    gw = O.selective_logsoftmax_bwd_fp64(go[rows].cpu().numpy(), xr, ir, want_lse)
    np.testing.assert_allclose(gx[rows].cpu().numpy(), gw, rtol=RTOL32, atol=1e-6)


def test_split_rows_f32_gib_rows(big):
    """Eight rows of 2^28 + 5 fp32 elements (1 GiB each, 8.6 GB): the
    split-row forward (its segments' offsets pass 2^31 elements) and the
    row-chunk backward; every element against float64 on the GPU."""
    B, N = 8, (1 << 28) + 5
    print(f"case large split f32 B={B} N={N}", flush=True)
    x = _randn((B, N), torch.float32, 16, big, scale=3.0)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(x)
    g = torch.randn(B, device=big, generator=torch.Generator(device=big).manual_seed(17))
    gx = ext.onepass_lse_float_backward(g, x, lse)
    for r in range(B):
        xr = x[r].double()
        want = torch.logsumexp(xr, 0)
        torch.testing.assert_close(lse[r].double(), want, rtol=RTOL32, atol=0.0)
        gw = g[r].double() * torch.exp(xr - want)
        torch.testing.assert_close(gx[r].double(), gw, rtol=RTOL32, atol=1e-30)
        del xr, gw


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fwd_bwd_half_past_4g_elements(big, dtype):
    """(4400000, 1000) fp16/bf16, 8.8 GB and 4.4e9 elements: the short-row
    forward (32 lanes per row) and the flat fused backward."""
    B, N = 4_400_000, 1000
    print(f"case large fwd/bwd {dtype} B={B} N={N}", flush=True)
    x = _randn((B, N), dtype, 18, big)
    rows = _boundary_rows(B, N, 2)
    xr = x[rows].float().cpu().numpy()
    want = O.lse_fp64(xr)
    ext = _ext()
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    lse = fn(x, robust=True)
    np.testing.assert_allclose(lse[rows].cpu().numpy(), want, rtol=2e-5, atol=1e-5)
    g = torch.randn(B, device=big, generator=torch.Generator(device=big).manual_seed(19))
    gx = ext.onepass_lse_half_backward(g, x, lse)
    gw = O.lse_bwd_fp64(g[rows].cpu().numpy(), xr, lse[rows].double().cpu().numpy())
    # the result is rounded to the half format: within half an ulp plus the fp32 arithmetic
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    np.testing.assert_allclose(gx[rows].float().cpu().numpy(), gw, rtol=ulp, atol=1e-7)


@pytest.mark.parametrize("use_lut", [True, False])
def test_intlse_q16_f32_past_2g_elements(big, use_lut):
    """IntLSE Q16.16 on (16400, 131072) fp32: out and raw accumulators bit
    for bit against the oracle's GPU tree."""
    B, N = 16400, 131072
    print(f"case large q16 f32 B={B} N={N} lut={use_lut}", flush=True)
    x = _randn((B, N), torch.float32, 20, big, scale=2.0)
    rows = _boundary_rows(B, N, 4)
    xr = x[rows].cpu().numpy()
    acc = torch.empty(B, dtype=torch.int32, device=big)
    fn = _ext().batched_logsumexp if use_lut else _ext().batched_logsumexp_nolut
    out = fn(x, acc_out=acc)
    # rows of 131072 fp32 are whole 16-byte vectors: every row has the base's alignment
    want, want_acc = O.q16_gpu_rows(xr, base_mod=x.data_ptr() & 15, use_lut=use_lut, raw=True)
    np.testing.assert_array_equal(acc[rows].cpu().numpy(), want_acc)
    np.testing.assert_array_equal(out[rows].cpu().numpy().view(np.int32), want.view(np.int32))


def test_intlse_q16_f32_rows_past_one_dispatch(big):
    """IntLSE Q16.16 on (2^24 + 3, 16) fp32, 1 GiB: one 256-thread block per
    row needs 2^32 + 768 work-items, more than one dispatch holds, so the
    launcher splits the rows over two launches.  The first and last rows and
    the rows on either side of the split, out and raw accumulators bit for bit
    against the oracle's GPU tree."""
    B, N = (1 << 24) + 3, 16
    split = (((1 << 32) - 1) // 256) & ~7
    print(f"case q16 f32 rows past one dispatch B={B} N={N}", flush=True)
    x = _randn((B, N), torch.float32, 21, big, scale=2.0)
    rows = sorted({0, 1, 2, split - 2, split - 1, split, split + 1, B - 2, B - 1})
    xr = x[rows].cpu().numpy()
    acc = torch.empty(B, dtype=torch.int32, device=big)
    out = _ext().batched_logsumexp(x, acc_out=acc)
    want, want_acc = O.q16_gpu_rows(xr, base_mod=x.data_ptr() & 15, use_lut=True, raw=True)
    np.testing.assert_array_equal(acc[rows].cpu().numpy(), want_acc)
    np.testing.assert_array_equal(out[rows].cpu().numpy().view(np.int32), want.view(np.int32))


def test_bwd_f32_flat_past_one_dispatch(big):
    """The flat fused backward over (2^21 + 1, 8192) fp32, 2^34 + 8192
    elements (64 GiB in, 64 GiB out): 2^26 + 32 one-wave blocks, more than one
    dispatch holds, so the launcher splits them over two launches.  The first
    and last rows and the rows around the split against float64."""
    B, N = (1 << 21) + 1, 8192
    split_row = ((((1 << 32) - 1) // 64) & ~7) * 64 * 4 // N
    print(f"case flat bwd f32 past one dispatch B={B} N={N}", flush=True)
    torch.cuda.empty_cache()
    x = _randn((B, N), torch.float32, 22, big, scale=3.0)
    rows = sorted({0, 1, split_row - 1, split_row, split_row + 1, B - 1})
    ext = _ext()
    lse = ext.onepass_lse_float_robust(x)
    g = torch.randn(B, device=big, generator=torch.Generator(device=big).manual_seed(23))
    gx = ext.onepass_lse_float_backward(g, x, lse)
    xr = x[rows].cpu().numpy()
    want = O.lse_fp64(xr)
    np.testing.assert_allclose(lse[rows].cpu().numpy(), want, rtol=RTOL32)
    gw = O.lse_bwd_fp64(g[rows].cpu().numpy(), xr, want)
    np.testing.assert_allclose(gx[rows].cpu().numpy(), gw, rtol=RTOL32, atol=1e-30)


@pytest.mark.parametrize("N", [1000, 1001])
def test_intlse_q10_6_past_4g_elements(big, N):
    """IntLSE Q10.6 on 4.4e9 int16 elements: N = 1000 takes the kernel with
    two virtual threads per thread, N = 1001 the one-virtual-thread kernel;
    bit for bit against the oracle."""
    B = 4_400_000
    print(f"case large q10_6 B={B} N={N}", flush=True)
    q = torch.empty((B, N), dtype=torch.int16, device=big)
    g = torch.Generator(device=big)
    g.manual_seed(21 + N)
    flat = q.view(-1)
    step = 1 << 28
    for i in range(0, flat.numel(), step):
        n = min(step, flat.numel() - i)
        flat[i:i + n] = torch.round(torch.randn(n, device=big, generator=g) * 128.0).clamp(-32768, 32767).to(torch.int16)
    acc = torch.empty(B, dtype=torch.int32, device=big)
    out = _ext().batched_logsumexp_q10_6(q, acc_out=acc)
    if N % 8 == 0:
        rows = _boundary_rows(B, N, 2)
        want, want_acc = O.q10_6_rows(q[rows].cpu().numpy(), base_mod=q.data_ptr() & 15, raw=True)
        np.testing.assert_array_equal(acc[rows].cpu().numpy(), want_acc)
        np.testing.assert_array_equal(out[rows].cpu().numpy().view(np.int32), want.view(np.int32))
    else:
        # rows start at every even offset mod 16: check each boundary row with its own alignment
        for r in _boundary_rows(B, N, 2):
            mod = (q.data_ptr() + r * N * 2) & 15
            want, want_acc = O.q10_6_rows(q[r:r + 1].cpu().numpy(), base_mod=mod, raw=True)
            assert int(acc[r]) == int(want_acc[0]), r
            assert out[r:r + 1].cpu().numpy().view(np.int32)[0] == want.view(np.int32)[0], r


def _far_children(rng, nch, nnz, batch):
    """Child ids spread over the whole child matrix with a third of them past
    the row whose offset crosses 2^32 bytes, and the last row."""
    cross = (1 << 32) // (batch * 4)
    ids = np.concatenate([rng.integers(0, nch, nnz - nnz // 3), rng.integers(cross, nch, nnz // 3)])
    ids[-1] = nch - 1
    ids[0] = cross
    rng.shuffle(ids)
    return ids


def test_sparse_csr_child_past_4g_bytes(big):
    """CSR forward (fp32 and Q16) and backward gathering child rows past
    2^32 bytes of a (2200000, 512) child matrix (4.5 GB)."""
    nch, batch, nodes = 2_200_000, 512, 300
    print(f"case large csr children={nch} batch={batch}", flush=True)
    rng = np.random.default_rng(22)
    fan = O.powerlaw_fanin(nodes, seed=22)
    fan[:3] = [1, 256, 33]
    off = np.concatenate([[0], np.cumsum(fan)]).astype(np.int64)
    cids = _far_children(rng, nch, int(off[-1]), batch).astype(np.int32)
    lp = np.log(rng.random(off[-1]) + 1e-12).astype(np.float32)
    child = _randn((nch, batch), torch.float32, 23, big, scale=3.0)
    used, remap = np.unique(cids, return_inverse=True)
    ch_small = child[torch.from_numpy(used).to(big)].cpu().numpy()
    cid_small = remap.astype(np.int32)
    offd, cidd, lpd = (torch.from_numpy(a).to(big) for a in (off, cids, lp))
    ext = _ext()
    out = ext.sparse_csr_forward(child, offd, cidd, lpd)
    want = O.sparse_csr_fp64(ch_small, off, cid_small, lp)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    outq = ext.sparse_csr_forward(child, offd, cidd, lpd, q16=True)
    wq = O.sparse_q16_csr(ch_small, off, cid_small, lp)
    np.testing.assert_array_equal(outq.cpu().numpy().view(np.int32), wq.view(np.int32))
    gout = torch.randn(nodes, batch, device=big, generator=torch.Generator(device=big).manual_seed(24))
    gc, gl = ext.sparse_csr_backward(child, out, gout, offd, cidd, lpd)
    wgc, wgl = O.sparse_csr_bwd_fp64(ch_small, out.cpu().numpy(), gout.cpu().numpy(), off, cid_small, lp)
    np.testing.assert_allclose(gc[torch.from_numpy(used).to(big)].cpu().numpy(), wgc, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(gl.cpu().numpy(), wgl, rtol=1e-4, atol=1e-4)
    # rows no edge reaches stay zero
    assert int(gc.abs().sum(1).count_nonzero()) <= len(used)


def test_sparse_blocked_elements_past_4g_bytes(big):
    """Block-layout forward (fp32 product and Q16) reading element rows past
    2^32 bytes of a (2200000, 512) element matrix (4.5 GB)."""
    nelem, batch, nb, ne, bs = 2_200_000, 512, 24, 32, 8
    print(f"case large blocked elements={nelem} batch={batch}", flush=True)
    rng = np.random.default_rng(25)
    nids = (np.arange(nb) * bs).astype(np.int64)
    cids = _far_children(rng, nelem, nb * ne, batch).astype(np.int64).reshape(nb, ne)
    nparams = 4000
    pids = rng.integers(0, nparams - bs, (nb, ne)).astype(np.int64)
    params = (rng.random(nparams) + 1e-3).astype(np.float32)
    em = _randn((nelem, batch), torch.float32, 26, big, scale=3.0)
    used, remap = np.unique(cids, return_inverse=True)
    em_small = em[torch.from_numpy(used).to(big)].cpu().numpy()
    cids_small = remap.reshape(nb, ne).astype(np.int64)
    d_nids, d_cids, d_pids, d_params = (torch.from_numpy(a).to(big) for a in (nids, cids, pids, params))
    nm0 = np.full((nb * bs, batch), 7.0, np.float32)
    ext = _ext()
    nm = torch.from_numpy(nm0.copy()).to(big)
    ext.sparse_forward_float(nm, em, d_params, d_nids, d_cids, d_pids, bs)
    rows, vals = O.sparse_blocked_fp64(em_small, params, nids, cids_small, pids, bs)
    np.testing.assert_allclose(nm.cpu().numpy()[rows], vals, rtol=1e-5, atol=1e-6)
    logw_full = np.log(params.astype(np.float64)).astype(np.float32)
    logw = np.stack([np.stack([logw_full[pids[j] + p] for p in range(bs)]) for j in range(nb)])
    nmq = torch.from_numpy(nm0.copy()).to(big)
    ext.sparse_forward_q16(nmq, em, torch.from_numpy(logw_full).to(big), d_nids, d_cids, d_pids, bs,
                           params_are_log=True)
    want = O.sparse_q16_blocked(nm0, em_small, logw, nids, cids_small, bs)
    np.testing.assert_array_equal(nmq.cpu().numpy().view(np.int32), want.view(np.int32))
