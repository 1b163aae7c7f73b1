"""GPU parity of the fused selective log-softmax (forward: target logit minus
row LSE in one pass; backward: g * (onehot - softmax) in one pass) against
the fp64 oracle, through the C ABI via fuselse_amd.ext and the
make_selective_log_softmax drop-in.

Tolerances: lse within 1e-5 relative (the fp32 LSE bar).  logp = x_t - lse
can cancel to near zero, so its bound is absolute, 1e-5 * (|lse| + 1).  The
gradient is within 1e-5 relative of each element plus 1e-6 * |g| absolute
(the target column is g * (1 - p_t), which can cancel).
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


def _check_fwd(logp, lse, x, idx):
    want_lp, want_lse = O.selective_logsoftmax_fp64(x, idx)
    np.testing.assert_allclose(np.asarray(lse, np.float64), want_lse, rtol=1e-5, atol=1e-6, equal_nan=True)
    tol = 1e-5 * (np.abs(np.nan_to_num(want_lse, posinf=0, neginf=0)) + 1.0)
    got = np.asarray(logp, np.float64)
    same_nan = np.isnan(got) == np.isnan(want_lp)
    assert same_nan.all(), np.nonzero(~same_nan)
    fin = ~np.isnan(want_lp)
    assert (np.abs(got[fin] - want_lp[fin]) <= tol[fin]).all() or np.array_equal(got[fin], want_lp[fin])


SHAPES = [(1, 2), (5, 7), (300, 1000), (33, 4097), (1023, 32000), (64, 50257), (3, 128256), (16, 128256),
          (2, 256128)]


@pytest.mark.parametrize("B,N", SHAPES)
def test_selective_fwd_matches_fp64(cuda, B, N):
    print(f"case sls_fwd B={B} N={N}", flush=True)
    rng = np.random.default_rng(B * 31 + N)
    x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
    idx = rng.integers(0, N, B)
    # make some targets the row maximum, where logp is close to zero
    if B > 2:
        idx[::3] = np.argmax(x[::3], axis=1)
    logp, lse = _ext().selective_log_softmax_float(torch.from_numpy(x).to(cuda), torch.from_numpy(idx).to(cuda))
    _check_fwd(logp.cpu().numpy(), lse.cpu().numpy(), x, idx)


def test_selective_fwd_special_values_and_bad_index(cuda):
    print("case sls_fwd special", flush=True)
    B, N = 6, 5000
    rng = np.random.default_rng(3)
    x = rng.standard_normal((B, N)).astype(np.float32)
    x[0, :] = -np.inf                 # all -inf: lse -inf, logp NaN
    x[1, 17] = np.inf                 # +inf target in a +inf row: NaN
    x[2, 17] = np.inf                 # +inf elsewhere: logp -inf
    x[3, 100] = np.nan                # NaN row: NaN
    idx = np.array([5, 17, 3, 4, -1, N])   # rows 4 and 5: index out of range -> NaN
    logp, lse = _ext().selective_log_softmax_float(torch.from_numpy(x).to(cuda), torch.from_numpy(idx).to(cuda))
    lp, ls = logp.cpu().numpy(), lse.cpu().numpy()
    # trl's fp32 branch: gather minus torch.logsumexp (not log_softmax, which
    # turns a whole row holding +inf into NaN)
    xt = torch.from_numpy(x[:4]).double()
    tl = xt.gather(-1, torch.from_numpy(idx[:4])[:, None])[:, 0] - torch.logsumexp(xt, -1)
    assert ls[0] == -np.inf and np.isnan(lp[0]) and np.isnan(tl[0].item())
    assert ls[1] == np.inf and np.isnan(lp[1]) and np.isnan(tl[1].item())
    assert lp[2] == -np.inf and tl[2].item() == -np.inf
    assert np.isnan(lp[3]) and np.isnan(tl[3].item())
    assert np.isnan(lp[4]) and np.isnan(lp[5]) and np.isfinite(ls[4]) and np.isfinite(ls[5])


@pytest.mark.parametrize("B,N", [(5, 7), (300, 1000), (64, 50257), (4, 128256), (7, 4099), (33, 260)])
def test_selective_bwd_matches_fp64(cuda, B, N):
    print(f"case sls_bwd B={B} N={N}", flush=True)
    rng = np.random.default_rng(B + 7 * N)
    x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
    idx = rng.integers(0, N, B)
    idx[0] = N - 1
    if B > 1:
        idx[1] = 0
    g = rng.standard_normal(B).astype(np.float32)
    ext = _ext()
    xd, id_ = torch.from_numpy(x).to(cuda), torch.from_numpy(idx).to(cuda)
    _, lse = ext.selective_log_softmax_float(xd, id_)
    got = ext.selective_log_softmax_float_backward(torch.from_numpy(g).to(cuda), xd, id_, lse).cpu().numpy()
    want = O.selective_logsoftmax_bwd_fp64(g, x, idx, O.lse_fp64(x))
    atol = 1e-6 * np.abs(g)[:, None] * np.ones_like(want)
    err = np.abs(got - want)
    assert (err <= 1e-5 * np.abs(want) + atol).all(), err.max()
    # each row of the gradient sums to zero (softmax sums to one)
    np.testing.assert_allclose(got.astype(np.float64).sum(axis=1), 0.0, atol=2e-5 * np.abs(g).max() + 1e-6)


@pytest.mark.parametrize("B,N", [(16, 257), (8, 50257), (6, 4098)])
def test_selective_bwd_vectors_straddling_rows(cuda, B, N):
    """Rows that are not whole 16-byte vectors over a matrix that is: the
    flat backward's vectors straddle row ends.  Targets sit at the last and
    first column of neighbouring rows, so the one-hot term lands in the
    straddling vectors on both sides."""
    print(f"case sls_bwd straddling B={B} N={N}", flush=True)
    assert (B * N) % 4 == 0 and N % 4 != 0
    rng = np.random.default_rng(B * 3 + N)
    x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
    idx = np.where(np.arange(B) % 2 == 0, N - 1, 0).astype(np.int64)
    idx[-1] = rng.integers(0, N)
    g = rng.standard_normal(B).astype(np.float32)
    ext = _ext()
    xd, id_ = torch.from_numpy(x).to(cuda), torch.from_numpy(idx).to(cuda)
    _, lse = ext.selective_log_softmax_float(xd, id_)
    got = ext.selective_log_softmax_float_backward(torch.from_numpy(g).to(cuda), xd, id_, lse).cpu().numpy()
    want = O.selective_logsoftmax_bwd_fp64(g, x, idx, O.lse_fp64(x))
    atol = 1e-6 * np.abs(g)[:, None] * np.ones_like(want)
    err = np.abs(got - want)
    assert (err <= 1e-5 * np.abs(want) + atol).all(), err.max()
    np.testing.assert_allclose(got.astype(np.float64).sum(axis=1), 0.0, atol=2e-5 * np.abs(g).max() + 1e-6)


def test_selective_bwd_unaligned_offsets(cuda):
    """Rows of odd length (scalar head and tail) and an x / grad_x pair of
    different 16-byte alignment (scalar kernel)."""
    print("case sls_bwd unaligned", flush=True)
    ext = _ext()
    B, N = 9, 2051
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    idx = np.array([0, 1, 2, 3, N - 1, N - 2, N - 3, 1000, 2047])
    g = rng.standard_normal(B).astype(np.float32)
    buf = torch.empty(B * N + 3, device=cuda)
    xv = buf[1:1 + B * N].view(B, N)
    xv.copy_(torch.from_numpy(x).to(cuda))
    id_ = torch.from_numpy(idx).to(cuda)
    _, lse = ext.selective_log_softmax_float(xv, id_)
    got = ext.selective_log_softmax_float_backward(torch.from_numpy(g).to(cuda), xv, id_, lse).cpu().numpy()
    want = O.selective_logsoftmax_bwd_fp64(g, x, idx, O.lse_fp64(x))
    assert (np.abs(got - want) <= 1e-5 * np.abs(want) + 1e-6 * np.abs(g)[:, None]).all()


def test_selective_dropin_autograd_3d(cuda):
    """trl's call shape: logits (B, T-1, V), index (B, T-1); the result and the
    gradient against torch autograd of log_softmax + gather in fp64."""
    print("case sls drop-in 3d", flush=True)
    import fuselse_amd

    rng = np.random.default_rng(6)
    Bt, T, V = 2, 33, 5003
    x = (rng.standard_normal((Bt, T, V)) * 2).astype(np.float32)
    idx = rng.integers(0, V, (Bt, T))
    w = rng.standard_normal((Bt, T)).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda).requires_grad_(True)
    y = fuselse_amd.selective_log_softmax(xd, torch.from_numpy(idx).to(cuda))
    (y * torch.from_numpy(w).to(cuda)).sum().backward()
    xr = torch.from_numpy(x).double().requires_grad_(True)
    ref = torch.log_softmax(xr, -1).gather(-1, torch.from_numpy(idx)[..., None])[..., 0]
    (ref * torch.from_numpy(w).double()).sum().backward()
    lse = torch.logsumexp(xr.detach(), -1).numpy()
    assert np.all(np.abs(y.detach().cpu().numpy() - ref.detach().numpy()) <= 1e-5 * (np.abs(lse) + 1))
    gw = np.abs(w)[..., None]
    err = np.abs(xd.grad.cpu().numpy() - xr.grad.numpy())
    assert (err <= 1e-5 * np.abs(xr.grad.numpy()) + 1e-6 * gw).all(), err.max()


def test_selective_split_path_small_b(cuda):
    """Few long rows take the split kernels with the selective output."""
    print("case sls split", flush=True)
    from fuselse_amd import _lib

    assert _lib.load().fl_lse_fwd_workspace_bytes(3, 128256, 4) > 0
    rng = np.random.default_rng(8)
    x = O.make_c2_input(3, 128256, seed=4)
    idx = np.array([0, 128255, int(np.argmax(x[2]))])
    logp, lse = _ext().selective_log_softmax_float(torch.from_numpy(x).to(cuda), torch.from_numpy(idx).to(cuda))
    _check_fwd(logp.cpu().numpy(), lse.cpu().numpy(), x, idx)
    del rng


@pytest.mark.parametrize("Bt,T,V", [(3, 34, 5003), (2, 400, 32000), (4, 9, 128256)])
def test_selective_dropin_on_trl_slice(cuda, Bt, T, V):
    """trl's actual argument, logits[:, :-1, :] (not contiguous): one launch per
    leading slice on views of the caller's tensor.  Result and gradient
    against torch autograd in fp64, and the gradient is the input's shape."""
    print(f"case sls drop-in trl slice {Bt}x{T}x{V}", flush=True)
    import fuselse_amd

    rng = np.random.default_rng(T)
    x = (rng.standard_normal((Bt, T, V)) * 2).astype(np.float32)
    idx = rng.integers(0, V, (Bt, T - 1))
    w = rng.standard_normal((Bt, T - 1)).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda).requires_grad_(True)
    view = xd[:, :-1, :]
    assert not view.is_contiguous()
    y = fuselse_amd.selective_log_softmax(view, torch.from_numpy(idx).to(cuda))
    (y * torch.from_numpy(w).to(cuda)).sum().backward()
    xr = torch.from_numpy(x).double().requires_grad_(True)
    ref = torch.log_softmax(xr[:, :-1, :], -1).gather(-1, torch.from_numpy(idx)[..., None])[..., 0]
    (ref * torch.from_numpy(w).double()).sum().backward()
    lse = torch.logsumexp(xr.detach()[:, :-1, :], -1).numpy()
    assert np.all(np.abs(y.detach().cpu().numpy() - ref.detach().numpy()) <= 1e-5 * (np.abs(lse) + 1))
    g = xd.grad.cpu().numpy()
    assert (g[:, -1, :] == 0).all()
    gw = np.abs(w)[..., None]
    err = np.abs(g[:, :-1, :] - xr.grad.numpy()[:, :-1, :])
    assert (err <= 1e-5 * np.abs(xr.grad.numpy()[:, :-1, :]) + 1e-6 * gw).all(), err.max()
    with torch.no_grad():
        y2 = fuselse_amd.selective_log_softmax(view, torch.from_numpy(idx).to(cuda))
        y3 = fuselse_amd.selective_log_softmax(view.contiguous(), torch.from_numpy(idx).to(cuda))
    torch.testing.assert_close(y2, y3, rtol=1e-6, atol=1e-6)
