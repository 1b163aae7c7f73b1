"""GPU parity of the float kernels (fp32 forward, robust forward, fused
backward, fp16/bf16 forward) against the fp64 oracle and torch's fp32
logsumexp, through the C ABI via fuselse_amd.ext.

Tolerances (stated by the north star): fp32 within 1e-5 relative, fp16/bf16
inputs within 1e-3 relative of the fp32 LSE of the same (rounded) inputs.
"""

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


def _offset_view(x_cpu: torch.Tensor, dev, elem_offset: int) -> torch.Tensor:
    """Contiguous (B, N) device tensor whose data pointer sits elem_offset
    elements past a 256-byte boundary (exercises the unaligned head path)."""
    B, N = x_cpu.shape
    buf = torch.empty(B * N + elem_offset + 8, dtype=x_cpu.dtype, device=dev)
    v = buf[elem_offset:elem_offset + B * N].view(B, N)
    v.copy_(x_cpu.to(dev))
    assert v.is_contiguous()
    return v


def _close(got, want, rtol, atol=0.0):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol, equal_nan=True)


SHAPES = [(1, 2), (5, 3), (32, 256), (200, 1000), (7, 1023), (33, 4097), (16, 16384), (9, 16385),
          (3, 50257), (4, 128256), (2, 300001)]


@pytest.mark.parametrize("B,N", SHAPES)
@pytest.mark.parametrize("robust", [False, True])
def test_fwd_f32_matches_fp64(cuda, B, N, robust):
    print(f"case fwd_f32 B={B} N={N} robust={robust}", flush=True)
    rng = np.random.default_rng(B * 1000 + N)
    x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
    ext = _ext()
    fn = ext.onepass_lse_float_robust if robust else ext.onepass_lse_float
    got = fn(torch.from_numpy(x).to(cuda)).cpu().numpy()
    want = O.lse_fp64(x)
    _close(got, want, RTOL32, atol=1e-6)
    # torch fp32 on the same device agrees to the same tolerance
    tor = torch.logsumexp(torch.from_numpy(x).to(cuda), dim=-1).cpu().numpy()
    _close(got, tor, RTOL32, atol=2e-6)


@pytest.mark.parametrize("elem_offset", [1, 2, 3])
@pytest.mark.parametrize("B,N", [(6, 7), (5, 1001), (3, 20000)])
def test_fwd_f32_unaligned_rows(cuda, B, N, elem_offset):
    print(f"case fwd_f32_unaligned B={B} N={N} off={elem_offset}", flush=True)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    v = _offset_view(torch.from_numpy(x), cuda, elem_offset)
    got = _ext().onepass_lse_float_robust(v).cpu().numpy()
    _close(got, O.lse_fp64(x), RTOL32, atol=1e-6)


def test_fwd_f32_c2_full_size(cuda):
    """Benchmark config C2 forward at (512, 128256): N(0, 3^2) with 0.1% +15 spikes."""
    print("case fwd_f32 C2 512x128256", flush=True)
    x = O.make_c2_input(512, 128256, seed=0)
    xd = torch.from_numpy(x).to(cuda)
    got = _ext().onepass_lse_float_robust(xd).cpu().numpy()
    _close(got, O.lse_fp64(x), RTOL32)
    got2 = _ext().onepass_lse_float(xd).cpu().numpy()
    _close(got2, O.lse_fp64(x), RTOL32)


def test_bwd_f32_c2_full_size(cuda):
    """Benchmark config C2 fused backward at (512, 128256) with g ~ N(0, 1), the
    bench's workload (fused_fp32_kernel.cu:135-150): every element against
    g * exp(x - lse) in fp64, and each row's sum against g."""
    print("case bwd_f32 C2 512x128256", flush=True)
    x = O.make_c2_input(512, 128256, seed=0)
    g = np.random.default_rng(1).standard_normal(512).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    want = O.lse_bwd_fp64(g, x, O.lse_fp64(x))
    np.testing.assert_allclose(gx, want, rtol=RTOL32, atol=1e-30)
    np.testing.assert_allclose(gx.astype(np.float64).sum(1), g, rtol=1e-4, atol=1e-6)


def test_f32_c2_robust_set_full_size(cuda):
    """Benchmark config C2 robust set at (512, 128256), the shape and kernel the bench
    times: 1% of rows with 10% -inf entries, an all -inf row, a +inf row, a NaN
    row, a row with +inf and -inf.  Forward against fp64 and torch with
    torch.logsumexp's special values; fused backward against g * exp(x - lse)
    in fp64 and torch autograd (NaN where torch gives NaN)."""
    print("case fwd+bwd_f32 C2 robust set 512x128256", flush=True)
    x = O.make_robust_rows(O.make_c2_input(512, 128256, seed=0), seed=1)
    g = np.random.default_rng(2).standard_normal(512).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    got = lse.cpu().numpy()
    want = O.lse_fp64(x)
    assert np.isneginf(got[0]) and np.isposinf(got[1]) and np.isnan(got[2]) and np.isposinf(got[3])
    _close(got, want, RTOL32)
    _close(got, torch.logsumexp(xd, dim=-1).cpu().numpy(), RTOL32, atol=2e-6)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    np.testing.assert_allclose(gx, O.lse_bwd_fp64(g, x, want), rtol=RTOL32, atol=1e-30, equal_nan=True)
    xt = xd.clone().requires_grad_(True)
    torch.logsumexp(xt, -1).backward(torch.from_numpy(g).to(cuda))
    np.testing.assert_allclose(gx, xt.grad.cpu().numpy(), rtol=RTOL32, atol=1e-30, equal_nan=True)


def test_fwd_f32_robust_special_values(cuda):
    print("case fwd_f32 robust specials", flush=True)
    for B, N in [(8, 5), (300, 1000), (64, 128256)]:
        x = O.make_robust_rows(O.make_c2_input(B, N, seed=3), seed=B)
        got = _ext().onepass_lse_float_robust(torch.from_numpy(x).to(cuda)).cpu().numpy()
        want = O.lse_fp64(x)
        assert np.isneginf(got[0]) and np.isposinf(got[1]) and np.isnan(got[2]) and np.isposinf(got[3])
        _close(got, want, RTOL32, atol=1e-6)
        tor = torch.logsumexp(torch.from_numpy(x).to(cuda), dim=-1).cpu().numpy()
        _close(got, tor, RTOL32, atol=2e-6)


def test_fwd_f32_robust_edge_rows(cuda):
    """Rows made only of -inf, +inf, NaN, or mixes, at short and long N."""
    print("case fwd_f32 robust edge rows", flush=True)
    for N in (2, 9, 4096, 70000):
        rows = [np.full(N, -np.inf), np.full(N, np.inf), np.full(N, np.nan)]
        r = np.full(N, -np.inf); r[N // 2] = 1.5; rows.append(r)
        r = np.full(N, -np.inf); r[-1] = np.nan; rows.append(r)
        r = np.zeros(N); r[0] = np.inf; r[1] = np.nan; rows.append(r)
        r = np.full(N, 80.0); rows.append(r)
        r = np.full(N, -1e30); rows.append(r)
        x = np.stack(rows).astype(np.float32)
        got = _ext().onepass_lse_float_robust(torch.from_numpy(x).to(cuda)).cpu().numpy()
        _close(got, O.lse_fp64(x), RTOL32, atol=1e-6)


@pytest.mark.parametrize("B,N", [(1, 2), (32, 256), (200, 1000), (8, 1023), (16, 4099), (64, 128256), (3, 50257)])
def test_bwd_f32_matches_fp64(cuda, B, N):
    print(f"case bwd_f32 B={B} N={N}", flush=True)
    rng = np.random.default_rng(N)
    x = O.make_c2_input(B, N, seed=N)
    g = rng.standard_normal(B).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    want = O.lse_bwd_fp64(g, x, O.lse_fp64(x))
    np.testing.assert_allclose(gx, want, rtol=RTOL32, atol=1e-30)
    # each row of softmax sums to 1: rows of grad sum to g
    np.testing.assert_allclose(gx.astype(np.float64).sum(1), g, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("B,N,off", [(7, 256, 0), (5, 300, 0), (3, 1000, 4), (1, 4096, 0), (33, 260, 0),
                                     (2, 262144, 516)])
def test_bwd_f32_flat(cuda, B, N, off):
    """Rows of 16-byte multiples from 1 KB up: the backward walks the matrix as
    one flat run of 1 KB chunks, a chunk spanning two rows where rows are not
    1 KB multiples, the last chunk partial."""
    print(f"case bwd_f32 flat B={B} N={N} off={off}", flush=True)
    rng = np.random.default_rng(B * 7 + N + off)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    g = rng.standard_normal(B).astype(np.float32)
    xd = _offset_view(torch.from_numpy(x), cuda, off)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    np.testing.assert_allclose(gx, O.lse_bwd_fp64(g, x, O.lse_fp64(x)), rtol=RTOL32, atol=1e-30)


@pytest.mark.parametrize("B,N", [(16, 257), (8, 1023), (4, 50257), (12, 32001), (6, 4098)])
def test_bwd_f32_flat_vectors_straddling_rows(cuda, B, N):
    """Rows of 1 KB or more that are not whole 16-byte vectors, over a matrix
    that is: the flat backward's vectors then hold the end of one row and the
    start of the next, and each element takes its own row's gradient and LSE
    (rows of 257 put a boundary inside almost every block)."""
    print(f"case bwd_f32 straddling B={B} N={N}", flush=True)
    assert (B * N) % 4 == 0 and N % 4 != 0 and N * 4 >= 1024
    rng = np.random.default_rng(B * 5 + N)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    x[1::2] += 40.0  # neighbouring rows at very different LSE levels
    g = rng.standard_normal(B).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    np.testing.assert_allclose(gx, O.lse_bwd_fp64(g, x, O.lse_fp64(x)), rtol=RTOL32, atol=1e-30)
    np.testing.assert_allclose(gx.astype(np.float64).sum(1), g, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("N,off", [(131073, 0), (131073, 4), (131073, 516), (40001, 0), (40001, 260), (32781, 8)])
def test_bwd_f32_row_granules(cuda, N, off):
    """Rows of at least 32 chunks that are not 16-byte multiples, so that
    their 4 KB granules fall anywhere in the row (x starts `off` elements past
    a 256-byte boundary): the backward's chunks follow absolute 4 KB
    boundaries, with a partial chunk at both ends of each row."""
    print(f"case bwd_f32 granules N={N} off={off}", flush=True)
    B = 3
    rng = np.random.default_rng(N + off)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    g = rng.standard_normal(B).astype(np.float32)
    xd = _offset_view(torch.from_numpy(x), cuda, off)
    ext = _ext()
    lse = ext.onepass_lse_float_robust(xd)
    gx = ext.onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    np.testing.assert_allclose(gx, O.lse_bwd_fp64(g, x, O.lse_fp64(x)), rtol=RTOL32, atol=1e-30)


def test_bwd_f32_unaligned_and_mismatched(cuda):
    print("case bwd_f32 unaligned", flush=True)
    rng = np.random.default_rng(11)
    for B, N, off in [(5, 1001, 1), (4, 9000, 3), (3, 7, 2)]:
        x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
        g = rng.standard_normal(B).astype(np.float32)
        xd = _offset_view(torch.from_numpy(x), cuda, off)  # grad buffer is aligned: scalar path
        lse = _ext().onepass_lse_float_robust(xd)
        gx = _ext().onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
        np.testing.assert_allclose(gx, O.lse_bwd_fp64(g, x, O.lse_fp64(x)), rtol=RTOL32, atol=1e-30)


@pytest.mark.parametrize("N", [300, 257, 1023])
def test_bwd_f32_special_rows(cuda, N):
    """All -inf row -> NaN gradient (torch's grad*exp(x-result)); +inf row.
    N = 257 and 1023 run the flat backward with vectors straddling rows, so
    special rows meet ordinary ones inside one vector."""
    print(f"case bwd_f32 special rows N={N}", flush=True)
    x = O.make_robust_rows(O.make_c2_input(8, N, seed=5), seed=8)
    g = np.ones(8, np.float32)
    xd = torch.from_numpy(x).to(cuda)
    lse = _ext().onepass_lse_float_robust(xd)
    gx = _ext().onepass_lse_float_backward(torch.from_numpy(g).to(cuda), xd, lse).cpu().numpy()
    want = O.lse_bwd_fp64(g, x, O.lse_fp64(x))
    np.testing.assert_allclose(gx, want, rtol=RTOL32, atol=1e-30, equal_nan=True)
    xt = torch.from_numpy(x).to(cuda).requires_grad_(True)
    torch.logsumexp(xt, -1).sum().backward()
    np.testing.assert_allclose(gx, xt.grad.cpu().numpy(), rtol=RTOL32, atol=1e-30, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N", [(4, 3), (65536, 256), (64, 32000), (16, 128256), (5, 50257), (100, 1000)])
def test_fwd_half_matches_fp64(cuda, dtype, B, N):
    print(f"case fwd_half {dtype} B={B} N={N}", flush=True)
    rng = np.random.default_rng(N + B)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    xh = torch.from_numpy(x).to(dtype)
    xf = xh.float().numpy()  # the values the kernel sees
    ext = _ext()
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    got = fn(xh.to(cuda)).cpu().numpy()
    assert got.dtype == np.float32
    want = O.lse_fp64(xf)
    _close(got, want, RTOL16)
    # fp32 accumulation: in fact far inside 1e-3
    _close(got, want, 2e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N,step", [(4096, 32000, 1), (2048, 128256, 7)])
def test_fwd_half_c3_full_size(cuda, dtype, B, N, step):
    """Benchmark config C3 shapes at full size, x ~ N(0, 2^2) cast from fp32 (the bench's
    recipe).  The kernel runs over the whole matrix; every step-th row is
    checked against fp64 of the rounded inputs (all rows at (4096, 32000))."""
    print(f"case fwd_half C3 {dtype} {B}x{N}", flush=True)
    x = (np.random.default_rng(B + N).standard_normal((B, N), dtype=np.float32) * np.float32(2.0))
    xh = torch.from_numpy(x).to(dtype)
    ext = _ext()
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    got = fn(xh.to(cuda)).cpu().numpy()
    rows = np.arange(0, B, step)
    want = O.lse_fp64(xh[rows].float().numpy())
    _close(got[rows], want, RTOL16)
    _close(got[rows], want, 2e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fwd_half_unaligned(cuda, dtype):
    print(f"case fwd_half unaligned {dtype}", flush=True)
    rng = np.random.default_rng(3)
    for B, N, off in [(5, 9, 1), (4, 1001, 3), (3, 20001, 5)]:
        x = torch.from_numpy((rng.standard_normal((B, N)) * 2).astype(np.float32)).to(dtype)
        v = _offset_view(x, cuda, off)
        ext = _ext()
        fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
        got = fn(v).cpu().numpy()
        _close(got, O.lse_fp64(x.float().numpy()), 2e-5, atol=1e-5)


def test_dropin_autograd_matches_torch(cuda):
    """make_fuselse_logsumexp(ext) vs torch.logsumexp: forward, backward,
    keepdim, N-D input, non-contiguous input and every fallback branch."""
    print("case dropin autograd", flush=True)
    import fuselse_amd

    for robust in (True, False):
        lse = fuselse_amd.make_fuselse_logsumexp(fuselse_amd.ext, robust=robust)
        x = torch.randn(4, 6, 1000, device=cuda) * 2
        a = x.clone().requires_grad_(True)
        b = x.clone().requires_grad_(True)
        ya = lse(a, dim=-1)
        yb = torch.logsumexp(b, dim=-1)
        assert ya.shape == yb.shape == (4, 6)
        torch.testing.assert_close(ya, yb, rtol=RTOL32, atol=2e-6)
        w = torch.randn_like(ya)
        (ya * w).sum().backward()
        (yb * w).sum().backward()
        torch.testing.assert_close(a.grad, b.grad, rtol=RTOL32, atol=1e-7)
        # keepdim, 2-D direct path, non-contiguous input
        x2 = torch.randn(37, 515, device=cuda)
        torch.testing.assert_close(lse(x2, dim=1, keepdim=True), torch.logsumexp(x2, 1, keepdim=True),
                                   rtol=RTOL32, atol=2e-6)
        xt = torch.randn(515, 37, device=cuda).t()
        assert not xt.is_contiguous()
        torch.testing.assert_close(lse(xt, -1), torch.logsumexp(xt, -1), rtol=RTOL32, atol=2e-6)
        # fallbacks: other dim, dtype, N == 1
        torch.testing.assert_close(lse(x2, dim=0), torch.logsumexp(x2, 0))
        xd = x2.double()
        assert lse(xd, -1).dtype == torch.float64
        x1 = torch.randn(5, 1, device=cuda)
        torch.testing.assert_close(lse(x1, -1), torch.logsumexp(x1, -1))
        # empty batch
        assert lse(torch.empty(0, 8, device=cuda), -1).shape == (0,)


@pytest.mark.parametrize("B,N", [(512, 128256), (1024, 20000)])
@pytest.mark.parametrize("keep", [False, True])
def test_dropin_autograd_at_size(cuda, B, N, keep):
    """The drop-in under autograd, with the plain forward (the default) and
    with keep=True (the keeping variant, which at C2, 256-thread blocks, and at
    1024 rows of 20000, 1024-thread blocks, leaves part of x for the backward):
    the forward and the gradient equal the plain ext calls bit for bit, and the
    gradient's first 64 rows match fp64."""
    import fuselse_amd

    print(f"case dropin autograd keep={keep} B={B} N={N}", flush=True)
    ext = fuselse_amd.ext
    x = O.make_c2_input(B, N, seed=11)
    g = np.random.default_rng(12).standard_normal(B).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    gd = torch.from_numpy(g).to(cuda)
    lse = fuselse_amd.make_fuselse_logsumexp(ext, robust=True, keep=keep)
    a = xd.clone().requires_grad_(True)
    y = lse(a, dim=-1)
    y.backward(gd)
    want_lse = ext.onepass_lse_float_robust(xd)
    assert torch.equal(y.detach(), want_lse)
    assert torch.equal(a.grad, ext.onepass_lse_float_backward(gd, xd, want_lse))
    rows = slice(0, 64)
    np.testing.assert_allclose(a.grad[rows].cpu().numpy(), O.lse_bwd_fp64(g[rows], x[rows], O.lse_fp64(x[rows])),
                               rtol=RTOL32, atol=1e-30)


def test_dropin_is_native(cuda):
    """The GPU drop-in path runs the native library (it is loaded in-process)."""
    import fuselse_amd
    from fuselse_amd import _lib

    x = torch.randn(8, 64, device=cuda)
    fuselse_amd.logsumexp(x)
    assert _lib._lib is not None
    maps = open("/proc/self/maps").read()
    assert "libfuselse_amd.so" in maps


# ---------------------------------------------------------------------------
# fp16 / bf16 backward (fp32 arithmetic, round to nearest even on store)
# ---------------------------------------------------------------------------
def _half_ulp(want: np.ndarray, dtype) -> np.ndarray:
    """One unit in the last place of the half type at |want| (its subnormal
    step below the normal range)."""
    a = np.abs(want)
    if dtype == torch.float16:
        e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
        return 2.0 ** (e - 10)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N,off", [(5, 7, 0), (300, 1000, 0), (64, 50257, 0), (4, 128256, 0), (7, 4099, 3),
                                     (3, 20001, 1), (3, 131072, 8), (2, 70001, 0), (2, 70001, 136), (7, 512, 0),
                                     (33, 520, 0), (5, 600, 8)])
def test_bwd_half_matches_fp64(cuda, dtype, B, N, off):
    """Within one half ulp of the fp64 value of g * exp(x - lse) on the half
    inputs (the rounding of the store), plus the fp32 arithmetic's 1e-5."""
    print(f"case bwd_half {dtype} B={B} N={N} off={off}", flush=True)
    rng = np.random.default_rng(B * 13 + N)
    xh = torch.from_numpy((rng.standard_normal((B, N)) * 2).astype(np.float32)).to(dtype)
    g = rng.standard_normal(B).astype(np.float32)
    x64 = xh.double().numpy()
    ext = _ext()
    xd = _offset_view(xh, cuda, off)
    lse = (ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16)(xd)
    got = ext.onepass_lse_half_backward(torch.from_numpy(g).to(cuda), xd, lse)
    assert got.dtype == dtype
    got = got.double().cpu().numpy()
    want = O.lse_bwd_fp64(g, x64, O.lse_fp64(x64))
    err = np.abs(got - want)
    bound = _half_ulp(want, dtype) + 1e-5 * np.abs(want)
    assert (err <= bound).all(), (err / bound).max()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N", [(16, 513), (8, 1001), (8, 50257), (4, 4098)])
def test_bwd_half_flat_vectors_straddling_rows(cuda, dtype, B, N):
    """Half rows of 1 KB or more that are not whole 16-byte vectors, the
    matrix a whole number of them: vectors straddle row ends in the flat
    backward.  Bound as in test_bwd_half_matches_fp64."""
    print(f"case bwd_half straddling {dtype} B={B} N={N}", flush=True)
    assert (B * N) % 8 == 0 and N % 8 != 0 and N * 2 >= 1024
    rng = np.random.default_rng(B * 17 + N)
    x32 = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    x32[1::2] += 30.0
    xh = torch.from_numpy(x32).to(dtype)
    g = rng.standard_normal(B).astype(np.float32)
    x64 = xh.double().numpy()
    ext = _ext()
    xd = xh.to(cuda)
    lse = (ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16)(xd)
    got = ext.onepass_lse_half_backward(torch.from_numpy(g).to(cuda), xd, lse).double().cpu().numpy()
    want = O.lse_bwd_fp64(g, x64, O.lse_fp64(x64))
    err = np.abs(got - want)
    bound = _half_ulp(want, dtype) + 1e-5 * np.abs(want)
    assert (err <= bound).all(), (err / bound).max()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dropin_half_inputs_autograd(cuda, dtype):
    print(f"case drop-in half {dtype}", flush=True)
    from fuselse_amd import make_fuselse_logsumexp

    lse_fn = make_fuselse_logsumexp(_ext(), robust=True, half_inputs=True)
    rng = np.random.default_rng(21)
    xh = torch.from_numpy((rng.standard_normal((3, 40, 3001)) * 2).astype(np.float32)).to(dtype)
    w = rng.standard_normal((3, 40)).astype(np.float32)
    xd = xh.to(cuda).requires_grad_(True)
    y = lse_fn(xd, dim=-1)
    assert y.dtype == dtype and y.shape == (3, 40)
    (y.float() * torch.from_numpy(w).to(cuda)).sum().backward()
    x64 = xh.double().numpy().reshape(120, 3001)
    want_y = O.lse_fp64(x64).reshape(3, 40)
    assert (np.abs(y.detach().double().cpu().numpy() - want_y) <= _half_ulp(want_y, dtype)).all()
    # the gradient reaching the half output is w rounded to the half dtype
    w_half = torch.from_numpy(w).to(dtype).double().numpy()
    want_g = O.lse_bwd_fp64(w_half.reshape(-1), x64, O.lse_fp64(x64)).reshape(3, 40, 3001)
    got_g = xd.grad.double().cpu().numpy()
    assert (np.abs(got_g - want_g) <= _half_ulp(want_g, dtype) + 1e-5 * np.abs(want_g)).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N", [300, 20000, 128256])
def test_fwd_half_robust_special_values(cuda, dtype, N):
    """Robust half forward (one-pass and, for few long rows, split path):
    all -inf -> -inf, any +inf -> +inf, any NaN -> NaN, as torch.logsumexp on
    the same values in fp32."""
    print(f"case fwd_half_robust {dtype} N={N}", flush=True)
    rng = np.random.default_rng(N)
    x = torch.from_numpy((rng.standard_normal((6, N)) * 2).astype(np.float32))
    x[0, :] = -float("inf")
    x[1, N // 2] = float("inf")
    x[2, N - 1] = float("nan")
    x[3, 0] = float("inf")
    x[3, N // 3] = -float("inf")
    x[4, : N - 1] = -float("inf")
    xh = x.to(dtype)
    ext = _ext()
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    got = fn(xh.to(cuda), robust=True).cpu().numpy()
    want = torch.logsumexp(xh.float(), dim=-1).numpy()
    assert got[0] == -np.inf and got[1] == np.inf and np.isnan(got[2]) and got[3] == np.inf
    _close(got[4:], want[4:], RTOL16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N,off", [(3, 9000, 0), (1024, 16000, 0), (77, 32000, 3), (5, 8193, 1)])
def test_fwd_mid_rows_block_geometry(cuda, dtype, B, N, off):
    """Few mid-length rows (1024 < vectors <= 4096, B <= 1024) take one
    128- or 256-thread block per row; parity with fp64 at the tolerance of the dtype,
    robust and plain, aligned and offset rows."""
    print(f"case fwd_mid {dtype} B={B} N={N} off={off}", flush=True)
    rng = np.random.default_rng(B + N + off)
    x32 = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    xt = torch.from_numpy(x32).to(dtype)
    xd = _offset_view(xt, cuda, off)
    ext = _ext()
    want = O.lse_fp64(xt.double().numpy())
    for robust in (False, True):
        if dtype == torch.float32:
            got = (ext.onepass_lse_float_robust if robust else ext.onepass_lse_float)(xd)
            tol = RTOL32
        else:
            fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
            got = fn(xd, robust=robust)
            tol = RTOL16
        _close(got.cpu().numpy(), want, tol, atol=1e-6)


# (dtype, label, B, vectors per row, batch size in vectors or None for the
# burst loop) for each branch of the forward launcher: long rows (fp16/bf16
# 512 x 4; fp32 512 x 2 / 256 x 2 / 1024 x 1 by row count), few mid-length
# rows (128- / 256-thread blocks), many mid-length rows (fp32 256-thread
# blocks, fp16/bf16 32 or 64 lanes per row in batches of 4), rows of a few
# vectors (4 lanes, one masked batch of 2), short rows (burst loop).
_F32, _F16, _BF16 = torch.float32, torch.float16, torch.bfloat16
GEOMETRIES = [
    (_F32, "long-blk512x2", 300, 5120, 1024),
    (_F32, "long-blk256x2", 600, 5120, 512),
    (_F32, "long-blk1024x1", 2048, 4608, 1024),
    (_F32, "mid-blk256x2", 33, 1536, 512),
    (_F32, "many-blk256x2", 1100, 1025, 512),
    (_F32, "tiny-grp4x2", 37, 8, 8),
    (_F32, "short-burst", 37, 257, None),
]
for _h in (_F16, _BF16):
    GEOMETRIES += [
        (_h, "long-blk512x4", 9, 5120, 2048),
        (_h, "mid-blk128x2", 33, 1536, 256),
        (_h, "mid-blk256x2", 33, 4096, 512),
        (_h, "many-grp32x4", 1100, 1536, 128),
        (_h, "many-grp64x4", 1100, 1025, 256),
        (_h, "tiny-grp4x2", 37, 8, 8),
        (_h, "short-burst", 37, 257, None),
    ]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fwd_half_many_rows_block_geometry(cuda, dtype):
    """fp16/bf16 rows of 2049..4096 vectors from 4096 rows take one 256-thread
    block per row in batches of 1024 vectors: rows one vector past, on and
    short of a batch boundary, on aligned and offset storage, robust and
    plain, against float64 logsumexp of the same half values."""
    ext = _ext()
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    B = 4096
    g = torch.Generator(device=cuda)
    g.manual_seed(17)
    for N in (2049 * 8 + 1, 3072 * 8 - 3, 3072 * 8, 3073 * 8 + 5, 32000):
        for off in (0, 1):
            print(f"case fwd_half_blk256x4 {dtype} B={B} N={N} off={off}", flush=True)
            buf = torch.empty(B * N + off + 8, dtype=dtype, device=cuda)
            xd = buf[off:off + B * N].view(B, N)
            xd.copy_((torch.randn(B, N, device=cuda, generator=g) * 2).to(dtype))
            want = torch.logsumexp(xd.double(), dim=1)
            for robust in (False, True):
                got = fn(xd, robust=robust).double()
                torch.testing.assert_close(got, want, rtol=RTOL16, atol=1e-6)


@pytest.mark.parametrize("dtype", [_F32, _F16, _BF16])
@pytest.mark.parametrize("lpr", [4, 8, 16, 32, 64])
def test_fwd_short_rows_burst_boundaries(cuda, dtype, lpr):
    """Short rows (16..512 vectors) take lpr lanes per row and bursts of 4
    loads per lane: whole bursts for every lane of the wave, then masked
    bursts.  Row lengths on, one vector under and one past a whole burst, and
    lengths that are no multiple of the vector width (rows of one wave then
    hold different vector counts), on aligned and offset storage, with a
    ragged last row group; robust and plain against fp64."""
    esize = torch.empty((), dtype=dtype).element_size()
    ve = 16 // esize
    burst = 4 * lpr  # vectors per whole burst of the wave's row group
    vec_counts = sorted({v for v in (burst - 1, burst, burst + 1, burst // 2 + 1, 2 * burst - 3)
                         if 16 <= v <= 512 and min(64, max(4, 1 << ((v + 3) // 4 - 1).bit_length())) == lpr})
    assert vec_counts, lpr
    ext = _ext()
    rng = np.random.default_rng(lpr * esize)
    B = 2051  # odd: the last row group of every lpr is ragged
    for vecs in vec_counts:
        for N, off in ((vecs * ve, 0), (vecs * ve, 1), (vecs * ve - 1, 0), (vecs * ve - ve // 2, 3)):
            print(f"case fwd_short_burst {dtype} lpr={lpr} B={B} N={N} off={off}", flush=True)
            xt = torch.from_numpy((rng.standard_normal((B, N)) * 2).astype(np.float32)).to(dtype)
            xd = _offset_view(xt, cuda, off)
            want = O.lse_fp64(xt.double().numpy())
            for robust in (False, True):
                if dtype == torch.float32:
                    got = (ext.onepass_lse_float_robust if robust else ext.onepass_lse_float)(xd)
                else:
                    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
                    got = fn(xd, robust=robust)
                _close(got.cpu().numpy(), want, RTOL32 if dtype == torch.float32 else RTOL16, atol=1e-6)


@pytest.mark.parametrize("dtype,label,B,vecs,step", GEOMETRIES)
def test_fwd_pipelined_batch_boundaries(cuda, dtype, label, B, vecs, step):
    """Rows that end exactly on, one vector short of, and past a batch
    boundary of each geometry, with row lengths that are not a multiple of
    the vector width (so rows of one wave start at different alignments and
    the masked last batch holds 0 .. all of a lane's vectors), on aligned and
    offset storage; robust and plain against fp64.  The no-workspace C entries
    run the one-pass geometry the label names for every B (the reference-named
    functions send some of these row counts to the split-row path); where no
    split applies, the reference-named function must give the same bits."""
    from fuselse_amd import _lib

    lib = _lib.load()
    esize = torch.empty((), dtype=dtype).element_size()
    entry = {torch.float32: "fl_lse_fwd_f32", torch.float16: "fl_lse_fwd_f16",
             torch.bfloat16: "fl_lse_fwd_bf16"}[dtype]

    def one_pass(xd, robust, name=entry):
        out = torch.empty(xd.shape[0], device=xd.device)
        _lib.call(name, xd.data_ptr(), out.data_ptr(), xd.shape[0], xd.shape[1], int(robust),
                  torch.cuda.current_stream().cuda_stream)
        return out

    ve = 16 // esize
    if step is None:
        ns = [vecs * ve, vecs * ve - 1]
    else:
        k = max(1, vecs // step)
        ns = sorted({vecs * ve, k * step * ve, k * step * ve - 1, (k * step + 1) * ve + 1, (k * step - 1) * ve + 3})
    ext = _ext()
    rng = np.random.default_rng(vecs + B)
    for N in ns:
        for off in (0, 1):
            print(f"case fwd_batches {label} {dtype} B={B} N={N} off={off}", flush=True)
            x32 = (rng.standard_normal((B, N)) * 2).astype(np.float32)
            xt = torch.from_numpy(x32).to(dtype)
            xd = _offset_view(xt, cuda, off)
            want = O.lse_fp64(xt.double().numpy())
            for robust in (False, True):
                got = one_pass(xd, robust)
                _close(got.cpu().numpy(), want, RTOL32 if dtype == torch.float32 else RTOL16, atol=1e-6)
                # the keeping forward: same kernels but for the loads' cache policy
                assert torch.equal(one_pass(xd, robust, entry + "_keep"), got)
                if lib.fl_lse_fwd_workspace_bytes(B, N, esize) == 0:
                    if dtype == torch.float32:
                        named = (ext.onepass_lse_float_robust if robust else ext.onepass_lse_float)(xd)
                    else:
                        fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
                        named = fn(xd, robust=robust)
                    assert torch.equal(named, got)


def test_rows_of_zero_and_one_elements(cuda):
    """N = 0: every forward gives -inf (torch.logsumexp over an empty dim), the
    backward entries return without launching and the selective forward gives
    NaN (no index is in range).  N = 1: lse = x and the gradient is g, up to
    the rounding of x * log2(e) in the fused exponent (a few ulp)."""
    print("case rows of 0 and 1 elements", flush=True)
    ext = _ext()
    B = 5
    for N in (0, 1):
        x = torch.randn(B, N, device=cuda) * 3
        for robust in (False, True):
            got = (ext.onepass_lse_float_robust if robust else ext.onepass_lse_float)(x)
            torch.testing.assert_close(got, torch.logsumexp(x, -1), rtol=1e-6, atol=1e-6)
            for dtype, fn in ((torch.float16, ext.batched_logsumexp_fp16), (torch.bfloat16, ext.batched_logsumexp_bf16)):
                xh = x.to(dtype)
                torch.testing.assert_close(fn(xh, robust=robust), torch.logsumexp(xh.float(), -1), rtol=1e-6, atol=1e-6)
        if N == 0:
            assert torch.isneginf(ext.onepass_lse_float(x)).all()
        g = torch.randn(B, device=cuda)
        lse = ext.onepass_lse_float_robust(x)
        gx = ext.onepass_lse_float_backward(g, x, lse)
        assert gx.shape == (B, N)
        if N == 1:
            torch.testing.assert_close(gx[:, 0], g, rtol=1e-6, atol=0.0)
            gh = ext.onepass_lse_half_backward(g, x.half(), ext.batched_logsumexp_fp16(x.half()))
            torch.testing.assert_close(gh[:, 0].float(), g.half().float(), rtol=2.0 ** -10, atol=0.0)
        idx = torch.zeros(B, dtype=torch.int64, device=cuda)
        logp, lse_s = ext.selective_log_softmax_float(x, idx)
        if N == 0:
            assert torch.isnan(logp).all() and torch.isneginf(lse_s).all()
        else:
            torch.testing.assert_close(logp, torch.zeros_like(logp), rtol=0.0, atol=1e-6)
            torch.testing.assert_close(lse_s, x[:, 0], rtol=1e-6, atol=1e-6)
            gs = ext.selective_log_softmax_float_backward(g, x, idx, lse_s)
            torch.testing.assert_close(gs, torch.zeros_like(gs), rtol=0.0, atol=1e-6)


@pytest.mark.parametrize("dtype,B,N", [(torch.float32, 512, 128256), (torch.float32, 256, 128256),
                                       (torch.float32, 1024, 20000), (torch.float32, 700, 3001),
                                       (torch.float32, 4096, 1000), (torch.bfloat16, 2048, 128256),
                                       (torch.float16, 4096, 32000), (torch.float16, 64, 3000)])
def test_fwd_keep_bit_identical(cuda, dtype, B, N):
    """fl_lse_fwd_*_keep (rows below the kept-row count load without the
    nontemporal hint) gives the bits of fl_lse_fwd_* on both sides of that
    count, robust on the C2 robust set and plain on finite rows, at
    C2, the bf16 C3 shape and the other one-block-per-row geometries (and a
    row-group shape, where the entries run the same kernel)."""
    from fuselse_amd import _lib

    print(f"case fwd_keep {dtype} B={B} N={N}", flush=True)
    entry = {torch.float32: "fl_lse_fwd_f32", torch.float16: "fl_lse_fwd_f16",
             torch.bfloat16: "fl_lse_fwd_bf16"}[dtype]
    finite = O.make_c2_input(B, N, seed=B + N)
    special = O.make_robust_rows(finite, seed=7)
    st = torch.cuda.current_stream().cuda_stream
    for data, robust in ((finite, False), (finite, True), (special, True)):
        xd = torch.from_numpy(data).to(cuda).to(dtype)
        outs = []
        for name in (entry, entry + "_keep"):
            out = torch.empty(B, device=cuda)
            _lib.call(name, xd.data_ptr(), out.data_ptr(), B, N, int(robust), st)
            outs.append(out)
        torch.testing.assert_close(outs[1], outs[0], rtol=0, atol=0, equal_nan=True)
        if data is special:
            got = outs[1].cpu().numpy()
            assert np.isneginf(got[0]) and np.isposinf(got[1]) and np.isnan(got[2]) and np.isposinf(got[3])
    ext = _ext()
    xd = torch.from_numpy(finite).to(cuda).to(dtype)
    if dtype == torch.float32:
        assert torch.equal(ext.onepass_lse_float_robust_keep(xd), ext.onepass_lse_float_robust(xd))
        assert torch.equal(ext.onepass_lse_float_keep(xd), ext.onepass_lse_float(xd))
    else:
        f, fk = ((ext.batched_logsumexp_fp16, ext.batched_logsumexp_fp16_keep) if dtype == torch.float16
                 else (ext.batched_logsumexp_bf16, ext.batched_logsumexp_bf16_keep))
        assert torch.equal(fk(xd, robust=True), f(xd, robust=True))
