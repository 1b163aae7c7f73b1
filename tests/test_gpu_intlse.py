"""GPU parity of the IntLSE kernels: bit-exact against the oracle's
restatement of the reference GPU tree (intlse/gpu/lse_kernel.cu:67-159,
lse_kernel_q10_6.cu:55-139), on float outputs and on the raw fixed-point
accumulators, through the C ABI via fuselse_amd.ext."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


def _offset_view(a: np.ndarray, dev, elem_offset: int) -> torch.Tensor:
    t = torch.from_numpy(a)
    B, N = a.shape
    buf = torch.empty(B * N + elem_offset + 8, dtype=t.dtype, device=dev)
    v = buf[elem_offset:elem_offset + B * N].view(B, N)
    v.copy_(t.to(dev))
    return v


def _run(fn, xd):
    acc = torch.empty(xd.shape[0], dtype=torch.int32, device=xd.device)
    out = fn(xd, acc_out=acc)
    return out.cpu().numpy(), acc.cpu().numpy()


def _assert_bits(out, acc, want_out, want_acc):
    np.testing.assert_array_equal(acc, want_acc)
    np.testing.assert_array_equal(out.view(np.int32), want_out.view(np.int32))


SHAPES = [(1, 1), (3, 2), (5, 7), (4, 64), (7, 1023), (3, 1024), (2, 4097), (5, 20000), (2, 128256), (3, 300001)]


@pytest.mark.parametrize("B,N", SHAPES)
@pytest.mark.parametrize("use_lut", [True, False])
def test_q16_f32_bit_exact(cuda, B, N, use_lut):
    print(f"case q16_f32 B={B} N={N} lut={use_lut}", flush=True)
    rng = np.random.default_rng(N * 7 + B)
    x = (rng.random((B, N), dtype=np.float32) * np.float32(100.0) - np.float32(100.0))
    xd = torch.from_numpy(x).to(cuda)
    fn = _ext().batched_logsumexp if use_lut else _ext().batched_logsumexp_nolut
    out, acc = _run(fn, xd)
    want, want_acc = O.q16_gpu_rows(x, base_mod=xd.data_ptr() & 15, use_lut=use_lut, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("elem_offset", [1, 2, 3])
@pytest.mark.parametrize("B,N", [(4, 3), (6, 9), (5, 1001), (3, 33333)])
def test_q16_f32_prefix_rows(cuda, B, N, elem_offset):
    """Row starts off a 16-byte boundary: prefix elements go to threads 0..p-1."""
    print(f"case q16_f32 prefix B={B} N={N} off={elem_offset}", flush=True)
    rng = np.random.default_rng(elem_offset + N)
    x = (rng.standard_normal((B, N)) * 4).astype(np.float32)
    xd = _offset_view(x, cuda, elem_offset)
    assert xd.data_ptr() % 16 != 0
    out, acc = _run(_ext().batched_logsumexp, xd)
    want, want_acc = O.q16_gpu_rows(x, base_mod=xd.data_ptr() & 15, raw=True)
    _assert_bits(out, acc, want, want_acc)


def test_q16_f32_special_values(cuda):
    """Saturation (|x*CONV| >= 2^31), NaN -> 0, -inf, wrapped differences."""
    print("case q16_f32 specials", flush=True)
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((8, 3000)) * 3).astype(np.float32)
    x[0, 5] = np.nan
    x[1, ::17] = -np.inf
    x[2, 7] = np.inf
    x[3, 0] = 4e9
    x[3, 1] = -4e9
    x[4, :] = -3e4
    x[5, 100] = 3e4
    x[6, :] = 0.0
    x[7, :] = 2.5 / np.float32(O.Q16_CONV)  # ties in the quantiser
    xd = torch.from_numpy(x).to(cuda)
    out, acc = _run(_ext().batched_logsumexp, xd)
    want, want_acc = O.q16_gpu_rows(x, base_mod=xd.data_ptr() & 15, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("B,N", [(3, 5), (16, 4096), (512, 128256)])
def test_q16_i32_bit_exact(cuda, B, N):
    """Benchmark config C4: Q16.16 int32 input quantised from N(0, 2^2) with saturation."""
    print(f"case q16_i32 B={B} N={N}", flush=True)
    rng = np.random.default_rng(B + N)
    x = (rng.standard_normal((B, N), dtype=np.float32) * np.float32(2.0))
    q = O.to_q16(x)
    qd = torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q16_i32, qd)
    want, want_acc = O.q16_gpu_rows(q, base_mod=qd.data_ptr() & 15, raw=True)
    _assert_bits(out, acc, want, want_acc)
    # the fp32-input kernel quantises the same way in-kernel
    out2, acc2 = _run(_ext().batched_logsumexp, torch.from_numpy(x).to(cuda))
    np.testing.assert_array_equal(acc2, acc)


def test_q16_i32_extreme_values(cuda):
    rng = np.random.default_rng(9)
    q = rng.integers(-2 ** 31, 2 ** 31, (6, 5000), dtype=np.int64).astype(np.int32)
    q[0, :] = 2 ** 31 - 1
    q[1, :] = -2 ** 31
    q[2, :] = O.GPU_NEG_INF
    qd = torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q16_i32, qd)
    want, want_acc = O.q16_gpu_rows(q, base_mod=qd.data_ptr() & 15, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("B,N", [(2, 1), (3, 6), (9, 64), (5, 1001), (1024, 32000), (2, 128256)])
def test_q10_6_bit_exact(cuda, B, N):
    """Benchmark config C4: Q10.6 int16 input from N(0, 2^2) through to_q10_6."""
    print(f"case q10_6 B={B} N={N}", flush=True)
    rng = np.random.default_rng(N)
    x = (rng.standard_normal((B, N), dtype=np.float32) * np.float32(2.0))
    q = O.to_q10_6(x)
    qd = torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 7, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("elem_offset", [1, 2, 3, 5])
def test_q10_6_prefix_and_extremes(cuda, elem_offset):
    print(f"case q10_6 prefix off={elem_offset}", flush=True)
    rng = np.random.default_rng(elem_offset)
    q = rng.integers(-32768, 32768, (7, 3001)).astype(np.int16)
    q[0, :] = 32767
    q[1, :] = -32768
    q[2, ::2] = -32768
    qd = _offset_view(q, cuda, elem_offset)
    out, acc = _run(_ext().batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 7, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("B,N", [(1, 8), (3, 1024), (5, 1032), (2, 4104), (511, 2048), (600, 1040), (1030, 3200)])
@pytest.mark.parametrize("elem_offset", [0, 5, 6, 7])
def test_q10_6_rows_and_prefixes(cuda, B, N, elem_offset):
    """Rows of whole 16-byte multiples with prefixes of 0..3 elements (row
    starts 0, 10, 12 and 14 bytes past a 256-byte boundary), rows with and
    without extra chunks (n4 % 256) and with no whole 256-chunk round
    (n4 < 256), saturated entries, against the oracle's tree bit for bit."""
    print(f"case q10_6 rows B={B} N={N} off={elem_offset}", flush=True)
    rng = np.random.default_rng(B * 131 + N + elem_offset)
    x = (rng.standard_normal((B, N), dtype=np.float32) * np.float32(2.0))
    q = O.to_q10_6(x)
    q[0, ::5] = 32767
    if B > 2:
        q[1, :] = -32768
        q[2, 1::3] = -32768
    qd = _offset_view(q, cuda, elem_offset) if elem_offset else torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 7, raw=True)
    _assert_bits(out, acc, want, want_acc)


@pytest.mark.parametrize("B,N", [(2048, 8), (2048, 1032), (2050, 2056), (4096, 4096), (2048, 32768), (2048, 32000)])
@pytest.mark.parametrize("elem_offset", [0, 8, 4])
def test_q10_6_many_short_rows(cuda, B, N, elem_offset):
    """Many rows of at most 32768 elements, N a multiple of 8: on 16-byte
    aligned storage (offsets 0 and 8 elements) these take the kernel whose
    threads hold two virtual threads each; at 4 elements (8 bytes) the
    one-virtual-thread kernel.  Rows with no whole 256-chunk round, with
    extra chunks and with whole rounds only; saturated entries; against the
    oracle's tree bit for bit."""
    print(f"case q10_6 many rows B={B} N={N} off={elem_offset}", flush=True)
    rng = np.random.default_rng(B * 7 + N + elem_offset)
    x = (rng.standard_normal((B, N), dtype=np.float32) * np.float32(2.0))
    q = O.to_q10_6(x)
    q[0, ::5] = 32767
    q[1, :] = -32768
    q[2, 1::3] = -32768
    qd = _offset_view(q, cuda, elem_offset) if elem_offset else torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 7, raw=True)
    _assert_bits(out, acc, want, want_acc)


def test_q10_6_published_shape(cuda):
    """The reference's published reduced-bit shape (512, 128256) with its
    U(-100, 0) inputs (reduced_bit/run_bench.py:58-71)."""
    print("case q10_6 512x128256 U(-100,0)", flush=True)
    rng = np.random.default_rng(42)
    x = (rng.random((512, 128256), dtype=np.float32) * np.float32(100.0) - np.float32(100.0))
    q = O.to_q10_6(x)
    qd = torch.from_numpy(q).to(cuda)
    out, acc = _run(_ext().batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 7, raw=True)
    _assert_bits(out, acc, want, want_acc)


def test_intlse_messages_and_empty(cuda):
    ext = _ext()
    with pytest.raises(RuntimeError, match="Input must be int16"):
        ext.batched_logsumexp_q10_6(torch.zeros(2, 3, dtype=torch.int32, device=cuda))
    with pytest.raises(RuntimeError, match="Expected 2-D tensor"):
        ext.batched_logsumexp(torch.zeros(3, device=cuda))
    assert ext.batched_logsumexp(torch.zeros(0, 5, device=cuda)).shape == (0,)


def test_acc_out_rejected_when_short(cuda):
    """The kernels write acc_out[r] for every row, so a buffer shorter than B
    (or of the wrong type) is rejected before any launch."""
    xd = torch.zeros((8, 64), dtype=torch.float32, device=cuda)
    for bad in (torch.empty(7, dtype=torch.int32, device=cuda), torch.empty(8, dtype=torch.int64, device=cuda),
                torch.empty(8, dtype=torch.int32)):
        with pytest.raises(RuntimeError, match="acc_out"):
            _ext().batched_logsumexp(xd, acc_out=bad)
    q = torch.zeros((8, 64), dtype=torch.int16, device=cuda)
    with pytest.raises(RuntimeError, match="acc_out must hold one int32 per row"):
        _ext().batched_logsumexp_q10_6(q, acc_out=torch.empty(3, dtype=torch.int32, device=cuda))


@pytest.mark.parametrize("N", [0, 1])
def test_rows_of_zero_and_one_elements(cuda, N):
    """Rows of 0 and 1 elements: an empty row gives the tree of identities
    (the chains start at the identity and nothing is folded), a single
    element passes through the butterfly; bit for bit against the oracle."""
    print(f"case intlse rows of {N}", flush=True)
    rng = np.random.default_rng(40 + N)
    x = (rng.standard_normal((5, N)) * 3).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    ext = _ext()
    for fn, lut in ((ext.batched_logsumexp, True), (ext.batched_logsumexp_nolut, False)):
        out, acc = _run(fn, xd)
        want, want_acc = O.q16_gpu_rows(x, base_mod=xd.data_ptr() & 15, use_lut=lut, raw=True)
        _assert_bits(out, acc, want, want_acc)
    q = O.to_q10_6(x)
    qd = torch.from_numpy(q).to(cuda)
    out, acc = _run(ext.batched_logsumexp_q10_6, qd)
    want, want_acc = O.q10_6_rows(q, base_mod=qd.data_ptr() & 15, raw=True)
    _assert_bits(out, acc, want, want_acc)
