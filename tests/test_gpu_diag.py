"""The measurement kernels the bench's ceilings and timings come from
(libfuselse_amd_diag.so, fuselse_amd/csrc/diag/fl_diag.hip).

They have no counterpart in the reference; these tests check that the copy
ceiling really copies, that the read ceiling reads without writing, that the
latency probe runs every kind and rejects bad arguments, and that the timed
variants of the forward and IntLSE kernels give the library's own results
with sane records."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture
def lib(cuda):
    """The library's entry points, returning their status codes."""
    from fuselse_amd import _lib

    return _lib.load_diag()


@pytest.mark.parametrize("threads,unroll", [(64, 1), (64, 2), (64, 4), (256, 1), (256, 2), (256, 4)])
def test_copy_stream_copies(cuda, lib, threads, unroll):
    """Every byte of x lands in y, for a size that is no multiple of the
    block's chunk, with more and with fewer blocks than chunks."""
    print(f"case diag_copy threads={threads} unroll={unroll}", flush=True)
    nbytes = 16 * 100003
    x = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    chunk = threads * unroll * 16
    for blocks in ((nbytes + chunk - 1) // chunk, 37):
        y = torch.zeros(nbytes + 64, dtype=torch.uint8, device=cuda)
        assert lib.fl_diag_copy_stream(x.data_ptr(), y.data_ptr(), nbytes, blocks, threads, unroll, st) == 0
        torch.cuda.synchronize()
        assert torch.equal(y[:nbytes], x)
        assert int(y[nbytes:].count_nonzero()) == 0  # nothing past the end


@pytest.mark.parametrize("threads,unroll", [(64, 2), (256, 4), (256, 8)])
def test_read_stream_reads_only(cuda, lib, threads, unroll):
    print(f"case diag_read threads={threads} unroll={unroll}", flush=True)
    x = torch.randn(4 * 100003, device=cuda)
    sink = torch.full((4,), 7, dtype=torch.int32, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_read_stream(x.data_ptr(), x.numel() * 4, 300, threads, unroll, sink.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7, 7, 7]


def test_diag_argument_checks(cuda, lib):
    x = torch.zeros(64, device=cuda)
    y = torch.zeros(64, device=cuda)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_copy_stream(x.data_ptr(), y.data_ptr(), 256, 4, 128, 1, st) != 0
    assert lib.fl_diag_copy_stream(x.data_ptr(), y.data_ptr(), 256, 4, 64, 3, st) != 0
    assert lib.fl_diag_copy_stream(x.data_ptr(), y.data_ptr(), 250, 4, 64, 1, st) != 0
    assert lib.fl_diag_read_stream(x.data_ptr(), 256, 4, 128, 1, sink.data_ptr(), st) != 0
    rec = torch.zeros(3, dtype=torch.int64, device=cuda)
    assert lib.fl_diag_chain_latency(10, 16, 1, rec.data_ptr(), st) != 0
    assert lib.fl_diag_chain_latency(0, 15, 1, rec.data_ptr(), st) != 0
    assert lib.fl_diag_chain_latency(0, 16, 17, rec.data_ptr(), st) != 0


@pytest.mark.parametrize("kind", range(10))
def test_chain_latency_kinds(cuda, lib, kind):
    """Each kind runs its chain and records positive cycle and tick counts
    for every wave."""
    print(f"case diag_latency kind={kind}", flush=True)
    waves = 4
    rec = torch.zeros(3 * waves, dtype=torch.int64, device=cuda)
    assert lib.fl_diag_chain_latency(kind, 256, waves, rec.data_ptr(), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    r = rec.view(waves, 3).cpu()
    assert (r[:, 0] > 256).all() and (r[:, 1] > 0).all()


def test_fwd_block_times_is_the_forward(cuda, lib):
    """(512, 20000) fp32 takes the 256-thread one-block-per-row geometry in
    fl_lse_fwd_f32 too: the timed kernel's results are the same bits, and
    every block's record is ordered and names its row and an XCD."""
    import fuselse_amd

    print("case diag fwd_block_times", flush=True)
    B, N = 512, 20000
    x = torch.randn(B, N, device=cuda) * 3
    out = torch.empty(B, device=cuda)
    rec = torch.zeros(6 * B, dtype=torch.int64, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_fwd_block_times(x.data_ptr(), out.data_ptr(), B, N, rec.data_ptr(), st) == 0
    assert torch.equal(out, fuselse_amd.ext.onepass_lse_float_robust(x))
    r = rec.view(B, 6).cpu()
    assert (r[:, 1] >= r[:, 0]).all() and (r[:, 2] > 0).all()
    assert ((r[:, 3] >= 0) & (r[:, 3] < 16)).all()
    assert torch.equal(r[:, 5], torch.arange(B))
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    rec.zero_()
    assert lib.fl_diag_read_rows_times(x.data_ptr(), B, N, rec.data_ptr(), sink.data_ptr(), st) == 0
    r = rec.view(B, 6).cpu()
    assert (r[:, 1] >= r[:, 0]).all() and torch.equal(r[:, 5], torch.arange(B))
    nb = x.numel() * 4 // 2048
    for every in (1, 7):
        nrec = (nb + every - 1) // every
        rec2 = torch.zeros(6 * nrec, dtype=torch.int64, device=cuda)
        assert lib.fl_diag_read_stream_times(x.data_ptr(), nb * 2048, every, rec2.data_ptr(), sink.data_ptr(), st) == 0
        r = rec2.view(nrec, 6).cpu()
        assert (r[:, 1] >= r[:, 0]).all() and torch.equal(r[:, 5], torch.arange(nrec) * every)
    assert int(sink.item()) == 0
    assert lib.fl_diag_read_stream_times(x.data_ptr(), 1000, 1, rec2.data_ptr(), sink.data_ptr(), st) != 0
    assert lib.fl_diag_read_stream_times(x.data_ptr(), 2048, 0, rec2.data_ptr(), sink.data_ptr(), st) != 0


@pytest.mark.parametrize("kind", [0, 1, 2])
def test_intlse_phases_is_the_kernel(cuda, lib, kind):
    """The phase-timed IntLSE kernels give the library's results bit for bit
    (shapes where it takes the same 256-thread kernel), and each block's
    phases are in order."""
    import fuselse_amd

    print(f"case diag intlse_phases kind={kind}", flush=True)
    ext = fuselse_amd.ext
    B, N = 300, 12345
    g = torch.Generator(device=cuda)
    g.manual_seed(kind)
    xf = torch.randn(B, N, device=cuda, generator=g) * 2
    if kind == 0:
        x, want = xf, ext.batched_logsumexp(xf)
    elif kind == 1:
        x = (xf * 94548.4609375).round().to(torch.int32)
        want = ext.batched_logsumexp_q16_i32(x)
    else:
        x = (xf * 92.33248261689366).round().clamp(-32768, 32767).to(torch.int16)
        want = ext.batched_logsumexp_q10_6(x)
    out = torch.empty(B, device=cuda)
    rec = torch.zeros(8 * B, dtype=torch.int64, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_intlse_phases(kind, x.data_ptr(), out.data_ptr(), B, N, rec.data_ptr(), st) == 0
    assert torch.equal(out.view(torch.int32), want.view(torch.int32))
    r = rec.view(B, 8).cpu()
    for a, b in ((0, 1), (1, 2), (2, 3), (3, 4)):
        assert (r[:, b] >= r[:, a]).all(), (a, b)
    assert (r[:, 5] > 0).all() and torch.equal(r[:, 7], torch.arange(B))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_rows_cap_is_the_forward(cuda, lib, dtype):
    """The half row kernel gives the library's results bit for bit at every
    cap, at (4096, 20000), a shape where the library takes that kernel."""
    import fuselse_amd

    print(f"case diag half_rows_cap {dtype}", flush=True)
    ext = fuselse_amd.ext
    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    B, N = 4096, 20000
    x = (torch.randn(B, N, device=cuda, generator=g) * 2).to(dtype)
    want = ext.batched_logsumexp_fp16(x) if dtype == torch.float16 else ext.batched_logsumexp_bf16(x)
    st = torch.cuda.current_stream().cuda_stream
    dt = 0 if dtype == torch.float16 else 1
    for cap in (0, 2, 3, 4, 8):
        out = torch.empty(B, device=cuda)
        assert lib.fl_diag_half_rows_cap(dt, x.data_ptr(), out.data_ptr(), B, N, cap, st) == 0
        assert torch.equal(out, want), cap


def test_lane_pairs_are_row_maxima(cuda, lib):
    """max_pair16 / max_pair32, the lane-swap maxima the block-layout kernels
    take their column and row maxima with, pair lane l with l ^ 16 and l ^ 32.
    The products are unchanged by the reference they are shifted by, so their
    own tests would not notice other pairs: this checks the pairs directly,
    on distinct values per lane (each 16-lane row's maximum at a different
    position) and on -inf and NaN lanes, against the maxima on the host."""
    print("case diag lane_pairs", flush=True)
    g = torch.Generator().manual_seed(3)
    cases = [torch.randperm(64, generator=g).float() - 20.0, torch.randn(64, generator=g)]
    special = torch.randn(64, generator=g)
    special[[0, 17, 33, 34, 50]] = float("-inf")
    special[[16, 48, 49]] = float("nan")
    special[[1, 2, 18, 35]] = torch.tensor([float("inf"), 0.0, -0.0, 7.0])
    cases.append(special)
    st = torch.cuda.current_stream().cuda_stream
    lanes = torch.arange(64)
    for v in cases:
        out = torch.full((192,), 123.0, device=cuda)
        assert lib.fl_diag_lane_pairs(v.to(cuda).data_ptr(), out.data_ptr(), st) == 0
        got = out.cpu()

        def fmax(a, b):  # fmaxf: a NaN operand gives the other one
            return torch.where(a.isnan(), b, torch.where(b.isnan(), a, torch.maximum(a, b)))

        p16 = fmax(v, v[lanes ^ 16])
        p32 = fmax(v, v[lanes ^ 32])
        p4 = fmax(p16, p16[lanes ^ 32])
        for name, want, have in (("16", p16, got[:64]), ("32", p32, got[64:128]), ("16+32", p4, got[128:])):
            same = (want == have) | (want.isnan() & have.isnan())
            assert bool(same.all()), (name, v, have)


@pytest.mark.parametrize("lanes,waves,policy",
                         [(16, 1, 0), (32, 1, 0), (64, 1, 0), (16, 1, 1), (16, 1, 2), (16, 1, 4), (64, 1, 5),
                          (16, 4, 2), (64, 4, 0)])
@pytest.mark.parametrize("nrows,batch", [(100, 100), (64, 512), (33, 4), (40, 1000)])
def test_gather_rows_copies(cuda, lib, nrows, batch, lanes, waves, policy):
    """The gather copy writes dst[i] = src[idx[i]] for every row and column
    (ragged row groups and column tiles, workgroups with idle waves) and
    nothing past them, at every lane geometry, workgroup size and cache
    policy."""
    print(f"case diag gather_rows {nrows}x{batch} lanes {lanes} waves {waves} policy {policy}", flush=True)
    g = torch.Generator(device=cuda)
    g.manual_seed(9)
    src = torch.randn(300, batch, device=cuda, generator=g)
    idx = torch.randint(0, 300, (nrows,), device=cuda, generator=g)
    dst = torch.full((nrows + 1, batch), 5.0, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_gather_rows(src.data_ptr(), idx.data_ptr(), dst.data_ptr(), nrows, batch, lanes, waves,
                                   policy, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(dst[:nrows], src[idx])
    assert bool((dst[nrows] == 5.0).all())


@pytest.mark.parametrize("waves,lds", [(1, 18432), (2, 0), (4, 18432)])
@pytest.mark.parametrize("nblocks,batch", [(5, 64), (12, 512), (3, 192)])
def test_blocked_bwd_pattern(cuda, lib, nblocks, batch, waves, lds):
    """The single pass's memory pattern writes, for every block edge and
    column, its child row plus the sum over the lane's eight parents of o * g
    (parents 4 ks + (e / 4) % 4), and nothing past the block's rows, at every
    workgroup size and with idle waves (batch 64 at four waves)."""
    print(f"case diag blocked_bwd_pattern {nblocks}x{batch} waves {waves} lds {lds}", flush=True)
    g = torch.Generator(device=cuda)
    g.manual_seed(11)
    nel = 70
    x = torch.randn(nel, batch, device=cuda, generator=g)
    o = torch.randn(nblocks * 32 + 8, batch, device=cuda, generator=g)
    gg = torch.randn(nblocks * 32 + 8, batch, device=cuda, generator=g)
    nids = torch.arange(nblocks, device=cuda, dtype=torch.int64) * 32 + 3
    cids = torch.randint(0, nel, (nblocks, 32), device=cuda, generator=g, dtype=torch.int64)
    F = torch.full((nblocks * 32 + 1, batch), 7.0, device=cuda)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.fl_diag_blocked_bwd_pattern(F.data_ptr(), gg.data_ptr(), o.data_ptr(), x.data_ptr(), nids.data_ptr(),
                                           cids.data_ptr(), nblocks, batch, waves, lds, st) == 0
    torch.cuda.synchronize()
    want = torch.empty(nblocks * 32, batch, device=cuda)
    for j in range(nblocks):
        for e in range(32):
            rows = int(nids[j]) + 4 * torch.arange(8, device=cuda) + (e // 4) % 4
            want[32 * j + e] = x[cids[j, e]] + (o[rows] * gg[rows]).sum(0)
    torch.testing.assert_close(F[:-1], want, rtol=1e-5, atol=1e-5)
    assert bool((F[-1] == 7.0).all())

