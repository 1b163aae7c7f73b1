"""The measurement kernels the bench's ceilings come from (fl_diag.hip).

They have no counterpart in the reference; these tests check that the copy
ceiling really copies, that the read ceiling reads without writing, and that
the latency probe runs every kind and rejects bad arguments."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture
def lib(cuda):
    """The library's entry points, returning their status codes."""
    from fuselse_amd import _lib

    return _lib.load()


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
