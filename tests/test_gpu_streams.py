"""Every entry point launches on the caller's current stream (the reference's
contract: asynchronous launches on torch's current stream, no host
synchronisation).

Each case queues about a millisecond of work on a side stream, then writes
the inputs on that stream and calls the entry point inside the stream's
context.  A launch that went to another stream would run before the inputs
were written and read the zeros left there."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ext():
    import fuselse_amd

    return fuselse_amd.ext


def _busy(t):
    for _ in range(6):
        t.mul_(1.0001)


@pytest.fixture
def side(cuda):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    busy = torch.ones(1 << 26, device=cuda)
    torch.cuda.synchronize()
    yield s, busy
    torch.cuda.synchronize()


def test_float_entries_follow_the_current_stream(cuda, side):
    print("case streams float", flush=True)
    s, busy = side
    ext = _ext()
    src = torch.randn(64, 20000, device=cuda) * 3
    g = torch.randn(64, device=cuda)
    idx = torch.randint(0, 20000, (64,), device=cuda)
    want = torch.logsumexp(src, -1)
    x = torch.zeros_like(src)
    xh = torch.zeros_like(src, dtype=torch.float16)
    xsplit = torch.zeros(4, 200000, device=cuda)
    src_split = torch.randn(4, 200000, device=cuda)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        _busy(busy)
        x.copy_(src)
        xh.copy_(src)
        xsplit.copy_(src_split)
        lse = ext.onepass_lse_float_robust(x)
        lse_plain = ext.onepass_lse_float(x)
        gx = ext.onepass_lse_float_backward(g, x, lse)
        lh = ext.batched_logsumexp_fp16(xh)
        gh = ext.onepass_lse_half_backward(g, xh, lh)
        logp, lse_s = ext.selective_log_softmax_float(x, idx)
        gs = ext.selective_log_softmax_float_backward(g, x, idx, lse_s)
        lsplit = ext.onepass_lse_float_robust(xsplit)  # the split-row kernels and their workspace
    s.synchronize()
    torch.testing.assert_close(lse, want, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(lse_plain, want, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(gx, g[:, None] * torch.exp(src - want[:, None]), rtol=1e-5, atol=1e-12)
    torch.testing.assert_close(lh, torch.logsumexp(src.half().float(), -1), rtol=2e-5, atol=1e-5)
    torch.testing.assert_close(gh.float(), (g[:, None] * torch.exp(src.half().float() - lh[:, None])),
                               rtol=2.0 ** -10, atol=1e-7)
    torch.testing.assert_close(logp, src.gather(1, idx[:, None])[:, 0] - want, rtol=1e-5, atol=1e-5)
    sm = torch.softmax(src, -1)
    want_gs = -g[:, None] * sm
    want_gs[torch.arange(64, device=cuda), idx] += g
    torch.testing.assert_close(gs, want_gs, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(lsplit, torch.logsumexp(src_split.double(), -1).float(), rtol=1e-5, atol=1e-5)


def test_integer_and_sparse_entries_follow_the_current_stream(cuda, side):
    print("case streams intlse sparse", flush=True)
    s, busy = side
    ext = _ext()
    src = torch.randn(32, 4096, device=cuda) * 2
    want16 = ext.batched_logsumexp(src)
    q = torch.round(src * 128.0).to(torch.int16)
    want10 = ext.batched_logsumexp_q10_6(q)
    rng = np.random.default_rng(3)
    nch, batch, nodes = 500, 256, 60
    fan = rng.integers(1, 20, nodes)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(fan)]).astype(np.int64)).to(cuda)
    cid = torch.from_numpy(rng.integers(0, nch, int(fan.sum())).astype(np.int32)).to(cuda)
    lp = torch.from_numpy(np.log(rng.random(int(fan.sum())) + 1e-9).astype(np.float32)).to(cuda)
    child_src = torch.log(torch.rand(nch, batch, device=cuda) + 1e-9)
    want_csr = ext.sparse_csr_forward(child_src, off, cid, lp)
    x = torch.zeros_like(src)
    qz = torch.zeros_like(q)
    child = torch.zeros_like(child_src)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        _busy(busy)
        x.copy_(src)
        qz.copy_(q)
        child.copy_(child_src)
        got16 = ext.batched_logsumexp(x)
        got10 = ext.batched_logsumexp_q10_6(qz)
        got_csr = ext.sparse_csr_forward(child, off, cid, lp)
    s.synchronize()
    assert torch.equal(got16, want16)
    assert torch.equal(got10, want10)
    assert torch.equal(got_csr, want_csr)
