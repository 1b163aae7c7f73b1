"""fl_lse_fwd_f32_noalloc (split partials in a static device array) against
fl_lse_fwd_f32_ws (the same kernels with a caller workspace): bit-identical
outputs on consecutive calls, the second smaller than the first, so the
second call runs over partials the first left in the shared array."""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _lib():
    from fuselse_amd import _lib

    return _lib


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ws_call(x, robust):
    lib = _lib()
    B, N = x.shape
    need = lib.load().fl_lse_fwd_workspace_bytes(B, N, 4)
    ws = torch.empty(max(need, 8), dtype=torch.uint8, device=x.device)
    ws.fill_(0xFF)  # any contents: the partials kernel writes what the merge reads
    out = torch.empty(B, device=x.device)
    lib.call("fl_lse_fwd_f32_ws", x.data_ptr(), out.data_ptr(), B, N, int(robust), ws.data_ptr() if need else 0,
             need, _stream())
    return out


def _noalloc_call(x, robust):
    B, N = x.shape
    out = torch.empty(B, device=x.device)
    _lib().call("fl_lse_fwd_f32_noalloc", x.data_ptr(), out.data_ptr(), B, N, int(robust), _stream())
    return out


# (first shape, second smaller shape): split plans with many segments, then
# fewer rows / segments; a one-pass shape (no partials) last.
PAIRS = [((64, 128256), (7, 50000)), ((319, 128256), (1, 16385)), ((200, 9000), (3, 4100)),
         ((300, 70001), (512, 1000))]


@pytest.mark.parametrize("first,second", PAIRS)
@pytest.mark.parametrize("robust", [False, True])
def test_noalloc_matches_workspace_entry(cuda, first, second, robust):
    print(f"case noalloc {first} then {second} robust={robust}", flush=True)
    rng = np.random.default_rng(first[0] + second[1])
    for B, N in (first, second):
        x = O.make_c2_input(B, N, seed=int(rng.integers(1 << 30)))
        if robust:
            x = O.make_robust_rows(x, seed=B)
        xd = torch.from_numpy(x).to(cuda)
        got = _noalloc_call(xd, robust)
        want = _ws_call(xd, robust)
        torch.cuda.synchronize()
        assert torch.equal(got.isnan(), want.isnan())
        assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want)), (B, N)
        np.testing.assert_allclose(got.cpu().numpy(), O.lse_fp64(x), rtol=1e-5, atol=1e-6, equal_nan=True)


def test_noalloc_under_graph_capture(cuda):
    """The point of the entry: it can be captured (after a first eager call on
    the device); replays with new inputs match the workspace entry."""
    print("case noalloc graph capture", flush=True)
    B, N = 16, 128256
    xd = torch.from_numpy(O.make_c2_input(B, N, seed=5)).to(cuda)
    out = torch.empty(B, device=cuda)
    _lib().call("fl_lse_fwd_f32_noalloc", xd.data_ptr(), out.data_ptr(), B, N, 1, _stream())
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            _lib().call("fl_lse_fwd_f32_noalloc", xd.data_ptr(), out.data_ptr(), B, N, 1, s.cuda_stream)
    for seed in (6, 7, 8):
        xd.copy_(torch.from_numpy(O.make_c2_input(B, N, seed=seed)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, _ws_call(xd, True))


def test_noalloc_rejects_bad_arguments(cuda):
    lib = _lib()
    with pytest.raises(RuntimeError, match="negative shape"):
        lib.call("fl_lse_fwd_f32_noalloc", 0, 0, -1, 4, 0, _stream())
    with pytest.raises(RuntimeError, match="out is NULL"):
        lib.call("fl_lse_fwd_f32_noalloc", 0, 0, 4, 4, 0, _stream())
