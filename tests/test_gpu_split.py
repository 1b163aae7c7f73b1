"""GPU parity of the split-row forward (few long rows: S blocks per row and a
last-block merge through a caller workspace) against the fp64 oracle, the
one-pass kernels of the same library and torch's special values.

The reference launches one block per row (fused_fp32_kernel.cu:168-170); the
split path must give the same results to the same tolerance: fp32 within
1e-5 relative, fp16/bf16 inputs within 1e-3 relative.  It must also be
deterministic (fixed merge order), whatever the workspace held before.
"""

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

RTOL32 = 1e-5
RTOL16 = 1e-3


def _mods():
    import fuselse_amd
    from fuselse_amd import _lib

    return fuselse_amd.ext, _lib


def _ws_bytes(B, N, elem_bytes):
    return _mods()[1].load().fl_lse_fwd_workspace_bytes(B, N, elem_bytes)


def _one_pass(x: torch.Tensor, robust: bool) -> torch.Tensor:
    """The no-workspace C entry, which always takes the one-pass kernels."""
    _, lib = _mods()
    B, N = x.shape
    out = torch.empty(B, device=x.device)
    entry = {torch.float32: "fl_lse_fwd_f32", torch.float16: "fl_lse_fwd_f16",
             torch.bfloat16: "fl_lse_fwd_bf16"}[x.dtype]
    lib.call(entry, x.data_ptr(), out.data_ptr(), B, N, int(robust), torch.cuda.current_stream().cuda_stream)
    return out


def _close(got, want, rtol, atol=0.0):
    np.testing.assert_allclose(np.asarray(got, np.float64), np.asarray(want, np.float64), rtol=rtol, atol=atol,
                               equal_nan=True)


SPLIT_SHAPES = [(1, 16385), (1, 128256), (2, 300001), (3, 50257), (7, 128256), (64, 128256), (191, 32003),
                (319, 20000)]


@pytest.mark.parametrize("B,N", SPLIT_SHAPES)
@pytest.mark.parametrize("robust", [False, True])
def test_split_f32_matches_fp64_and_one_pass(cuda, B, N, robust):
    print(f"case split_f32 B={B} N={N} robust={robust}", flush=True)
    assert _ws_bytes(B, N, 4) > 0, "shape expected on the split path"
    ext, _ = _mods()
    rng = np.random.default_rng(B * 7919 + N)
    x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
    xd = torch.from_numpy(x).to(cuda)
    fn = ext.onepass_lse_float_robust if robust else ext.onepass_lse_float
    got = fn(xd)
    _close(got.cpu().numpy(), O.lse_fp64(x), RTOL32, atol=1e-6)
    _close(got.cpu().numpy(), _one_pass(xd, robust).cpu().numpy(), RTOL32, atol=1e-6)


def test_split_is_deterministic(cuda):
    print("case split determinism", flush=True)
    ext, _ = _mods()
    x = torch.from_numpy(O.make_c2_input(48, 128256, seed=5)).to(cuda)
    a = ext.onepass_lse_float_robust(x)
    for _ in range(5):
        b = ext.onepass_lse_float_robust(x)
        assert torch.equal(a, b)


def test_split_c_entry_with_dirty_workspace(cuda):
    """The C entry with a caller workspace full of garbage (NaN bytes), reused
    across shapes whose partial areas overlap."""
    print("case split dirty workspace", flush=True)
    _, lib = _mods()
    ws = torch.full((1 << 20,), 0xFF, dtype=torch.uint8, device=cuda)
    rng = np.random.default_rng(9)
    for B, N in [(64, 128256), (180, 32003), (3, 50257), (180, 32003), (1, 128256)]:
        x = (rng.standard_normal((B, N)) * 3).astype(np.float32)
        xd = torch.from_numpy(x).to(cuda)
        out = torch.empty(B, device=cuda)
        need = lib.load().fl_lse_fwd_workspace_bytes(B, N, 4)
        assert 0 < need <= ws.numel()
        lib.call("fl_lse_fwd_f32_ws", xd.data_ptr(), out.data_ptr(), B, N, 1, ws.data_ptr(), ws.numel(),
                 torch.cuda.current_stream().cuda_stream)
        _close(out.cpu().numpy(), O.lse_fp64(x), RTOL32, atol=1e-6)


def test_split_spike_input_c2_rows(cuda):
    """The C2 recipe (N(0, 3^2), 0.1% of entries +15) at small B."""
    print("case split C2 recipe B=16", flush=True)
    ext, _ = _mods()
    x = O.make_c2_input(16, 128256, seed=3)
    got = ext.onepass_lse_float_robust(torch.from_numpy(x).to(cuda)).cpu().numpy()
    _close(got, O.lse_fp64(x), RTOL32)


def test_split_robust_special_values(cuda):
    print("case split robust special rows", flush=True)
    ext, _ = _mods()
    B, N = 6, 128256
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    x[0, :] = -np.inf                   # all -inf -> -inf
    x[1, 70000] = np.inf                # +inf in a middle segment -> +inf
    x[2, 127000] = np.nan               # NaN in the last segment -> NaN
    x[3, 5] = np.inf
    x[3, 100000] = -np.inf              # +inf wins over -inf
    x[4, : N // 2] = -np.inf            # whole segments empty
    x[5, 1:] = -np.inf                  # one finite element
    xd = torch.from_numpy(x).to(cuda)
    got = ext.onepass_lse_float_robust(xd).cpu().numpy()
    want = torch.logsumexp(torch.from_numpy(x).double(), dim=-1).numpy()
    assert got[0] == -np.inf and got[1] == np.inf and np.isnan(got[2]) and got[3] == np.inf
    _close(got[4:], want[4:], RTOL32)


@pytest.mark.parametrize("elem_offset", [1, 2, 3])
def test_split_unaligned_rows(cuda, elem_offset):
    print(f"case split unaligned off={elem_offset}", flush=True)
    ext, _ = _mods()
    B, N = 3, 20001
    rng = np.random.default_rng(elem_offset)
    x = (rng.standard_normal((B, N)) * 2).astype(np.float32)
    buf = torch.empty(B * N + elem_offset + 8, device=cuda)
    v = buf[elem_offset:elem_offset + B * N].view(B, N)
    v.copy_(torch.from_numpy(x).to(cuda))
    got = ext.onepass_lse_float_robust(v).cpu().numpy()
    _close(got, O.lse_fp64(x), RTOL32, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,N", [(1, 128256), (5, 65537), (100, 128256)])
def test_split_half(cuda, dtype, B, N):
    print(f"case split half {dtype} B={B} N={N}", flush=True)
    assert _ws_bytes(B, N, 2) > 0
    ext, _ = _mods()
    rng = np.random.default_rng(B + N)
    x = torch.from_numpy((rng.standard_normal((B, N)) * 2).astype(np.float32)).to(dtype)
    xd = x.to(cuda)
    fn = ext.batched_logsumexp_fp16 if dtype == torch.float16 else ext.batched_logsumexp_bf16
    got = fn(xd).cpu().numpy()
    _close(got, O.lse_fp64(x.float().numpy()), RTOL16)
    _close(got, _one_pass(xd, False).cpu().numpy(), RTOL32, atol=1e-6)


def test_split_on_a_side_stream(cuda):
    print("case split side stream", flush=True)
    ext, _ = _mods()
    x = torch.randn(8, 128256, device=cuda)
    want = ext.onepass_lse_float_robust(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = ext.onepass_lse_float_robust(x)
    torch.cuda.current_stream().wait_stream(s)
    assert torch.equal(got, want)


def test_one_pass_entry_still_one_pass_for_small_b(cuda):
    """The no-workspace entry keeps the reference's one-block-per-row geometry."""
    print("case one-pass small B", flush=True)
    x = np.random.default_rng(2).standard_normal((4, 128256)).astype(np.float32)
    got = _one_pass(torch.from_numpy(x).to(cuda), True).cpu().numpy()
    _close(got, O.lse_fp64(x), RTOL32, atol=1e-6)


def test_split_in_a_hip_graph_replays(cuda):
    """The split entry captured in a HIP graph (two kernel nodes, no memset):
    several replays, each after eager work that rewrites the input, each
    checked against an eager call."""
    print("case split graph replays", flush=True)
    _, lib = _mods()
    B, N = 16, 128256
    x = torch.empty(B, N, device=cuda)
    out = torch.empty(B, device=cuda)
    need = lib.load().fl_lse_fwd_workspace_bytes(B, N, 4)
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def call(st):
        lib.call("fl_lse_fwd_f32_ws", x.data_ptr(), out.data_ptr(), B, N, 1, ws.data_ptr(), need, st)

    x.normal_()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        call(s.cuda_stream)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call(s.cuda_stream)
    for rep in range(4):
        x.normal_(mean=float(rep), std=1.0 + rep)
        want = torch.logsumexp(x.double(), dim=-1).float()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(out, want, rtol=1e-5, atol=1e-5)
