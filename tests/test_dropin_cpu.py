"""CPU tests of the drop-in's dispatch (fuselse/gpu/autograd.py:6-61) with a
fake extension and a tensor subclass that reports is_cuda=True.

They pin which function runs for which input (kernel vs torch fallback), the
shapes handed to the kernel (2-D contiguous rows), keepdim, the autograd path
(forward saves (rows, lse); backward flattens grad_output) and the factory's
robust switch, without a GPU."""

import pytest
import torch

from fuselse_amd.autograd import make_fuselse_logsumexp


class FakeCuda(torch.Tensor):
    @property
    def is_cuda(self):
        return True


def fake(t):
    return t.as_subclass(FakeCuda)


class FakeExt:
    def __init__(self):
        self.calls = []

    def _rec(self, name, *args):
        self.calls.append((name, [tuple(a.shape) for a in args], [a.is_contiguous() for a in args]))

    def onepass_lse_float(self, x):
        self._rec("fwd", x)
        assert x.dim() == 2 and x.is_contiguous()
        return torch.logsumexp(x.as_subclass(torch.Tensor), -1).as_subclass(FakeCuda)

    def onepass_lse_float_robust(self, x):
        self._rec("fwd_robust", x)
        assert x.dim() == 2 and x.is_contiguous()
        return torch.logsumexp(x.as_subclass(torch.Tensor), -1).as_subclass(FakeCuda)

    def batched_logsumexp_fp16(self, x, robust=False):
        self._rec("fwd_fp16", x)
        assert x.dtype == torch.float16 and x.dim() == 2 and x.is_contiguous()
        return torch.logsumexp(x.as_subclass(torch.Tensor).float(), -1).as_subclass(FakeCuda)

    def batched_logsumexp_bf16(self, x, robust=False):
        self._rec("fwd_bf16", x)
        assert x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous()
        return torch.logsumexp(x.as_subclass(torch.Tensor).float(), -1).as_subclass(FakeCuda)

    def onepass_lse_half_backward(self, g, x, lse):
        self._rec("bwd_half", g, x, lse)
        assert g.dtype == torch.float32 and lse.dtype == torch.float32 and x.dtype in (torch.float16, torch.bfloat16)
        gt, xt, lt = (t.as_subclass(torch.Tensor) for t in (g, x, lse))
        return (gt[:, None] * torch.exp(xt.float() - lt[:, None])).to(x.dtype).as_subclass(FakeCuda)

    def onepass_lse_float_backward(self, g, x, lse):
        self._rec("bwd", g, x, lse)
        assert g.dim() == 1 and x.dim() == 2 and lse.dim() == 1
        gt, xt, lt = (t.as_subclass(torch.Tensor) for t in (g, x, lse))
        return (gt[:, None] * torch.exp(xt - lt[:, None])).as_subclass(FakeCuda)


def test_robust_flag_selects_forward():
    ext = FakeExt()
    make_fuselse_logsumexp(ext, robust=True)(fake(torch.randn(3, 5)))
    make_fuselse_logsumexp(ext, robust=False)(fake(torch.randn(3, 5)))
    assert [c[0] for c in ext.calls] == ["fwd_robust", "fwd"]


def test_2d_contiguous_goes_straight_to_the_kernel():
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    x = torch.randn(4, 9)
    y = lse(fake(x))
    assert ext.calls == [("fwd_robust", [(4, 9)], [True])]
    torch.testing.assert_close(y.as_subclass(torch.Tensor), torch.logsumexp(x, -1))


def test_nd_and_noncontiguous_inputs_are_flattened():
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    x = torch.randn(2, 3, 7)
    y = lse(fake(x), dim=2)
    assert ext.calls[-1][1] == [(6, 7)] and y.shape == (2, 3)
    xt = torch.randn(7, 5).t()
    y = lse(fake(xt), -1)
    assert ext.calls[-1][1] == [(5, 7)] and ext.calls[-1][2] == [True]
    torch.testing.assert_close(y.as_subclass(torch.Tensor), torch.logsumexp(xt, -1))


def test_keepdim():
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    assert lse(fake(torch.randn(4, 6)), -1, keepdim=True).shape == (4, 1)
    assert lse(fake(torch.randn(2, 4, 6)), dim=-1, keepdim=True).shape == (2, 4, 1)


@pytest.mark.parametrize("case", ["cpu", "fp64", "fp16", "dim0", "n1", "middle_dim"])
def test_fallbacks_do_not_touch_the_extension(case):
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    x = {
        "cpu": torch.randn(3, 4),
        "fp64": fake(torch.randn(3, 4, dtype=torch.float64)),
        "fp16": fake(torch.randn(3, 4).half()),
        "dim0": fake(torch.randn(3, 4)),
        "n1": fake(torch.randn(3, 1)),
        "middle_dim": fake(torch.randn(2, 3, 4)),
    }[case]
    dim = {"dim0": 0, "middle_dim": 1}.get(case, -1)
    y = lse(x, dim=dim)
    assert ext.calls == []
    want = torch.logsumexp(x.as_subclass(torch.Tensor).float(), dim=dim)
    torch.testing.assert_close(y.as_subclass(torch.Tensor).float(), want, rtol=1e-3, atol=1e-3)


def test_factory_captures_torch_logsumexp_so_patching_does_not_recurse(monkeypatch):
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    monkeypatch.setattr(torch, "logsumexp", lse)
    x = torch.randn(3, 4)  # CPU -> fallback to the captured original
    torch.testing.assert_close(lse(x, -1), torch.log(torch.exp(x).sum(-1)))


def test_autograd_path_saves_rows_and_flattens_grad():
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    x = torch.randn(2, 3, 6, requires_grad=True)
    xf = fake(x)
    y = lse(xf, -1)
    assert y.shape == (2, 3)
    assert ext.calls[0][1] == [(6, 6)]
    w = torch.randn(2, 3)
    (y.as_subclass(torch.Tensor) * w).sum().backward()
    name, shapes, _ = ext.calls[-1]
    assert name == "bwd" and shapes == [(6,), (6, 6), (6,)]
    x2 = x.detach().clone().requires_grad_(True)
    (torch.logsumexp(x2, -1) * w).sum().backward()
    torch.testing.assert_close(x.grad, x2.grad)


def test_no_grad_uses_direct_path():
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    x = torch.randn(3, 4, requires_grad=True)
    with torch.no_grad():
        lse(fake(x))
    assert [c[0] for c in ext.calls] == ["fwd_robust"]


class FakeKeepExt(FakeExt):
    """An ext with the keeping forwards (this package's has them)."""

    def onepass_lse_float_keep(self, x):
        self._rec("fwd_keep", x)
        return torch.logsumexp(x.as_subclass(torch.Tensor), -1).as_subclass(FakeCuda)

    def onepass_lse_float_robust_keep(self, x):
        self._rec("fwd_robust_keep", x)
        return torch.logsumexp(x.as_subclass(torch.Tensor), -1).as_subclass(FakeCuda)

    def batched_logsumexp_fp16_keep(self, x, robust=False):
        self._rec("fwd_fp16_keep", x)
        return torch.logsumexp(x.as_subclass(torch.Tensor).float(), -1).as_subclass(FakeCuda)

    def batched_logsumexp_bf16_keep(self, x, robust=False):
        self._rec("fwd_bf16_keep", x)
        return torch.logsumexp(x.as_subclass(torch.Tensor).float(), -1).as_subclass(FakeCuda)


@pytest.mark.parametrize("robust", [True, False])
def test_autograd_forward_is_the_plain_forward_by_default(robust):
    """By default the forward under autograd is the plain forward, as in the
    reference (autograd.py:15-34), even where the ext has a keeping variant."""
    ext = FakeKeepExt()
    lse = make_fuselse_logsumexp(ext, robust=robust)
    assert lse.fuselse_keep is False
    x = torch.randn(4, 7, requires_grad=True)
    y = lse(fake(x))
    y.as_subclass(torch.Tensor).sum().backward()
    assert [c[0] for c in ext.calls] == ["fwd_robust" if robust else "fwd", "bwd"]


@pytest.mark.parametrize("robust", [True, False])
def test_autograd_forward_keeps_x_for_the_backward(robust):
    """With keep=True and grad the forward is the keeping variant, where the ext
    has one; without grad (nothing reads x again) it is the plain forward.  An
    ext without the keeping variants (the reference's) gets the plain forward
    both ways."""
    ext = FakeKeepExt()
    lse = make_fuselse_logsumexp(ext, robust=robust, keep=True)
    x = torch.randn(4, 7, requires_grad=True)
    y = lse(fake(x))
    y.as_subclass(torch.Tensor).sum().backward()
    assert [c[0] for c in ext.calls] == ["fwd_robust_keep" if robust else "fwd_keep", "bwd"]
    ext.calls.clear()
    with torch.no_grad():
        lse(fake(x))
    lse(fake(x.detach()))
    assert [c[0] for c in ext.calls] == ["fwd_robust" if robust else "fwd"] * 2
    plain = FakeExt()
    y = make_fuselse_logsumexp(plain, robust=robust, keep=True)(fake(x))
    y.as_subclass(torch.Tensor).sum().backward()
    assert [c[0] for c in plain.calls] == ["fwd_robust" if robust else "fwd", "bwd"]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("keep", [False, True])
def test_half_autograd_forward_keeps_x_only_when_asked(dtype, keep):
    ext = FakeKeepExt()
    lse = make_fuselse_logsumexp(ext, half_inputs=True, keep=keep)
    x = torch.randn(3, 9).to(dtype).requires_grad_(True)
    y = lse(fake(x))
    y.as_subclass(torch.Tensor).float().sum().backward()
    tag = "fwd_fp16" if dtype == torch.float16 else "fwd_bf16"
    assert [c[0] for c in ext.calls] == [tag + ("_keep" if keep else ""), "bwd_half"]


# ---------------------------------------------------------------------------
# make_selective_log_softmax (trl.trainer.utils.selective_log_softmax drop-in)
# ---------------------------------------------------------------------------
class FakeSelExt:
    def __init__(self):
        self.calls = []

    def selective_log_softmax_float(self, logits, index, robust=True, out=None):
        self.calls.append(("fwd", tuple(logits.shape), tuple(index.shape), index.dtype, robust))
        self.ptrs = getattr(self, "ptrs", []) + [logits.data_ptr()]
        assert logits.dim() == 2 and logits.is_contiguous() and index.dim() == 1
        lt = logits.as_subclass(torch.Tensor)
        lse = torch.logsumexp(lt, -1)
        logp = lt.gather(-1, index.as_subclass(torch.Tensor)[:, None])[:, 0] - lse
        if out is not None:
            out[0].copy_(logp)
            out[1].copy_(lse)
            return out
        return logp.as_subclass(FakeCuda), lse.as_subclass(FakeCuda)

    def selective_log_softmax_float_backward(self, g, logits, index, lse, out=None):
        self.calls.append(("bwd", tuple(g.shape), tuple(logits.shape), tuple(index.shape), tuple(lse.shape)))
        gt, lt, it, st = (t.as_subclass(torch.Tensor) for t in (g, logits, index, lse))
        grad = -gt[:, None] * torch.exp(lt - st[:, None])
        grad[torch.arange(len(it)), it] += gt
        if out is not None:
            assert out.is_contiguous()
            out.copy_(grad)
            return out
        return grad.as_subclass(FakeCuda)


def test_selective_dispatch_shapes_and_autograd():
    from fuselse_amd.selective import make_selective_log_softmax

    ext = FakeSelExt()
    sls = make_selective_log_softmax(ext)
    logits = torch.randn(2, 3, 11, requires_grad=True)
    index = torch.randint(0, 11, (2, 3), dtype=torch.int32)
    y = sls(fake(logits), fake(index))
    assert y.shape == (2, 3)
    assert ext.calls[0] == ("fwd", (6, 11), (6,), torch.int64, True)
    w = torch.randn(2, 3)
    (y.as_subclass(torch.Tensor) * w).sum().backward()
    assert ext.calls[-1][0] == "bwd" and ext.calls[-1][1:] == ((6,), (6, 11), (6,), (6,))
    l2 = logits.detach().clone().requires_grad_(True)
    ref = torch.log_softmax(l2, -1).gather(-1, index.long()[..., None])[..., 0]
    (ref * w).sum().backward()
    torch.testing.assert_close(logits.grad, l2.grad)
    torch.testing.assert_close(y.as_subclass(torch.Tensor), ref.detach())


def test_selective_takes_trl_slices_without_copying_the_logits():
    """trl passes logits[:, :-1, :]: rows contiguous within each leading index
    but not across.  The kernel runs once per leading slice on views of the
    caller's tensor (no copy); values and gradients match torch."""
    from fuselse_amd.selective import make_selective_log_softmax

    ext = FakeSelExt()
    sls = make_selective_log_softmax(ext)
    full = torch.randn(3, 5, 11)
    logits = fake(full)[:, :-1, :]
    assert not logits.is_contiguous()
    leaf = full.clone().requires_grad_(True)
    index = torch.randint(0, 11, (3, 4))
    with torch.no_grad():
        y0 = sls(logits, fake(index))
    assert [c[1] for c in ext.calls] == [(4, 11)] * 3
    assert ext.ptrs == [full[b].data_ptr() for b in range(3)]
    ext.calls.clear()
    view = fake(leaf)[:, :-1, :]
    y = sls(view, fake(index))
    w = torch.randn(3, 4)
    (y.as_subclass(torch.Tensor) * w).sum().backward()
    assert [c[0] for c in ext.calls] == ["fwd"] * 3 + ["bwd"] * 3
    l2 = full.clone().requires_grad_(True)
    ref = torch.log_softmax(l2[:, :-1, :], -1).gather(-1, index[..., None])[..., 0]
    (ref * w).sum().backward()
    torch.testing.assert_close(y0.as_subclass(torch.Tensor), ref.detach())
    torch.testing.assert_close(leaf.grad, l2.grad)
    # a layout with no contiguous slices is copied once
    ext.calls.clear()
    sls(fake(torch.randn(11, 3, 4)).permute(1, 2, 0), fake(torch.randint(0, 11, (3, 4))))
    assert [c[1] for c in ext.calls] == [(12, 11)]


def test_selective_fallbacks_do_not_touch_the_extension():
    from fuselse_amd.selective import make_selective_log_softmax

    seen = []

    def original(logits, index):
        seen.append(logits.dtype)
        return torch.zeros(index.shape)

    ext = FakeSelExt()
    sls = make_selective_log_softmax(ext, original=original)
    idx = torch.zeros(3, dtype=torch.int64)
    sls(torch.randn(3, 5), idx)                                   # CPU
    sls(fake(torch.randn(3, 5).bfloat16()), fake(idx))            # bf16
    sls(fake(torch.randn(3, 5, dtype=torch.float64)), fake(idx))  # fp64
    sls(fake(torch.randn(3, 5)), fake(torch.zeros(4, dtype=torch.int64)))  # shape mismatch
    assert ext.calls == [] and len(seen) == 4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_inputs_policy(dtype):
    """half_inputs=True sends CUDA fp16/bf16 rows to the half kernels; the result
    has the input dtype; the backward gets the fp32 LSE and returns the input
    dtype.  The default keeps the reference's fallback."""
    ext = FakeExt()
    tag = "fwd_fp16" if dtype == torch.float16 else "fwd_bf16"
    lse = make_fuselse_logsumexp(ext, half_inputs=True)
    x = torch.randn(2, 3, 10).to(dtype)
    y = lse(fake(x))
    assert y.dtype == dtype and y.shape == (2, 3) and ext.calls[-1][0] == tag
    xg = x.clone().requires_grad_(True)
    y = lse(fake(xg), -1)
    (y.as_subclass(torch.Tensor).float() * torch.randn(2, 3)).sum().backward()
    assert ext.calls[-1][0] == "bwd_half" and ext.calls[-1][1] == [(6,), (6, 10), (6,)]
    assert xg.grad.dtype == dtype
    ext2 = FakeExt()
    make_fuselse_logsumexp(ext2)(fake(x))
    assert ext2.calls == []


# ---------------------------------------------------------------------------
# pyjuice _forward_sparse dispatcher (experiment_pyjuice/run_pyjuice.py:63-77)
# ---------------------------------------------------------------------------
def test_sparse_dispatcher_local_ids_and_fallback():
    from fuselse_amd.pc import make_sparse_dispatcher

    calls, fb = [], []

    def ext_call(node_mars, element_mars, params, nids, cids, pids, block_size):
        calls.append((nids.tolist(), cids.tolist(), pids.tolist(), block_size))

    def original(self, *a, **kw):
        fb.append(kw["propagation_alg"])
        return "fallback"

    class Layer:
        block_size = 4

    fwd = make_sparse_dispatcher(ext_call, fallback=original)
    nids = torch.tensor([0, 4, 8])
    cids = torch.tensor([[1, 2], [3, 4], [5, 6]])
    pids = torch.tensor([[10, 20], [30, 40], [50, 60]])
    assert fwd(Layer(), None, None, None, nids, cids, pids, local_ids=torch.tensor([2, 0])) is None
    assert calls[-1] == ([8, 0], [[5, 6], [1, 2]], [[50, 60], [10, 20]], 4)
    fwd(Layer(), None, None, None, nids, cids, pids)
    assert calls[-1][0] == [0, 4, 8]
    assert fwd(Layer(), None, None, None, nids, cids, pids, propagation_alg="MPE") == "fallback"
    assert fb == ["MPE"] and len(calls) == 2
    with pytest.raises(NotImplementedError):
        make_sparse_dispatcher(ext_call)(Layer(), None, None, None, nids, cids, pids, propagation_alg="GeneralLL")


def test_reference_edge_cases_of_the_dispatch():
    """The reference's dispatch (autograd.py:37-43) evaluates dim >= 0 first and
    shape[-1] last, so: a tuple dim raises TypeError on any input, a 0-d CUDA
    fp32 tensor raises IndexError at shape[-1], a 0-d CPU tensor falls back to
    torch, and dim defaults to the last axis."""
    ext = FakeExt()
    lse = make_fuselse_logsumexp(ext)
    with pytest.raises(TypeError):
        lse(fake(torch.randn(3, 4)), dim=(0, 1))
    with pytest.raises(TypeError):
        lse(torch.randn(3, 4), dim=(0, 1))
    with pytest.raises(IndexError):
        lse(fake(torch.tensor(1.5)))
    y = lse(torch.tensor(1.5))
    torch.testing.assert_close(y, torch.logsumexp(torch.tensor(1.5), dim=-1))
    out = lse(fake(torch.randn(3, 4)))
    assert ext.calls and ext.calls[-1][0] == "fwd_robust" and tuple(out.shape) == (3,)
    assert not hasattr(lse, "out")


@pytest.mark.parametrize("bs", [1, 4])
def test_blocked_plan_lists_each_elements_block_edges_in_order(bs):
    """The block-layout backward's plan (built by torch ops on the tensors'
    device; here the CPU): csc_offsets delimit, for each element row, the
    block edges j * num_edges + e with cids[j, e] equal to it, in increasing
    order; block size 1 adds each edge's node row and parameter id."""
    from fuselse_amd.ext import _blocked_plan

    g = torch.Generator().manual_seed(3)
    nb, ne, nel = 7, 5, 9
    nids = torch.arange(nb, dtype=torch.int64) * bs + 2
    cids = torch.randint(0, nel, (nb, ne), generator=g)
    cids[0, :3] = 4                                     # repeats within a block
    pids = (torch.arange(nb * ne, dtype=torch.int64) * bs).reshape(nb, ne)
    plan = _blocked_plan(nids, cids, pids, bs, nel + 2)  # two element rows no block uses
    off, edges = plan.csc_offsets.tolist(), plan.csc_edges.tolist()
    assert len(off) == nel + 3 and off[0] == 0 and off[-1] == nb * ne
    for c in range(nel + 2):
        want = [j * ne + e for j in range(nb) for e in range(ne) if int(cids[j, e]) == c]
        assert edges[off[c]:off[c + 1]] == want
    if bs == 1:
        assert plan.csc_nodes.tolist() == [int(nids[k // ne]) for k in edges]
        assert plan.param_ids.tolist() == pids.reshape(-1).tolist()
    else:
        assert plan.csc_nodes is None and plan.param_ids is None
    with pytest.raises(RuntimeError, match=">= element_mars rows"):
        _blocked_plan(nids, cids, pids, bs, 3)
