"""Probabilistic-circuit integration: the sum-layer dispatcher contract the
reference patches into pyjuice (experiment_pyjuice/run_pyjuice.py:63-77).

``sparse_csr_layer(child, offsets, child_ids, logparams)`` is a CSR sum
layer with autograd: its backward is the flows kernel (gradients of the
children's log-values and of the log-weights), which the reference does not
have.  ``sparse_blocked_layer`` is the same for pyjuice's block layout, with
log-weights.

``make_sparse_dispatcher(ext_call)`` returns a ``_forward_sparse``-compatible
method: for the log-likelihood propagation it selects ``local_ids`` (when
given) and calls ``ext_call(node_mars, element_mars, params, nids, cids, pids,
self.block_size)``; any other propagation algorithm goes to ``fallback`` (the
layer's original method), with the same arguments.
"""

from __future__ import annotations

import torch


def make_sparse_dispatcher(ext_call, fallback=None):
    def _forward_sparse(self, node_mars, element_mars, params, nids, cids, pids, local_ids=None, partition_id=-1,
                        propagation_alg="LL", **kwargs):
        if propagation_alg != "LL":
            if fallback is None:
                raise NotImplementedError(f"propagation_alg={propagation_alg!r} has no kernel and no fallback")
            return fallback(self, node_mars, element_mars, params, nids, cids, pids, local_ids=local_ids,
                            partition_id=partition_id, propagation_alg=propagation_alg, **kwargs)
        if local_ids is not None:
            nids = nids[local_ids]
            cids = cids[local_ids]
            pids = pids[local_ids]
        ext_call(node_mars, element_mars, params, nids, cids, pids, self.block_size)
        return None

    return _forward_sparse


class _SparseCSRLayer(torch.autograd.Function):
    @staticmethod
    def forward(ctx, child, logparams, offsets, child_ids, csc):
        from . import ext

        out = ext.sparse_csr_forward(child, offsets, child_ids, logparams)
        ctx.save_for_backward(child, logparams, offsets, child_ids, out)
        ctx.csc = csc
        return out

    @staticmethod
    def backward(ctx, grad_out):
        from . import ext

        child, logparams, offsets, child_ids, out = ctx.saved_tensors
        if ctx.csc is None:
            ctx.csc = ext.sparse_csr_transpose(offsets, child_ids, child.size(0))
        gc, gl = ext.sparse_csr_backward(child, out, grad_out.contiguous(), offsets, child_ids, logparams, ctx.csc)
        return gc, gl, None, None, None


def sparse_csr_layer(child, offsets, child_ids, logparams, csc=None):
    """out[n, b] = LSE over the node's edges e of (logparams[e] + child[child_ids[e], b]),
    differentiable in child and logparams (fp32).  csc: a cached
    ext.sparse_csr_transpose(offsets, child_ids, child.size(0)) for this layer."""
    return _SparseCSRLayer.apply(child, logparams, offsets, child_ids, csc)


class _SparseBlockedLayer(torch.autograd.Function):
    @staticmethod
    def forward(ctx, element_mars, logparams, nids, cids, pids, block_size, num_nodes, plan):
        from . import ext

        node_mars = torch.full((num_nodes, element_mars.size(1)), float("-inf"), dtype=torch.float32,
                               device=element_mars.device)
        ext.sparse_forward_float(node_mars, element_mars, logparams, nids, cids, pids, block_size, params_are_log=True)
        ctx.save_for_backward(element_mars, logparams, nids, cids, pids, node_mars)
        ctx.block_size = block_size
        ctx.plan = plan
        return node_mars

    @staticmethod
    def backward(ctx, grad_out):
        from . import ext

        element_mars, logparams, nids, cids, pids, node_mars = ctx.saved_tensors
        if ctx.plan is None:
            ctx.plan = ext.sparse_blocked_transpose(nids, cids, pids, ctx.block_size, element_mars.size(0))
        ge = torch.zeros_like(element_mars)
        gl = torch.zeros_like(logparams)
        ext.sparse_blocked_backward(grad_out.contiguous(), ge, node_mars, element_mars, logparams, gl, nids, cids, pids,
                                    ctx.block_size, params_are_log=True, plan=ctx.plan)
        return ge, gl, None, None, None, None, None, None


def sparse_blocked_layer(element_mars, logparams, nids, cids, pids, block_size, num_nodes, plan=None):
    """pyjuice's block-layout sum layer with autograd, in fp32:
    out[nids[j] + p, b] = LSE over e of (logparams[pids[j, e] + p] + element_mars[cids[j, e], b])
    for every block j and position p < block_size; rows of out [num_nodes, batch]
    that no block writes are -inf.  Differentiable in element_mars and
    logparams: the backward is ext.sparse_blocked_backward with the upstream
    gradient as node flows (a term through a row of -inf contributes 0).
    plan: a cached ext.sparse_blocked_transpose(nids, cids, pids, block_size,
    element_mars.size(0)) for this layer."""
    return _SparseBlockedLayer.apply(element_mars, logparams, nids, cids, pids, int(block_size), int(num_nodes), plan)
