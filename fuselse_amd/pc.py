"""Probabilistic-circuit integration: the sum-layer dispatcher contract the
reference patches into pyjuice (experiment_pyjuice/run_pyjuice.py:63-77).

``sparse_csr_layer(child, offsets, child_ids, logparams)`` is a CSR sum
layer with autograd: its backward is the flows kernel (gradients of the
children's log-values and of the log-weights), which the reference does not
have.

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
