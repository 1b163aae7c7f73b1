"""Probabilistic-circuit integration: the sum-layer dispatcher contract the
reference patches into pyjuice (experiment_pyjuice/run_pyjuice.py:63-77).

``make_sparse_dispatcher(ext_call)`` returns a ``_forward_sparse``-compatible
method: for the log-likelihood propagation it selects ``local_ids`` (when
given) and calls ``ext_call(node_mars, element_mars, params, nids, cids, pids,
self.block_size)``; any other propagation algorithm goes to ``fallback`` (the
layer's original method), with the same arguments.
"""

from __future__ import annotations


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
