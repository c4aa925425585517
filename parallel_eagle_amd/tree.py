"""Parallel tree drafting with the API of src/pe/decode/tree.py:19-57.

The drafter's logits stay on the device: the per-depth log_softmax, each depth's
top candidates and the beam over depths run in two kernels (``pe_propose_tree``)
instead of one ``.tolist()`` per depth and a Python sort. ``propose_tree`` keeps
the reference's signature and list results; ``propose_tree_device`` returns the
device tensors the verification pass takes, without waiting for the GPU.

Order among equal candidates: tokens of one depth with equal logits are taken
lowest index first (the reference leaves torch.topk's order among equal values
open); candidates with equal cumulative log-probability keep the reference's
parent-major list order (its sort is stable).
"""

from __future__ import annotations

import torch

from . import _lib, ops


def beam_width(k: int, top_k: int, max_nodes: int) -> int:
    """The reference's beam width: max(1, min(top_k, max_nodes // k)) (src/pe/decode/tree.py:37)."""
    return max(1, min(top_k, max_nodes // max(1, k)))


def propose_tree_device(draft_logits: torch.Tensor, widths, top_k: int):
    """Beam over ``draft_logits`` [k][V] (row d predicts depth d) with ``widths[d]``
    nodes kept per depth and min(top_k, widths[d]) candidates per parent.
    Returns device tensors (node_tokens int64, parents int32, status int32[1])."""
    if not draft_logits.is_cuda:
        raise ValueError("parallel_eagle_amd proposes trees from HIP device logits")
    lg = draft_logits
    if lg.stride(-1) != 1:
        lg = lg.contiguous()
    return ops.propose_tree(lg, widths, top_k)


def propose_tree_from_logits(draft_logits: torch.Tensor, k: int, top_k: int, max_nodes: int,
                             pending: int = 0) -> tuple[list[int], list[int]]:
    """The post-drafter part of propose_tree on logits of k + pending depths."""
    if k < 1:
        return [], []
    w = beam_width(k, top_k, max_nodes)
    tokens, parents, status = propose_tree_device(draft_logits[pending: pending + k], [w] * k, w)
    st = int(status.item())
    if st:
        raise _lib.PEError(st, "propose_tree")
    return tokens.cpu().tolist(), parents.cpu().tolist()


def propose_tree(drafter, context_ids: torch.Tensor, context_feats: torch.Tensor, k: int, top_k: int,
                 max_nodes: int, pending: int = 0) -> tuple[list[int], list[int]]:
    """Return ``(node_tokens, parents)`` in topological order (parent before child);
    ``parents[t] == -1`` hangs off the confirmed prefix. ``drafter`` is any object
    with the reference drafter's ``draft_logits(context_ids, context_feats, n)``
    returning (n, V) logits on the device."""
    logits = drafter.draft_logits(context_ids, context_feats, k + pending)
    return propose_tree_from_logits(logits, k, top_k, max_nodes, pending)
