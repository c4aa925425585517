"""Beam tree proposal restated from src/pe/decode/tree.py:34-55 (oracle; test
infrastructure only).

``propose_tree_beam`` is the post-drafter part of propose_tree: log_softmax in
fp32 over the per-depth draft logits, then per depth every surviving parent is
expanded by the depth's top candidates, the candidates are stably sorted by
cumulative log-probability (Python float sums) and the best ``w_d`` are kept,
appended in that order with their parent's node index. ``widths`` generalises
the reference's constant ``beam_width``; with ``widths == [w] * k`` and
``cand_per_parent == w`` it is exactly the reference's beam.
"""

from __future__ import annotations

import torch


def propose_tree_beam(draft_logits: torch.Tensor, widths: list[int], top_k: int) -> tuple[list[int], list[int]]:
    logprobs = torch.log_softmax(draft_logits.float(), dim=-1)
    beam: list[tuple[int, float]] = [(-1, 0.0)]
    node_tokens: list[int] = []
    parents: list[int] = []
    for d, w in enumerate(widths):
        per_parent = min(top_k, w)
        topv, topi = logprobs[d].topk(per_parent)
        topv, topi = topv.tolist(), topi.tolist()
        cand = [(par, tok, cum + lp) for (par, cum) in beam for lp, tok in zip(topv, topi)]
        cand.sort(key=lambda c: c[2], reverse=True)
        cand = cand[:w]
        beam = []
        for par, tok, cum in cand:
            beam.append((len(node_tokens), cum))
            node_tokens.append(tok)
            parents.append(par)
    return node_tokens, parents


def reference_constant_width(draft_logits: torch.Tensor, k: int, top_k: int, max_nodes: int):
    """The reference's width rule: beam_width = max(1, min(top_k, max_nodes // k))."""
    w = max(1, min(top_k, max_nodes // max(1, k)))
    return propose_tree_beam(draft_logits[:k], [w] * k, w)
