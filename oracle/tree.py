"""Beam tree proposal restated from src/pe/decode/tree.py:34-55 (oracle; test
infrastructure only).

``propose_tree_beam`` is the post-drafter part of propose_tree: log_softmax in
fp32 over the per-depth draft logits, then per depth every surviving parent is
expanded by the depth's top candidates, the candidates are stably sorted by
cumulative log-probability (Python float sums) and the best ``w_d`` are kept,
appended in that order with their parent's node index. ``widths`` generalises
the reference's constant ``beam_width``; with ``widths == [w] * k`` and
``cand_per_parent == w`` it is exactly the reference's beam. Among equal
log-probabilities of one depth the lowest token index comes first (the
reference's torch.topk leaves that order open).

Pinned by brute force: every depth's log-probabilities are the same for every
parent, so with non-increasing widths the beam at depth d is the set of the
best widths[d] token sequences of length d + 1 by summed log-probability over
all V^(d+1) sequences, best first; tests enumerate them for small V.
"""

from __future__ import annotations

import numpy as np
import torch


def row_candidates(logprobs: torch.Tensor, d: int, per_parent: int) -> tuple[list[float], list[int]]:
    """The best ``per_parent`` tokens of depth ``d`` (log-probability descending,
    lowest index first among equal values) with their log-probabilities."""
    row = logprobs[d].numpy()
    topi = np.lexsort((np.arange(row.shape[0]), -row))[:per_parent].tolist()
    return [float(row[i]) for i in topi], topi


def beam_from_candidates(topv: list[list[float]], topi: list[list[int]], widths: list[int]):
    """The beam of src/pe/decode/tree.py:41-55 over given per-depth candidates:
    every parent extended by the depth's candidates, a stable sort by cumulative
    log-probability (Python float sums), the best ``widths[d]`` kept."""
    beam: list[tuple[int, float]] = [(-1, 0.0)]
    node_tokens: list[int] = []
    parents: list[int] = []
    for d, w in enumerate(widths):
        cand = [(par, tok, cum + lp) for (par, cum) in beam for lp, tok in zip(topv[d], topi[d])]
        cand.sort(key=lambda c: c[2], reverse=True)
        cand = cand[:w]
        beam = []
        for par, tok, cum in cand:
            beam.append((len(node_tokens), cum))
            node_tokens.append(tok)
            parents.append(par)
    return node_tokens, parents


def propose_tree_beam(draft_logits: torch.Tensor, widths: list[int], top_k: int) -> tuple[list[int], list[int]]:
    logprobs = torch.log_softmax(draft_logits.float(), dim=-1)
    topv, topi = [], []
    for d, w in enumerate(widths):
        v, i = row_candidates(logprobs, d, min(top_k, w))
        topv.append(v)
        topi.append(i)
    return beam_from_candidates(topv, topi, list(widths))


def reference_constant_width(draft_logits: torch.Tensor, k: int, top_k: int, max_nodes: int):
    """The reference's width rule: beam_width = max(1, min(top_k, max_nodes // k))."""
    w = max(1, min(top_k, max_nodes // max(1, k)))
    return propose_tree_beam(draft_logits[:k], [w] * k, w)
