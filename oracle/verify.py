"""Greedy tree acceptance restated from src/pe/decode/verify.py (oracle; test
infrastructure only).

- accept_tree_cached  src/pe/decode/verify.py:104-125
- accept_tree_greedy  src/pe/decode/verify.py:35-57

Argmax follows torch.argmax: the first index among equal maxima (NaN counts as
the maximum). The walk descends into the first child, in node order, whose
token equals the current argmax.
"""

from __future__ import annotations

from collections import defaultdict

import numpy as np
import torch


def first_argmax(row) -> int:
    if isinstance(row, torch.Tensor):
        return int(row.float().argmax()) if not torch.isnan(row.float()).any() else int(
            torch.isnan(row.float()).nonzero()[0])
    a = np.asarray(row, dtype=np.float64)
    nan = np.isnan(a)
    if nan.any():
        return int(np.flatnonzero(nan)[0])
    return int(np.argmax(a))


def _children(parents):
    ch: dict[int, list[int]] = defaultdict(list)
    for t, par in enumerate(parents):
        ch[par].append(t)
    return ch


def accept_tree_cached(root_logit, node_logits, node_tokens, parents) -> tuple[list[int], int]:
    children = _children(parents)
    path: list[int] = []
    cur, parent = root_logit, -1
    while True:
        truth = first_argmax(cur)
        nxt = next((t for t in children.get(parent, []) if int(node_tokens[t]) == truth), None)
        if nxt is None:
            return path, truth
        path.append(nxt)
        parent, cur = nxt, node_logits[nxt]


def accept_tree_greedy(logits, prefix_len: int, node_tokens, parents) -> tuple[list[int], int]:
    children = _children(parents)
    path: list[int] = []
    pos, parent = prefix_len - 1, -1
    while True:
        truth = first_argmax(logits[pos])
        nxt = next((t for t in children.get(parent, []) if int(node_tokens[t]) == truth), None)
        if nxt is None:
            return path, truth
        path.append(nxt)
        parent, pos = nxt, prefix_len + nxt


def compact_rows(cache_rows: np.ndarray, prefix_len: int, path: list[int]) -> np.ndarray:
    """Reference semantics of gather_cache with keep = [0..P) + [P + t for t in path]
    (src/pe/target.py:194-201, src/pe/serve.py:308-309) on the sequence axis (-2)."""
    keep = list(range(prefix_len)) + [prefix_len + t for t in path]
    return np.take(cache_rows, keep, axis=-2)
