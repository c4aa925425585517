"""Tree masks restated from src/pe/masks.py (oracle; test infrastructure only).

- tree_depths        src/pe/masks.py:118-124
- tree_allow_mask    src/pe/masks.py:127-147
- tree_position_ids  src/pe/masks.py:150-156
- to_additive_bias   src/pe/masks.py:29-33
- ancestor_bits      the per-node ancestor set of tree_allow_mask's tree block as
                     integers (bit u of bits[t] set iff u is t or an ancestor of t)
"""

from __future__ import annotations

import numpy as np
import torch


def tree_depths(parents: list[int]) -> list[int]:
    depths = [0] * len(parents)
    for t, p in enumerate(parents):
        depths[t] = 0 if p < 0 else depths[p] + 1
    return depths


def tree_allow_mask(parents: list[int], prefix_len: int) -> np.ndarray:
    """bool (P+T, P+T): prefix causal; node rows see the whole prefix and their
    ancestor chain including themselves."""
    t = len(parents)
    n = prefix_len + t
    allow = np.zeros((n, n), dtype=bool)
    if prefix_len:
        allow[:prefix_len, :prefix_len] = np.tril(np.ones((prefix_len, prefix_len), dtype=bool))
        allow[prefix_len:, :prefix_len] = True
    for node in range(t):
        a = node
        while a != -1:
            allow[prefix_len + node, prefix_len + a] = True
            a = parents[a]
    return allow


def tree_position_ids(parents: list[int], prefix_len: int) -> list[int]:
    return list(range(prefix_len)) + [prefix_len + d for d in tree_depths(parents)]


def to_additive_bias(allow: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    a = torch.from_numpy(np.asarray(allow, dtype=bool))
    bias = torch.zeros(a.shape, dtype=dtype)
    bias.masked_fill_(~a, torch.finfo(dtype).min)
    return bias.unsqueeze(0).unsqueeze(0)


def ancestor_bits(parents: list[int]) -> list[int]:
    out = []
    for node in range(len(parents)):
        b, a = 0, node
        while a != -1:
            b |= 1 << a
            a = parents[a]
        out.append(b)
    return out


def is_topological(parents: list[int]) -> bool:
    return all(-1 <= p < t for t, p in enumerate(parents))
