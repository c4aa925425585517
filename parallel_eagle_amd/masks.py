"""Tree-verification masks with the API of src/pe/masks.py:29-33,118-156.

``tree_depths`` works on the host list, as the reference's does. The device
functions build the ancestor structure with ``pe_tree_masks`` (one small kernel:
bit u of bits[t] is set iff node u is t or an ancestor of t) instead of one
element write per ancestor into a dense (P+T)^2 matrix; the dense forms are
produced from those bits only for callers that ask for them.
"""

from __future__ import annotations

import math

import torch

from . import _lib, ops


def _cuda(device) -> torch.device:
    d = torch.device(device) if device is not None else torch.device("cuda")
    if d.type != "cuda":
        raise ValueError("parallel_eagle_amd builds tree masks on the HIP device (pass device='cuda')")
    return d


def tree_depths(parents: list[int]) -> list[int]:
    """Depth of each node; parents[t] == -1 hangs off the prefix (depth 0)."""
    depths = [0] * len(parents)
    for t, p in enumerate(parents):
        depths[t] = 0 if p < 0 else depths[p] + 1
    return depths


def tree_ancestor_bits(parents: list[int], prefix_len: int, device="cuda"):
    """(bits int64 [T][words], positions int64 [T] = P + depth, depths int32 [T]) on device.
    Raises ValueError for a non-topological parent list."""
    d = _cuda(device)
    t = len(parents)
    words = max(1, math.ceil(t / 64))
    if words > _lib.PE_TREE_MAX_WORDS:
        raise ValueError(f"tree of {t} nodes exceeds {64 * _lib.PE_TREE_MAX_WORDS}")
    status = torch.zeros(4, dtype=torch.int32, device=d)
    par = torch.as_tensor(list(parents), dtype=torch.int32).to(d)
    bits, pos, dep = ops.tree_masks(par, prefix_len, words, status)
    if int(status[0].item()):
        raise ValueError("parents must be topologically ordered (parent index < child index, -1 for roots)")
    return bits, pos, dep


def tree_allow_mask(parents: list[int], prefix_len: int, device="cuda") -> torch.Tensor:
    """Boolean (P+T, P+T) attend-mask over [prefix | tree nodes]: prefix causal,
    every node sees the whole prefix and its ancestor chain (itself included)."""
    bits, _, _ = tree_ancestor_bits(parents, prefix_len, device)
    return ops.tree_allow_dense(bits, prefix_len)


def tree_position_ids(parents: list[int], prefix_len: int, device="cuda") -> torch.Tensor:
    """Prefix positions 0..P-1, then P + depth per node (siblings share a position)."""
    d = _cuda(device)
    _, pos, _ = tree_ancestor_bits(parents, prefix_len, d)
    if prefix_len:
        return torch.cat([torch.arange(prefix_len, device=d), pos])
    return pos


def to_additive_bias(allow: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Boolean attend-mask -> 4-D additive bias (1, 1, S, S'): 0 where allowed,
    finfo(dtype).min elsewhere."""
    bias = torch.zeros(allow.shape, dtype=dtype, device=allow.device)
    bias.masked_fill_(~allow, torch.finfo(dtype).min)
    return bias.unsqueeze(0).unsqueeze(0)
