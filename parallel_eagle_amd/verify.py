"""Greedy tree acceptance with the API of src/pe/decode/verify.py:35-57,104-125.

The argmax of every logit row and the descent into the first matching child run
on the device (``pe_accept_tree``); the host reads back one int32 vector
(|path|, bonus, path) instead of syncing once per accepted depth.
"""

from __future__ import annotations

import torch

from . import ops


def _device_lists(node_tokens, parents, device):
    tok = torch.as_tensor(list(node_tokens), dtype=torch.int64).to(device)
    par = torch.as_tensor(list(parents), dtype=torch.int32).to(device)
    return tok, par


def accept_tree_cached(root_logit: torch.Tensor, node_logits: torch.Tensor, node_tokens: list[int],
                       parents: list[int]) -> tuple[list[int], int]:
    """``root_logit`` (V,) predicts the token after the last confirmed one;
    ``node_logits[t]`` predicts the token after node t. Returns (accepted node
    indices, bonus token)."""
    if not root_logit.is_cuda:
        raise ValueError("parallel_eagle_amd accepts HIP device logits")
    tok, par = _device_lists(node_tokens, parents, root_logit.device)
    root = root_logit.reshape(-1)
    if root.stride(0) != 1:
        root = root.contiguous()
    nodes = node_logits.reshape(len(node_tokens), -1) if len(node_tokens) else node_logits
    out = ops.accept_tree(root, nodes, tok, par).cpu().tolist()
    n = out[0]
    return out[2: 2 + n], out[1]


def accept_tree_greedy(logits: torch.Tensor, prefix_len: int, node_tokens: list[int],
                       parents: list[int]) -> tuple[list[int], int]:
    """``logits`` covers [prefix | tree nodes] (P + T, V): the root prediction is row
    P - 1 and node t's is row P + t."""
    lg = logits.reshape(-1, logits.shape[-1])
    t = len(node_tokens)
    return accept_tree_cached(lg[prefix_len - 1], lg[prefix_len: prefix_len + t], node_tokens, parents)
