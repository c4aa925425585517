"""Synthetic inputs for the verification pass (host side).

A counter-based generator gives every synthetic tensor a fixed value per
(seed, stream, index) on any machine: splitmix64 hashes the counter and the
four 16-bit fields of the hash are summed (Irwin-Hall, n = 4), centred and
scaled to unit variance. Only integer arithmetic and two correctly rounded
float64 multiplies are involved, so this numpy version and the device kernel
``pe_fill_normal`` produce identical bits. The distribution is bounded at
+-2*sqrt(3) sigma, close to normal in shape; it stands in for the N(0, 0.02)
random init of the workloads and the N(0, 1) draft logits.

``build_tree`` turns per-depth draft logits into a candidate tree with the beam
of the reference's propose_tree (src/pe/decode/tree.py:34-55), generalised to
per-depth widths; ``plant_chain`` writes a known accepted path into a tree.
"""

from __future__ import annotations

import numpy as np
import torch

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z ^ (z >> np.uint64(30))
    z = z * _M1
    z = z ^ (z >> np.uint64(27))
    z = z * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, stream_id: int) -> np.uint64:
    with np.errstate(over="ignore"):
        z = (np.uint64(seed) * _GOLD + np.uint64(stream_id) * np.uint64(0xD1B54A32D192ED03)
             + np.uint64(0x632BE59BD9B4E019))
        return _mix64(np.asarray(z, dtype=np.uint64))


def _hash(seed: int, stream_id: int, start: int, n: int) -> np.ndarray:
    key = stream_key(seed, stream_id)
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(key + i * _GOLD)


def normal(seed: int, stream_id: int, n: int, std: float = 1.0, start: int = 0) -> np.ndarray:
    """float32 [n]."""
    z = _hash(seed, stream_id, start, n)
    m = np.uint64(0xFFFF)
    s = (z & m) + ((z >> np.uint64(16)) & m) + ((z >> np.uint64(32)) & m) + (z >> np.uint64(48))
    x = (s.astype(np.float64) + 2.0) / 65536.0 - 2.0
    v = x * 1.7320508075688772
    return (v * float(std)).astype(np.float32)


def uniform_int(seed: int, stream_id: int, n: int, hi: int, start: int = 0) -> np.ndarray:
    """int64 [n] in [0, hi)."""
    z = _hash(seed, stream_id, start, n)
    with np.errstate(over="ignore"):
        return (((z >> np.uint64(32)) * np.uint64(hi)) >> np.uint64(32)).astype(np.int64)


# stream ids of the synthetic model: one per tensor kind, offset per layer
STREAM_EMBED = 1
STREAM_LM_HEAD = 2
STREAM_PROMPT = 3
STREAM_DRAFT = 4
STREAM_KV = 5
STREAM_KV_V = 6
STREAM_LAYER0 = 1000  # layer l, tensor j -> 1000 + 16 * l + j
LINEAR_ORDER = ("q", "k", "v", "o", "gate", "up", "down", "q_bias", "k_bias", "v_bias")


def layer_stream(layer: int, name: str) -> int:
    return STREAM_LAYER0 + 16 * layer + LINEAR_ORDER.index(name)


def build_tree(draft_logits: torch.Tensor, widths, top_k: int) -> tuple[list[int], list[int]]:
    """(node_tokens, parents) in topological order from draft logits (k, V)."""
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
        beam = []
        for par, tok, cum in cand[:w]:
            beam.append((len(node_tokens), cum))
            node_tokens.append(tok)
            parents.append(par)
    return node_tokens, parents


def tree_for_seed(seed: int, vocab: int, depth: int, widths, top_k: int) -> tuple[list[int], list[int]]:
    logits = torch.from_numpy(normal(seed, STREAM_DRAFT, depth * vocab, 1.0).reshape(depth, vocab))
    return build_tree(logits, widths, top_k)


def chain_nodes(parents: list[int], leaf: int) -> list[int]:
    """Root-to-leaf node indices ending at ``leaf``."""
    out = []
    a = leaf
    while a != -1:
        out.append(a)
        a = parents[a]
    return out[::-1]


def deepest_first_leaf(parents: list[int]) -> int:
    depth = [0] * len(parents)
    for t, p in enumerate(parents):
        depth[t] = 0 if p < 0 else depth[p] + 1
    best = max(depth)
    return depth.index(best)


def set_token(node_tokens: list[int], parents: list[int], node: int, token: int, vocab: int) -> None:
    """Set node's token and keep its siblings' tokens distinct from it."""
    node_tokens[node] = token
    par = parents[node]
    used = {node_tokens[t] for t, p in enumerate(parents) if p == par and t != node}
    for t, p in enumerate(parents):
        if p == par and t != node and node_tokens[t] == token:
            cand = (token + 1) % vocab
            while cand == token or cand in used:
                cand = (cand + 1) % vocab
            node_tokens[t] = cand
            used.add(cand)
