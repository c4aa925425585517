"""Batched tree verification: several independent sequences in one pass.

The reference verifies one sequence at a time (src/pe/serve.py:289-314: masks,
``forward_cached`` over the tree, ``accept_tree_cached``, ``gather_cache``). The
batched workload runs that step for B sequences at once, each with its own tree
over its own cached prefix of its own length:

- ``BatchKVCache``: K, V [B][L][nkv][capacity][hd]; ``seq(b)`` is sequence b's
  cache with the TreeKVCache API (prefill it with ``forward_cached``);
- ``forward_tree_batch``: one ``pe_forward`` over all B trees' rows (every
  weight streamed once per 64-row chunk for the whole batch), each row's
  K/V appended at its own sequence's rows, attention over each sequence's
  own keys in one launch;
- ``accept_tree_batch``: the greedy walk of every sequence in one launch;
- ``commit_batch``: every sequence's accepted rows compacted in one launch
  (ragged: each sequence moves its own path at its own prefix).

``BatchVerifyStep`` is the device-resident form (static buffers, HIP graph
capture), as ``VerifyStep`` is for one sequence.
"""

from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib, ops
from .target import TargetModel, TreeKVCache


class BatchKVCache:
    """One cache per sequence, contiguous per sequence: K, V [B][L][nkv][capacity][hd]."""

    def __init__(self, target: TargetModel, batch: int, capacity: int):
        s = target.shape
        self.shape, self.batch, self.capacity = s, int(batch), int(capacity)
        self.k = torch.zeros((batch, s.num_layers, s.num_kv_heads, capacity, s.head_dim), dtype=target.dtype,
                             device=target.device)
        self.v = torch.zeros_like(self.k)
        self._seqs = [TreeKVCache.view(s, self.k[b], self.v[b]) for b in range(batch)]

    def seq(self, b: int) -> TreeKVCache:
        return self._seqs[b]

    @property
    def seq_lens(self) -> list[int]:
        return [c.seq_len for c in self._seqs]

    @property
    def seq_stride(self) -> int:
        """Elements between two sequences' caches."""
        return self.k[0].numel()


class BatchTrees:
    """The device-side description of B trees: row offsets, each sequence's
    prefix, the concatenated tokens and (per-sequence) parents."""

    def __init__(self, node_tokens: list[list[int]], parents: list[list[int]], prefix_lens: list[int], device):
        if not (len(node_tokens) == len(parents) == len(prefix_lens)) or not node_tokens:
            raise ValueError("one token list, parent list and prefix length per sequence")
        rows = [len(t) for t in node_tokens]
        if any(r == 0 or r != len(p) for r, p in zip(rows, parents)):
            raise ValueError("every sequence needs a non-empty tree with one parent per node")
        self.batch = len(rows)
        self.rows = rows
        self.row0 = [0]
        for r in rows:
            self.row0.append(self.row0[-1] + r)
        self.M = self.row0[-1]
        self.max_rows = max(rows)
        self.words = max(1, math.ceil(self.max_rows / 64))
        if self.words > _lib.PE_TREE_MAX_WORDS:
            raise ValueError(f"a tree of {self.max_rows} nodes exceeds {64 * _lib.PE_TREE_MAX_WORDS}")
        self.prefix = [int(p) for p in prefix_lens]
        flat_t = [int(t) for ts in node_tokens for t in ts]
        flat_p = [int(q) for ps in parents for q in ps]
        self.tokens = torch.tensor(flat_t, dtype=torch.int64).to(device)
        self.parents = torch.tensor(flat_p, dtype=torch.int32).to(device)
        self.seq_row0 = torch.tensor(self.row0, dtype=torch.int32).to(device)
        self.seq_prefix = torch.tensor(self.prefix, dtype=torch.int64).to(device)


def tree_masks_batch(trees: BatchTrees, status: torch.Tensor):
    """(bits int64 [M][words], positions int64 [M], depths int32 [M]) of every sequence's tree."""
    dev = trees.tokens.device
    bits = torch.empty((trees.M, trees.words), dtype=torch.int64, device=dev)
    pos = torch.empty(trees.M, dtype=torch.int64, device=dev)
    dep = torch.empty(trees.M, dtype=torch.int32, device=dev)
    _lib.check(_lib.load().pe_tree_masks_batch(trees.parents.data_ptr(), trees.seq_row0.data_ptr(),
                                               trees.seq_prefix.data_ptr(), trees.batch, trees.max_rows,
                                               bits.data_ptr(), trees.words, pos.data_ptr(), dep.data_ptr(),
                                               status.data_ptr(), ops.stream_ptr()), "pe_tree_masks_batch")
    return bits, pos, dep


def _pass_args(tm: TargetModel, trees: BatchTrees, cache: BatchKVCache, ids, pos, bits, logits, fused, ws,
               status) -> _lib.PassArgs:
    a = _lib.PassArgs()
    a.input_ids, a.positions, a.M, a.mask_mode = ids.data_ptr(), pos.data_ptr(), trees.M, _lib.PE_MASK_TREE
    a.prefix_len = max(trees.prefix)
    a.tree_bits, a.bits_words = bits.data_ptr(), trees.words
    fl = tm.feature_layers
    a.num_features = len(fl) if fused is not None else 0
    for i, f in enumerate(fl[:4]):
        a.feature_layers[i] = f
    a.k_cache, a.v_cache, a.cache_capacity = cache.k.data_ptr(), cache.v.data_ptr(), cache.capacity
    a.logits = logits.data_ptr() if logits is not None else None
    a.fused = fused.data_ptr() if fused is not None else None
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.status = status.data_ptr()
    a.batch, a.max_seq_rows = trees.batch, trees.max_rows
    a.seq_row0, a.seq_prefix = trees.seq_row0.data_ptr(), trees.seq_prefix.data_ptr()
    a.cache_seq_stride = cache.seq_stride
    return a


def batch_workspace_bytes(tm: TargetModel, trees: BatchTrees) -> int:
    return int(_lib.load().pe_forward_batch_workspace_bytes(C.byref(tm.model.desc()), trees.M, trees.max_rows,
                                                             max(trees.prefix) + trees.max_rows, trees.batch))


@torch.no_grad()
def forward_tree_batch(tm: TargetModel, node_tokens: list[list[int]], parents: list[list[int]],
                       cache: BatchKVCache) -> tuple[torch.Tensor, torch.Tensor, BatchTrees]:
    """Verify B trees in one pass, tree b over ``cache.seq(b)``'s cached rows.
    Returns (logits [M][V], fused [M][F], trees); sequence b's rows are
    trees.row0[b] .. trees.row0[b+1] - 1. The tree rows' K/V sit at
    [P_b, P_b + T_b) of each sequence's cache (the lengths are unchanged until
    ``commit_batch``)."""
    dev = tm.device
    trees = BatchTrees(node_tokens, parents, cache.seq_lens, dev)
    if max(p + r for p, r in zip(trees.prefix, trees.rows)) > cache.capacity:
        raise _lib.PEError(_lib.PE_ERR_CAPACITY, "forward_tree_batch")
    bits, pos, _ = tree_masks_batch(trees, tm.status)
    logits = torch.empty((trees.M, tm.shape.vocab), dtype=tm.dtype, device=dev)
    fused = torch.empty((trees.M, tm.feature_dim), dtype=tm.dtype, device=dev)
    ws = torch.zeros(batch_workspace_bytes(tm, trees), dtype=torch.uint8, device=dev)
    a = _pass_args(tm, trees, cache, trees.tokens, pos, bits, logits, fused, ws, tm.status)
    _lib.check(_lib.load().pe_forward(C.byref(tm.model.desc()), C.byref(a), ops.stream_ptr()), "pe_forward (batch)")
    ops.read_status(tm.status, "forward_tree_batch")
    return logits, fused, trees


def accept_batch_device(root_logits: torch.Tensor, node_logits: torch.Tensor, trees: BatchTrees,
                        out: torch.Tensor | None = None, scratch: torch.Tensor | None = None) -> torch.Tensor:
    """Device result int32 [B][2 + max_rows]: per sequence (|path|, bonus, path...)."""
    B, V = root_logits.shape
    if B != trees.batch or node_logits.shape[0] != trees.M:
        raise ValueError("one root row per sequence and one node row per tree node")
    dev = root_logits.device
    if out is None:
        out = torch.zeros((B, 2 + trees.max_rows), dtype=torch.int32, device=dev)
    if scratch is None:
        scratch = torch.zeros(B * (trees.max_rows + 2), dtype=torch.int32, device=dev)
    _lib.check(_lib.load().pe_accept_tree_batch(root_logits.data_ptr(), root_logits.stride(0),
                                                node_logits.data_ptr(), node_logits.stride(0), V,
                                                ops.dcode(root_logits.dtype), trees.seq_row0.data_ptr(), B,
                                                trees.max_rows, trees.tokens.data_ptr(), trees.parents.data_ptr(),
                                                out.data_ptr(), scratch.data_ptr(), ops.stream_ptr()),
               "pe_accept_tree_batch")
    return out


def accept_tree_batch(root_logits: torch.Tensor, node_logits: torch.Tensor,
                      trees: BatchTrees) -> list[tuple[list[int], int]]:
    """accept_tree_cached (src/pe/decode/verify.py:104-125) for every sequence:
    [(accepted node indices in the sequence's own numbering, bonus)]."""
    out = accept_batch_device(root_logits, node_logits, trees).cpu().tolist()
    return [(row[2: 2 + row[0]], row[1]) for row in out]


def commit_batch(tm: TargetModel, cache: BatchKVCache, trees: BatchTrees, accept_out: torch.Tensor) -> None:
    """Keep each sequence's accepted path (gather_cache with the keep index of
    serve.py:308-309, per sequence) on the device; reads the path lengths back
    to set the cache lengths."""
    s = tm.shape
    _lib.check(_lib.load().pe_kv_compact_batch(cache.k.data_ptr(), cache.v.data_ptr(), trees.batch, cache.seq_stride,
                                               s.num_layers, s.num_kv_heads, cache.capacity, s.head_dim,
                                               ops.dcode(tm.dtype), trees.seq_prefix.data_ptr(),
                                               accept_out.data_ptr(), trees.max_rows, ops.stream_ptr()),
               "pe_kv_compact_batch")
    lens = accept_out[:, 0].cpu().tolist()
    for b, n in enumerate(lens):
        cache.seq(b).seq_len = trees.prefix[b] + int(n)


class BatchVerifyStep:
    """The batched verification step with every buffer preallocated (graph
    capturable): masks -> pe_forward over all sequences -> acceptance ->
    ragged compaction, at fixed per-sequence prefixes and tree sizes."""

    def __init__(self, tm: TargetModel, cache: BatchKVCache, node_tokens: list[list[int]],
                 parents: list[list[int]]):
        self.tm, self.cache = tm, cache
        dev = tm.device
        self.trees = BatchTrees(node_tokens, parents, cache.seq_lens, dev)
        t = self.trees
        self.bits = torch.zeros((t.M, t.words), dtype=torch.int64, device=dev)
        self.pos = torch.zeros(t.M, dtype=torch.int64, device=dev)
        self.depth = torch.zeros(t.M, dtype=torch.int32, device=dev)
        self.root = torch.zeros((t.batch, tm.shape.vocab), dtype=tm.dtype, device=dev)
        self.logits = torch.empty((t.M, tm.shape.vocab), dtype=tm.dtype, device=dev)
        self.fused = torch.empty((t.M, tm.feature_dim), dtype=tm.dtype, device=dev)
        self.accept_out = torch.zeros((t.batch, 2 + t.max_rows), dtype=torch.int32, device=dev)
        self.scratch = torch.zeros(t.batch * (t.max_rows + 2), dtype=torch.int32, device=dev)
        self.ws = torch.zeros(batch_workspace_bytes(tm, t), dtype=torch.uint8, device=dev)
        self._args = _pass_args(tm, t, cache, t.tokens, self.pos, self.bits, self.logits, self.fused, self.ws,
                                tm.status)
        self._buffers = (cache.k.data_ptr(), cache.v.data_ptr())
        self.graph = None

    def launch(self) -> None:
        if (self.cache.k.data_ptr(), self.cache.v.data_ptr()) != self._buffers:
            raise RuntimeError("the batch cache was replaced after this step was built")
        L, st, t, s = _lib.load(), ops.stream_ptr(), self.trees, self.tm.shape
        _lib.check(L.pe_tree_masks_batch(t.parents.data_ptr(), t.seq_row0.data_ptr(), t.seq_prefix.data_ptr(),
                                         t.batch, t.max_rows, self.bits.data_ptr(), t.words, self.pos.data_ptr(),
                                         self.depth.data_ptr(), self.tm.status.data_ptr(), st), "pe_tree_masks_batch")
        _lib.check(L.pe_forward(C.byref(self.tm.model.desc()), C.byref(self._args), st), "pe_forward (batch)")
        _lib.check(L.pe_accept_tree_batch(self.root.data_ptr(), self.root.stride(0), self.logits.data_ptr(),
                                          self.logits.stride(0), s.vocab, ops.dcode(self.tm.dtype),
                                          t.seq_row0.data_ptr(), t.batch, t.max_rows, t.tokens.data_ptr(),
                                          t.parents.data_ptr(), self.accept_out.data_ptr(), self.scratch.data_ptr(),
                                          st), "pe_accept_tree_batch")
        _lib.check(L.pe_kv_compact_batch(self.cache.k.data_ptr(), self.cache.v.data_ptr(), t.batch,
                                         self.cache.seq_stride, s.num_layers, s.num_kv_heads, self.cache.capacity,
                                         s.head_dim, ops.dcode(self.tm.dtype), t.seq_prefix.data_ptr(),
                                         self.accept_out.data_ptr(), t.max_rows, st), "pe_kv_compact_batch")

    def capture(self) -> None:
        self.launch()
        torch.cuda.synchronize(self.tm.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.launch()
        self.graph = g

    def run(self) -> None:
        if self.graph is not None:
            self.graph.replay()
        else:
            self.launch()

    def results(self) -> list[tuple[list[int], int]]:
        out = self.accept_out.cpu().tolist()
        ops.read_status(self.tm.status, "batch verify step")
        return [(row[2: 2 + row[0]], row[1]) for row in out]
