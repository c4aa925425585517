"""Decoding loops over the device path.

``greedy_decode`` is the target alone: one prefill, then one one-token
``forward_cached`` pass per new token. It is the yardstick of the reference's
lossless invariant (tests/test_lossless.py:56-62): speculative decoding must
emit exactly its tokens.

``SpeculativeDecoder`` runs the reference's one-forward tree loop
(src/pe/serve.py:221-355, tree mode): a prefill, then per step a tree drafted
from the confirmed context, one verification pass over it against the cache,
the greedy walk, the accepted path's rows kept; on a miss, one one-token pass
of the pending bonus. Its design is not the reference's host loop:

- the loop's state lives on the device (``pe_loop_commit``): the context ids,
  the fused feature rows, the root logit row, the prefix length P and the
  pending bonus; nothing is re-uploaded or concatenated per step;
- for 16-bit models the verification step (masks -> pass -> walk ->
  compaction -> commit) and the miss pass are each recorded once as a HIP
  graph whose kernels read P from device memory (``pe_forward`` with a batch
  of one), so every step replays the same two graphs;
- the host reads one small record per step (the accepted length, the bonus,
  the accepted tokens and every status word); the bonus of a miss pass is
  read with the next step's record.

Other models (fp32) run the same kernels eagerly with P passed from the host.
"""

from __future__ import annotations

import ctypes as C
import math
import time
from dataclasses import dataclass, field

import torch

from . import _lib, ops
from .target import TargetModel, TreeKVCache
from .tree import beam_width


@dataclass
class LoopStats:
    """What a decode produced and what it cost."""

    tokens: list[int]
    steps: int = 0          # loop iterations after the prefill
    target_passes: int = 1  # verification and one-token passes, the prefill included
    draft_calls: int = 0
    accepted: int = 0       # drafted tokens accepted beyond the re-confirmed pending one
    host_reads: int = 0     # device-to-host reads inside the timed loop
    seconds: float = 0.0
    per_step: list[int] = field(default_factory=list)  # tokens each step committed

    @property
    def tokens_per_second(self) -> float:
        return len(self.tokens) / self.seconds if self.seconds > 0 else 0.0

    @property
    def tokens_per_step(self) -> float:
        return len(self.tokens) / max(1, self.steps)


def _first_argmax(row: torch.Tensor) -> int:
    return int(ops.argmax_rows(row.reshape(1, -1).contiguous())[0])


@torch.no_grad()
def greedy_decode(target: TargetModel, prompt_ids: list[int], max_new_tokens: int,
                  eos_token_id: int | None = None) -> LoopStats:
    """Greedy decoding through ``forward_cached``: the prompt as one causal pass,
    then the argmax of the last logit row is emitted and fed back as a
    one-token pass at the next position, until ``max_new_tokens`` tokens or
    ``eos_token_id`` (emitted, then stop)."""
    dev = target.device
    n0 = len(prompt_ids)
    cache = target.make_cache(n0 + max_new_tokens + 1)
    logits, _, cache = target.forward_cached(torch.tensor([list(prompt_ids)], device=dev), cache,
                                             torch.arange(n0, device=dev)[None])
    stats = LoopStats(tokens=[])
    t0 = time.perf_counter()
    while max_new_tokens > 0:
        tok = _first_argmax(logits[0, -1])
        stats.tokens.append(tok)
        stats.host_reads += 1
        if len(stats.tokens) >= max_new_tokens or tok == eos_token_id:
            break
        pos = n0 + len(stats.tokens) - 1
        logits, _, cache = target.forward_cached(torch.tensor([[tok]], device=dev), cache,
                                                 torch.tensor([[pos]], device=dev))
        stats.target_passes += 1
        stats.steps += 1
    torch.cuda.synchronize(dev)
    stats.seconds = time.perf_counter() - t0
    return stats


class _Step:
    """The device buffers and launches of one kind of loop step over ``rows`` rows:
    the verification step (``rows`` = the tree's node count) or the miss pass
    (one node, the pending token)."""

    def __init__(self, dec: "SpeculativeDecoder", rows: int):
        tm, dev = dec.tm, dec.tm.device
        s = tm.shape
        self.dec, self.rows = dec, rows
        self.words = max(1, math.ceil(rows / 64))
        self.parents = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(rows, dtype=torch.int64, device=dev)
        self.bits = torch.zeros((rows, self.words), dtype=torch.int64, device=dev)
        self.pos = torch.zeros(rows, dtype=torch.int64, device=dev)
        self.depth = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.row0 = torch.tensor([0, rows], dtype=torch.int32, device=dev)
        self.fused = torch.empty((rows, tm.feature_dim), dtype=tm.dtype, device=dev)
        # the miss pass writes its logit row straight into the loop's root row
        self.logits = dec.root.view(1, -1) if rows == 1 else torch.empty((rows, s.vocab), dtype=tm.dtype, device=dev)
        self.groups = int(_lib.load().pe_dense_gemm_argmax_groups(rows, s.vocab, s.hidden)) if dec.keys else 0
        self.keys = torch.zeros((rows, max(1, self.groups)), dtype=torch.int64, device=dev)
        self.acc_out = torch.zeros(2 + rows, dtype=torch.int32, device=dev)
        self.acc_scratch = torch.zeros(rows + 2, dtype=torch.int32, device=dev)
        self.amax = torch.zeros(1, dtype=torch.int32, device=dev)
        cap = dec.cache.capacity
        if dec.device_prefix:
            need = tm.model.desc()
            ws = int(_lib.load().pe_forward_batch_workspace_bytes(C.byref(need), rows, rows, cap, 1))
        else:
            ws = tm.model.workspace_bytes(rows, cap)
        self.ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        self.graph = None

    def _pass_args(self, P: int) -> _lib.PassArgs:
        dec, tm = self.dec, self.dec.tm
        c = dec.cache
        a = _lib.PassArgs()
        a.M = self.rows
        a.mask_mode = _lib.PE_MASK_TREE if (dec.device_prefix or self.rows > 1) else _lib.PE_MASK_CAUSAL
        a.input_ids = self.tokens.data_ptr() if self.rows > 1 else dec.state.data_ptr() + 8  # the pending token
        a.positions = self.pos.data_ptr()
        a.tree_bits = self.bits.data_ptr() if a.mask_mode == _lib.PE_MASK_TREE else None
        a.bits_words = self.words if a.mask_mode == _lib.PE_MASK_TREE else 0
        fl = tm.feature_layers
        a.num_features = len(fl)
        for i, f in enumerate(fl[:4]):
            a.feature_layers[i] = f
        a.k_cache, a.v_cache, a.cache_capacity = c.k.data_ptr(), c.v.data_ptr(), c.capacity
        a.logits, a.fused = self.logits.data_ptr(), self.fused.data_ptr()
        a.workspace, a.workspace_bytes = self.ws.data_ptr(), self.ws.numel()
        a.status = tm.status.data_ptr()
        a.node_keys = self.keys.data_ptr() if dec.keys else None
        if dec.device_prefix:
            # one sequence whose P is state[0], up to the cache's capacity
            a.batch, a.max_seq_rows = 1, self.rows
            a.seq_row0, a.seq_prefix = self.row0.data_ptr(), dec.state.data_ptr()
            a.cache_seq_stride = c.k.numel()
            a.prefix_len = c.capacity - self.rows
        else:
            a.prefix_len = P
        return a

    def launch(self, P: int) -> None:
        """Enqueue the step on the current stream (P: the host's prefix, used
        when the model does not read it on the device)."""
        dec, tm = self.dec, self.dec.tm
        L, st = _lib.load(), ops.stream_ptr()
        s, c, dt = tm.shape, dec.cache, ops.dcode(tm.dtype)
        status = tm.status.data_ptr()
        if dec.device_prefix:
            _lib.check(L.pe_tree_masks_batch(self.parents.data_ptr(), self.row0.data_ptr(), dec.state.data_ptr(), 1,
                                             self.rows, self.bits.data_ptr(), self.words, self.pos.data_ptr(),
                                             self.depth.data_ptr(), status, st), "pe_tree_masks_batch")
        elif self.rows > 1:
            _lib.check(L.pe_tree_masks(self.parents.data_ptr(), self.rows, P, self.bits.data_ptr(), self.words,
                                       self.pos.data_ptr(), self.depth.data_ptr(), status, st), "pe_tree_masks")
        else:
            self.pos.fill_(P)
        _lib.check(L.pe_forward(C.byref(tm.model.desc()), C.byref(self._pass_args(P)), st), "pe_forward")
        stats = (status, dec.draft_status, dec.propose_status.data_ptr())
        feat = tm.feature_dim
        if self.rows == 1:  # the miss pass: its bonus is the argmax of the root row
            if not dec.keys:
                _lib.check(L.pe_argmax_rows(dec.root.data_ptr(), s.vocab, 1, s.vocab, dt, self.amax.data_ptr(), st),
                           "pe_argmax_rows")
            _lib.check(L.pe_loop_miss_commit(self.fused.data_ptr(), feat, self.keys.data_ptr() if dec.keys else None,
                                             self.groups, None if dec.keys else self.amax.data_ptr(), dt,
                                             dec.feats.data_ptr(), dec.ids.data_ptr(), c.capacity,
                                             dec.state.data_ptr(), dec.rec.data_ptr(), *stats, st),
                       "pe_loop_miss_commit")
            return
        if dec.keys:
            _lib.check(L.pe_accept_tree_keys(dec.root.data_ptr(), s.vocab, dt, self.keys.data_ptr(), self.groups,
                                             self.rows, self.tokens.data_ptr(), self.parents.data_ptr(),
                                             self.acc_out.data_ptr(), self.acc_scratch.data_ptr(), st),
                       "pe_accept_tree_keys")
        else:
            _lib.check(L.pe_accept_tree(dec.root.data_ptr(), self.logits.data_ptr(), s.vocab, self.rows, s.vocab, dt,
                                        self.tokens.data_ptr(), self.parents.data_ptr(), self.acc_out.data_ptr(),
                                        self.acc_scratch.data_ptr(), st), "pe_accept_tree")
        if dec.device_prefix:
            _lib.check(L.pe_kv_compact_batch(c.k.data_ptr(), c.v.data_ptr(), 1, c.k.numel(), s.num_layers,
                                             s.num_kv_heads, c.capacity, s.head_dim, dt, dec.state.data_ptr(),
                                             self.acc_out.data_ptr(), self.rows, st), "pe_kv_compact_batch")
        else:
            _lib.check(L.pe_kv_compact(c.k.data_ptr(), c.v.data_ptr(), s.num_layers, s.num_kv_heads, c.capacity,
                                       s.head_dim, dt, P, self.acc_out.data_ptr(), st), "pe_kv_compact")
        _lib.check(L.pe_loop_commit(self.acc_out.data_ptr(), self.rows, self.tokens.data_ptr(), self.fused.data_ptr(),
                                    feat, self.logits.data_ptr(), s.vocab, dt, dec.feats.data_ptr(),
                                    dec.ids.data_ptr(), dec.root.data_ptr(), c.capacity, dec.state.data_ptr(),
                                    dec.rec.data_ptr(), dec.rec_path, *stats, st), "pe_loop_commit")

    def run(self, P: int) -> None:
        if self.dec.device_prefix:
            if self.graph is None:
                self.graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.graph):
                    self.launch(P)
            self.graph.replay()
        else:
            self.launch(P)


class SpeculativeDecoder:
    """Tree speculative decoding with the step's work and state on the device.

    ``drafter``: any object with ``draft_logits(context_ids, context_feats, k)``
    returning (k, V) device logits (the reference drafter's API); a drafter with
    ``draft_logits_extend`` (DeviceDrafter) keeps its context K/V across steps,
    and one with ``sync_status`` / ``status`` lets the loop fold its status word
    into the step's one read. The tree is the reference's constant-width beam:
    width max(1, min(tree_top_k, tree_max_nodes // k)) at each of k depths.
    ``use_graphs``: replay recorded steps (16-bit models with 128-dim heads);
    otherwise the kernels are launched each step.
    """

    def __init__(self, target: TargetModel, drafter, *, k: int, tree_top_k: int = 3, tree_max_nodes: int = 24,
                 use_graphs: bool = True):
        self.tm, self.drafter, self.k = target, drafter, int(k)
        w = beam_width(k, tree_top_k, tree_max_nodes)
        self.widths = [w] * self.k
        self.top_k = w
        self.T = w * self.k
        if self.T > 64 * _lib.PE_TREE_MAX_WORDS:
            raise ValueError(f"a tree of {self.T} nodes exceeds {64 * _lib.PE_TREE_MAX_WORDS}")
        s = target.shape
        # argmax keys from the lm_head for trees of one chunk; wider trees run as
        # a batch of one and their walk reads the node rows
        self.keys = target.dtype != torch.float32 and self.T <= 64
        self.device_prefix = (bool(use_graphs) and target.dtype != torch.float32 and s.head_dim == 128
                              and target.model.qkv_paired)

    # ------------------------------------------------------------ set-up per generate call
    def _allocate(self, capacity: int) -> None:
        tm, dev = self.tm, self.tm.device
        self.cache = TreeKVCache(tm.shape, tm.dtype, dev, capacity)
        self.ids = torch.zeros(capacity, dtype=torch.int64, device=dev)
        self.feats = torch.zeros((capacity, tm.feature_dim), dtype=tm.dtype, device=dev)
        self.root = torch.zeros(tm.shape.vocab, dtype=tm.dtype, device=dev)
        self.state = torch.zeros(2, dtype=torch.int64, device=dev)
        self.rec_path = self.T
        self.rec = torch.zeros(_lib.PE_LOOP_REC_HEAD + self.rec_path, dtype=torch.int32, device=dev)
        self.propose_status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.propose_scratch = torch.zeros(self.k * _lib.PE_PROPOSE_SCRATCH_PER_DEPTH, dtype=torch.uint8, device=dev)
        st = getattr(self.drafter, "status", None)
        self.draft_status = st.data_ptr() if isinstance(st, torch.Tensor) else None
        self.verify = _Step(self, self.T)
        self.miss = _Step(self, 1)

    def _propose(self, logits: torch.Tensor) -> None:
        """pe_propose_tree into the verification step's token and parent buffers."""
        if logits.shape != (self.k, self.tm.shape.vocab) or logits.stride(1) != 1:
            raise ValueError(f"the drafter must return ({self.k}, V) logits with contiguous rows")
        n = C.c_int32(0)
        widths = (C.c_int32 * self.k)(*self.widths)
        _lib.check(_lib.load().pe_propose_tree(logits.data_ptr(), logits.stride(0), self.k, logits.shape[1],
                                               ops.dcode(logits.dtype), widths, self.top_k,
                                               self.verify.tokens.data_ptr(), self.verify.parents.data_ptr(),
                                               C.byref(n), self.propose_scratch.data_ptr(),
                                               self.propose_status.data_ptr(), ops.stream_ptr()), "pe_propose_tree")
        if n.value != self.T:
            raise RuntimeError(f"the beam proposed {n.value} nodes, expected {self.T}")

    @torch.no_grad()
    def generate(self, prompt_ids: list[int], max_new_tokens: int, eos_token_id: int | None = None) -> LoopStats:
        tm, dev = self.tm, self.tm.device
        if hasattr(self.drafter, "reset"):
            self.drafter.reset()  # its cached context belongs to another prompt
        sync_before = getattr(self.drafter, "sync_status", None)
        if sync_before is not None:
            self.drafter.sync_status = False
        P = len(prompt_ids)
        self._allocate(P + max_new_tokens + self.T + 2)
        try:
            return self._loop(list(prompt_ids), max_new_tokens, eos_token_id)
        finally:
            if sync_before is not None:
                self.drafter.sync_status = sync_before
            torch.cuda.synchronize(dev)

    def _loop(self, prompt: list[int], max_new: int, eos: int | None) -> LoopStats:
        tm, dev = self.tm, self.tm.device
        P = len(prompt)
        ids_p = torch.tensor(prompt, device=dev)
        logits, fused, self.cache = tm.forward_cached(ids_p[None], self.cache, torch.arange(P, device=dev)[None])
        self.ids[:P] = ids_p
        self.feats[:P] = fused[0]
        self.root.copy_(logits[0, -1])
        bonus = _first_argmax(self.root)
        self.ids[P] = bonus
        self.state.copy_(torch.tensor([P, bonus], dtype=torch.int64))
        stats = LoopStats(tokens=[bonus])
        draft = getattr(self.drafter, "draft_logits_extend", None) or self.drafter.draft_logits
        stop = bonus == eos
        miss_pending = False  # a miss pass ran; its bonus comes with the next record
        t0 = time.perf_counter()
        while not stop and len(stats.tokens) + miss_pending < max_new:
            self._propose(draft(self.ids[:P], self.feats[:P], self.k))
            stats.draft_calls += 1
            self.verify.run(P)
            stats.target_passes += 1
            rec = self.rec.cpu().tolist()  # the step's one read
            stats.host_reads += 1
            if rec[2]:
                self.rec[2] = 0
                raise _lib.PEError(rec[2], "speculative step")
            if miss_pending:
                miss_pending = False
                stats.tokens.append(rec[3])
                if rec[3] == eos or len(stats.tokens) >= max_new:
                    break  # this step's verification is discarded
            n = rec[0]
            stats.steps += 1
            if n:
                # rec[4] re-confirms the pending bonus (already emitted)
                emit = rec[_lib.PE_LOOP_REC_HEAD + 1: _lib.PE_LOOP_REC_HEAD + n] + [rec[1]]
                P += n
                stats.accepted += n - 1
            else:
                self.miss.run(P)
                stats.target_passes += 1
                P += 1
                miss_pending, emit = True, []
            before = len(stats.tokens)
            for tok in emit:
                stats.tokens.append(tok)
                if tok == eos:
                    stop = True
                    break
                if len(stats.tokens) >= max_new:
                    break
            stats.per_step.append(len(stats.tokens) - before + (1 if miss_pending else 0))
        if miss_pending:
            rec = self.rec.cpu().tolist()
            stats.host_reads += 1
            if rec[2]:
                raise _lib.PEError(rec[2], "miss pass")
            stats.tokens.append(rec[3])
        torch.cuda.synchronize(dev)
        stats.seconds = time.perf_counter() - t0
        self.cache.seq_len = P
        del stats.tokens[max_new:]
        return stats
