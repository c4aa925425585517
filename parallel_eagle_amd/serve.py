"""The reference's decode loops over this package's target, drafter and acceptance.

``generate_speculative_cached`` follows the shipped one-forward loop of
src/pe/serve.py:221-355 (tree mode) step for step: prefill, the pending bonus
re-confirmed at depth 0, one tree verification per step through
``forward_cached`` with the dense tree bias of masks.py, ``accept_tree_cached``,
the commit by ``gather_cache`` with keep = [0, P) + [P + t for t in path], the
fused features of the accepted path appended, and on a miss ``crop`` plus a
one-token forward of the pending bonus. ``vanilla_generate_cached`` is the
greedy baseline of src/pe/decode/baselines.py:49-94 (one incremental forward
per token). Both loops only call the reference-shaped API (TargetModel,
propose_tree, accept_tree_cached, the mask helpers), so they are the proof that
a serve.py-style caller runs unchanged on the device path: their outputs must
be equal (the reference's lossless invariant, tests/test_lossless.py:56-62).

``SpeculativeDecoder`` is the same loop with the step's device work kept on the
device: the tree goes from the drafter's logits to the verification pass as
device tensors (no per-depth host reads), the masks come from the parent list
on the device, the acceptance walk and the compaction of the accepted rows run
there too, and the host reads one small vector per step (the accepted path and
the bonus), which it needs to emit tokens anyway.
"""

from __future__ import annotations

import time
from collections.abc import Callable
from dataclasses import dataclass

import torch

from . import _lib, ops
from .masks import to_additive_bias, tree_allow_mask, tree_position_ids
from .tree import beam_width, propose_tree, propose_tree_device
from .verify import accept_tree_cached


@dataclass
class GenResult:
    """src/pe/decode/result.py: the loop's output and counters."""

    output_ids: list[int]
    steps: int
    target_calls: int
    drafter_calls: int
    accepted_tokens: int
    num_generated: int
    seconds: float

    @property
    def acceptance_length(self) -> float:
        return self.num_generated / max(1, self.steps)

    @property
    def tokens_per_second(self) -> float:
        return self.num_generated / self.seconds if self.seconds > 0 else 0.0


def _argmax(row: torch.Tensor) -> int:
    return int(ops.argmax_rows(row.reshape(1, -1).contiguous())[0])


@torch.no_grad()
def vanilla_generate_cached(target, prompt_ids: list[int], max_new_tokens: int, eos_token_id: int | None = None,
                            on_commit: Callable[[list[int]], None] | None = None) -> GenResult:
    """Greedy decoding with a KV cache (src/pe/decode/baselines.py:49-94)."""
    dev = target.device
    seq = list(prompt_ids)
    base = len(seq)
    cache = target.make_cache()
    pos = torch.arange(len(seq), device=dev).unsqueeze(0)
    logits, _, cache = target.forward_cached(torch.tensor(seq, device=dev).unsqueeze(0), cache, pos)
    nxt = _argmax(logits[0, -1])
    target_calls = 1
    t0 = time.perf_counter()
    while len(seq) - base < max_new_tokens:
        seq.append(nxt)
        if on_commit is not None:
            on_commit([nxt])
        if eos_token_id is not None and nxt == eos_token_id:
            break
        if len(seq) - base >= max_new_tokens:
            break
        npos = torch.tensor([[len(seq) - 1]], device=dev)
        logits, _, cache = target.forward_cached(torch.tensor([[nxt]], device=dev), cache, npos)
        target_calls += 1
        nxt = _argmax(logits[0, -1])
    torch.cuda.synchronize(dev)
    n = len(seq) - base
    return GenResult(seq[base:], n, target_calls, 0, 0, n, time.perf_counter() - t0)


@torch.no_grad()
def generate_speculative_cached(target, drafter, prompt_ids: list[int], *, k: int, mode: str = "tree",
                                max_new_tokens: int = 256, tree_top_k: int = 3, tree_max_nodes: int = 24,
                                eos_token_id: int | None = None,
                                on_commit: Callable[[list[int]], None] | None = None) -> GenResult:
    """One-forward KV-cache speculative decoding, tree mode (src/pe/serve.py:221-355)."""
    if mode != "tree":
        raise ValueError(f"unknown mode {mode!r}: the device path verifies trees")
    dev = target.device
    seq = list(prompt_ids)
    base = len(seq)
    cache = target.make_cache()
    pos = torch.arange(len(seq), device=dev).unsqueeze(0)
    logits, fused, cache = target.forward_cached(torch.tensor(seq, device=dev).unsqueeze(0), cache, pos)
    feats = fused[0]
    cache_len = len(seq)
    root_logit = logits[0, -1]
    target_calls, drafter_calls, accepted, steps = 1, 0, 0, 0
    bonus = _argmax(root_logit)
    seq.append(bonus)
    if on_commit is not None:
        on_commit([bonus])
    stop = eos_token_id is not None and bonus == eos_token_id
    t0 = time.perf_counter()
    while len(seq) - base < max_new_tokens and not stop:
        ctx = torch.tensor(seq[:cache_len], device=dev)
        node_tokens, parents = propose_tree(drafter, ctx, feats, k, tree_top_k, tree_max_nodes)
        drafter_calls += 1
        allow = tree_allow_mask(parents, cache_len, device=dev)[cache_len:, :]
        bias = to_additive_bias(allow, target.dtype)
        npos = tree_position_ids(parents, cache_len, device=dev)[cache_len:].unsqueeze(0)
        vlogits, vfused, cache = target.forward_cached(torch.tensor(node_tokens, device=dev).unsqueeze(0), cache,
                                                       npos, attention_mask=bias)
        target_calls += 1
        path, new_bonus = accept_tree_cached(root_logit, vlogits[0], node_tokens, parents)
        acc_tokens = [node_tokens[t] for t in path]
        if acc_tokens:
            keep = torch.tensor(list(range(cache_len)) + [cache_len + t for t in path], device=dev)
            target.gather_cache(cache, keep)
            feats = torch.cat([feats, vfused[0][path]], dim=0)
            cache_len += len(acc_tokens)
            root_logit = vlogits[0][path[-1]]
            emit = [*acc_tokens[1:], int(new_bonus)]
            accepted += len(acc_tokens) - 1
        else:
            pending = seq[cache_len]
            cache.crop(cache_len)
            blogits, bfused, cache = target.forward_cached(torch.tensor([[pending]], device=dev), cache,
                                                           torch.tensor([[cache_len]], device=dev))
            target_calls += 1
            feats = torch.cat([feats, bfused[0]], dim=0)
            cache_len += 1
            root_logit = blogits[0, -1]
            emit = [_argmax(root_logit)]
        steps += 1
        emitted: list[int] = []
        for tok in emit:
            seq.append(tok)
            emitted.append(tok)
            if eos_token_id is not None and tok == eos_token_id:
                stop = True
                break
            if len(seq) - base >= max_new_tokens:
                break
        if on_commit is not None and emitted:
            on_commit(emitted)
    torch.cuda.synchronize(dev)
    return GenResult(seq[base: base + max_new_tokens], steps, target_calls, drafter_calls, accepted,
                     min(len(seq) - base, max_new_tokens), time.perf_counter() - t0)


class SpeculativeDecoder:
    """``generate_speculative_cached`` with the step's work resident on the device.

    Per step: the drafter's logits (device) -> ``pe_propose_tree`` (device
    tokens and parents) -> ``pe_tree_masks`` (bitmasks and positions from the
    parents) -> ``pe_forward`` over the tree -> ``pe_accept_tree`` against the
    root logit row -> ``pe_kv_compact`` of the accepted rows, all enqueued
    without a host read; then one read of (|path|, bonus, path). The root logit
    and the fused features stay device tensors. The tree's node count is known
    on the host before the kernels run (the widths fix it).
    """

    def __init__(self, target, drafter, *, k: int, tree_top_k: int = 3, tree_max_nodes: int = 24):
        self.tm, self.drafter = target, drafter
        self.k = k
        w = beam_width(k, tree_top_k, tree_max_nodes)
        self.widths = [w] * k
        self.top_k = w
        self.T = w * k

    @torch.no_grad()
    def generate(self, prompt_ids: list[int], max_new_tokens: int, eos_token_id: int | None = None) -> GenResult:
        tm, dev = self.tm, self.tm.device
        seq = list(prompt_ids)
        base = len(seq)
        cache = tm.make_cache()
        cache.ensure_capacity(len(seq) + max_new_tokens + self.T + 1)
        pos = torch.arange(len(seq), device=dev).unsqueeze(0)
        logits, fused, cache = tm.forward_cached(torch.tensor(seq, device=dev).unsqueeze(0), cache, pos)
        feats = fused[0]
        cache_len = len(seq)
        root = logits[0, -1].contiguous()
        target_calls, drafter_calls, accepted, steps = 1, 0, 0, 0
        bonus = _argmax(root)
        seq.append(bonus)
        stop = eos_token_id is not None and bonus == eos_token_id
        T, V = self.T, tm.shape.vocab
        # the context only grows, so a drafter that can keep its cache across
        # calls (DeviceDrafter.draft_logits_extend) runs only the new rows
        draft = getattr(self.drafter, "draft_logits_extend", None) or self.drafter.draft_logits
        vlogits = torch.empty((T, V), dtype=tm.dtype, device=dev)
        vfused = torch.empty((T, tm.feature_dim), dtype=tm.dtype, device=dev)
        acc_out = torch.zeros(2 + T, dtype=torch.int32, device=dev)
        acc_scratch = torch.zeros(T + 2, dtype=torch.int32, device=dev)
        t0 = time.perf_counter()
        while len(seq) - base < max_new_tokens and not stop:
            ctx = torch.tensor(seq[:cache_len], device=dev)
            dl = draft(ctx, feats, self.k)
            drafter_calls += 1
            tokens, parents, pstatus = propose_tree_device(dl, self.widths, self.top_k)
            words = max(1, (T + 63) // 64)
            bits, npos, _ = ops.tree_masks(parents, cache_len, words, tm.status)
            tm.run_pass(tokens, npos, cache, _lib.PE_MASK_TREE, bits, vlogits, vfused)
            target_calls += 1
            ops.accept_tree(root, vlogits, tokens, parents, out=acc_out, scratch=acc_scratch)
            tm.commit_path(cache, cache_len, acc_out)
            out = acc_out.cpu().tolist()  # the step's one host read
            ops.read_status(tm.status, "speculative step")
            if int(pstatus.item()):
                raise _lib.PEError(int(pstatus.item()), "propose_tree")
            n, new_bonus, path = out[0], out[1], out[2: 2 + out[0]]
            if n:
                acc_tokens = tokens[torch.tensor(path, device=dev)].tolist()
                feats = torch.cat([feats, vfused[path]], dim=0)
                cache_len += n
                cache.seq_len = cache_len
                root = vlogits[path[-1]].clone()
                emit = [*acc_tokens[1:], int(new_bonus)]
                accepted += n - 1
            else:
                cache.seq_len = cache_len
                pending = seq[cache_len]
                blogits, bfused, cache = tm.forward_cached(torch.tensor([[pending]], device=dev), cache,
                                                           torch.tensor([[cache_len]], device=dev))
                target_calls += 1
                feats = torch.cat([feats, bfused[0]], dim=0)
                cache_len += 1
                root = blogits[0, -1].contiguous()
                emit = [_argmax(root)]
            steps += 1
            for tok in emit:
                seq.append(tok)
                if eos_token_id is not None and tok == eos_token_id:
                    stop = True
                    break
                if len(seq) - base >= max_new_tokens:
                    break
        torch.cuda.synchronize(dev)
        return GenResult(seq[base: base + max_new_tokens], steps, target_calls, drafter_calls, accepted,
                         min(len(seq) - base, max_new_tokens), time.perf_counter() - t0)
