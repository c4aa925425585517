"""The frozen target behind the reference's TargetModel API (src/pe/target.py:77-224).

``TargetModel.forward_cached`` is the masked verification forward: one call of
``pe_forward`` (libpe_hip.so) runs embeddings, every decoder layer with the
in-place K/V append, the final norm and lm_head on the device. ``gather_cache``
keeps the accepted path by moving only the rows that change. The cache is a
preallocated ``TreeKVCache`` ([L][nkv][capacity][hd] for K and V) with the
DynamicCache operations the reference's loop uses (``crop`` with absolute
length, ``get_seq_length``, ``layers[i].keys/.values``).

Signatures follow the reference so serve.py-style loops drive it unchanged;
``forward_cached`` additionally accepts ``parents=`` (the tree's parent list) to
build the ancestor bitmask on the device instead of reading a dense bias.
"""

from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from types import SimpleNamespace

import torch

from . import _lib, ops
from .config import ModelShape
from .model import DeviceModel


@dataclass
class TargetOutput:
    logits: torch.Tensor  # (B, S, V)
    fused: torch.Tensor  # (B, S, num_feature_layers * H)


class _LayerView:
    def __init__(self, cache: "TreeKVCache", layer: int):
        self._c, self._l = cache, layer

    @property
    def keys(self) -> torch.Tensor:
        return self._c.k[self._l, :, : self._c.seq_len].unsqueeze(0)

    @property
    def values(self) -> torch.Tensor:
        return self._c.v[self._l, :, : self._c.seq_len].unsqueeze(0)


class TreeKVCache:
    """Preallocated KV cache: K, V [L][nkv][capacity][hd] in the model dtype."""

    def __init__(self, shape: ModelShape, dtype: torch.dtype, device, capacity: int):
        self.shape = shape
        self.capacity = int(capacity)
        self.k = torch.zeros((shape.num_layers, shape.num_kv_heads, self.capacity, shape.head_dim), dtype=dtype,
                             device=device)
        self.v = torch.zeros_like(self.k)
        self.seq_len = 0
        self.fixed = False  # a view into a batch cache: it cannot grow

    @classmethod
    def view(cls, shape: ModelShape, k: torch.Tensor, v: torch.Tensor) -> "TreeKVCache":
        """A cache over existing K/V storage [L][nkv][capacity][hd] (one sequence
        of a BatchKVCache); it cannot be reallocated."""
        self = cls.__new__(cls)
        self.shape, self.k, self.v = shape, k, v
        self.capacity = int(k.shape[2])
        self.seq_len = 0
        self.fixed = True
        return self

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.seq_len

    def crop(self, max_length: int) -> None:
        """DynamicCache.crop (HF cache_utils.py:165-188): keep the first max_length
        rows; a negative value removes that many rows from the end."""
        if max_length < 0:
            max_length = self.seq_len - abs(max_length)
        if self.seq_len <= max_length:
            return
        self.seq_len = max(0, max_length)

    @property
    def layers(self) -> list[_LayerView]:
        return [_LayerView(self, i) for i in range(self.shape.num_layers)]

    def buffers(self) -> tuple[int, int, int]:
        """(K pointer, V pointer, capacity): what a captured step baked in."""
        return self.k.data_ptr(), self.v.data_ptr(), self.capacity

    def ensure_capacity(self, n: int) -> None:
        """Grow to at least ``n`` rows. Growing replaces the K/V buffers (a copy of
        the cached rows); a ``VerifyStep`` built on the old buffers refuses to run
        afterwards."""
        if n <= self.capacity:
            return
        if self.fixed:
            raise _lib.PEError(_lib.PE_ERR_CAPACITY, f"cache of {self.capacity} rows (part of a batch) needs {n}")
        cap = max(n, 2 * self.capacity)
        k = torch.zeros((self.k.shape[0], self.k.shape[1], cap, self.k.shape[3]), dtype=self.k.dtype,
                        device=self.k.device)
        v = torch.zeros_like(k)
        k[:, :, : self.seq_len] = self.k[:, :, : self.seq_len]
        v[:, :, : self.seq_len] = self.v[:, :, : self.seq_len]
        self.k, self.v, self.capacity = k, v, cap


class _SharedModule(torch.nn.Module):
    """A frozen module over the target's device tensors. The reference's drafter
    keeps these in tuples and only calls them (src/pe/drafter.py:81-83,120,123,
    161); ``to`` checks the request instead of copying, because the pass keeps
    pointers to the same tensors."""

    def __init__(self, weight: torch.Tensor):
        super().__init__()
        object.__setattr__(self, "_w", weight)

    @property
    def weight(self) -> torch.Tensor:
        return self._w

    def to(self, *args, **kwargs):
        dev, dt, _, _ = torch._C._nn._parse_to(*args, **kwargs)
        if dev is not None and torch.device(dev) != self._w.device and not (
                torch.device(dev).type == self._w.device.type and torch.device(dev).index is None):
            raise ValueError(f"shared target module lives on {self._w.device}")
        if dt is not None and dt != self._w.dtype:
            raise ValueError(f"shared target module computes in {self._w.dtype}")
        return self

    def requires_grad_(self, requires_grad: bool = True):
        return self

    def _rows(self, x: torch.Tensor, width: int) -> torch.Tensor:
        if not x.is_cuda:
            raise ValueError("parallel_eagle_amd modules take HIP device tensors")
        if x.dtype != self._w.dtype:
            raise TypeError(f"expected {self._w.dtype} input, got {x.dtype}")
        if x.shape[-1] != width:
            raise ValueError(f"expected last dimension {width}, got {x.shape[-1]}")
        return x.reshape(-1, width).contiguous()


class DeviceEmbedding(_SharedModule):
    """The target's embed_tokens (HF modeling_llama.py:381): ids of any shape ->
    rows (*ids.shape, H), gathered by pe_embed; an id outside the vocabulary
    raises."""

    def __init__(self, weight: torch.Tensor, status: torch.Tensor):
        super().__init__(weight)
        object.__setattr__(self, "_status", status)

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        ids = torch.as_tensor(ids, device=self._w.device)
        flat = ids.reshape(-1).to(torch.int64).contiguous()
        out = ops.embed(flat, self._w, self._status)
        ops.read_status(self._status, "embedding")
        return out.view(*ids.shape, self._w.shape[1])


class DeviceRMSNorm(_SharedModule):
    """The target's final norm (HF LlamaRMSNorm, modeling_llama.py:62-67):
    ``w * round(x * rsqrt(mean(x^2) + eps))`` with fp32 statistics, by pe_rmsnorm."""

    def __init__(self, weight: torch.Tensor, eps: float):
        super().__init__(weight)
        self.variance_epsilon = float(eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = self._rows(x, self._w.shape[0])
        return ops.rmsnorm(rows, self._w, self.variance_epsilon).view(x.shape)


class DeviceLMHead(_SharedModule):
    """The target's lm_head (HF modeling_llama.py:480, ``F.linear`` without bias):
    hidden (*, H) -> logits (*, V) in the model dtype, by pe_dense_gemm on the
    tiled weight. ``weight`` is the logical [V][H] matrix."""

    def __init__(self, logical: torch.Tensor, tiled: torch.Tensor):
        super().__init__(logical)
        object.__setattr__(self, "_tiled", tiled)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        v, h = self._w.shape
        rows = self._rows(x, h)
        return ops.linear(rows, v, dense=self._tiled).view(*x.shape[:-1], v)


class TargetModel:
    """Frozen target on the HIP device (mirror of src/pe/target.py:77-224)."""

    def __init__(self, model: DeviceModel, tokenizer=None, cache_capacity: int | None = None):
        self.model = model
        self.shape = model.shape
        self.dtype = model.dtype
        self.tokenizer = tokenizer
        self.feature_layers = self.shape.resolved_feature_layers()
        self.cache_capacity = cache_capacity or min(self.shape.max_positions, 4096)
        self._ws = None
        self._ws_key = (0, 0)
        self.status = torch.zeros(4, dtype=torch.int32, device=model.device)
        self.check_status = True

    @classmethod
    def synthetic(cls, shape: ModelShape, seed: int = 0, device="cuda", **kw) -> "TargetModel":
        keep = kw.pop("keep_logical", False)
        noise = kw.pop("norm_noise", 0.0)
        return cls(DeviceModel.synthetic(shape, seed, device, keep_logical=keep, norm_noise=noise), **kw)

    @classmethod
    def from_bnb_state_dict(cls, shape: ModelShape, state_dict: dict, device="cuda", **kw) -> "TargetModel":
        """A pre-quantized bitsandbytes NF4 checkpoint (the state dict of the model
        src/pe/target.py:32-38 loads), run with the fp32-absmax kernels."""
        from . import bnb

        keep = kw.pop("keep_logical", False)
        weights = bnb.weights_from_state_dict(shape, state_dict, device)
        return cls(DeviceModel.from_weights(shape, weights, device, keep_logical=keep), **kw)

    # ------------------------------------------------------------ attributes of the reference API
    @property
    def config(self):
        s = self.shape
        return SimpleNamespace(num_hidden_layers=s.num_layers, hidden_size=s.hidden, num_attention_heads=s.num_heads,
                               num_key_value_heads=s.num_kv_heads, head_dim=s.head_dim,
                               intermediate_size=s.intermediate, vocab_size=s.vocab, rms_norm_eps=s.rms_eps,
                               rope_theta=s.rope_theta)

    @property
    def hidden_size(self) -> int:
        return self.shape.hidden

    @property
    def vocab_size(self) -> int:
        return self.shape.vocab

    @property
    def num_feature_layers(self) -> int:
        return len(self.feature_layers)

    @property
    def feature_dim(self) -> int:
        return self.hidden_size * self.num_feature_layers

    @property
    def device(self) -> torch.device:
        return self.model.device

    def get_input_embeddings(self) -> DeviceEmbedding:
        """Callable embedding module over the device table (target.py:150-151)."""
        return DeviceEmbedding(self.model.embed, torch.zeros(4, dtype=torch.int32, device=self.device))

    def get_lm_head(self) -> DeviceLMHead:
        """Callable lm_head module (target.py:153-154)."""
        return DeviceLMHead(self.model.lm_head_logical, self.model.lm_head)

    def get_final_norm(self) -> DeviceRMSNorm:
        """Callable final RMSNorm with HF rounding (target.py:156-159)."""
        return DeviceRMSNorm(self.model.final_norm, self.shape.rms_eps)

    # ------------------------------------------------------------ cache
    def make_cache(self, capacity: int | None = None) -> TreeKVCache:
        return TreeKVCache(self.shape, self.dtype, self.device, capacity or self.cache_capacity)

    def gather_cache(self, cache: TreeKVCache, keep_index: torch.Tensor) -> None:
        """Keep only ``keep_index`` rows (sequence axis) of every layer's K/V, in place.
        ``keep_index`` must be strictly increasing (as serve.py:308-309 builds it)."""
        keep = torch.as_tensor(keep_index, device=self.device).to(torch.int64).contiguous()
        ops.kv_gather(cache.k, cache.v, keep, self.status)
        if self.check_status:
            ops.read_status(self.status, "gather_cache")
        cache.seq_len = keep.numel()

    def commit_path(self, cache: TreeKVCache, prefix_len: int, accept_out: torch.Tensor) -> None:
        """Device-side commit of an ``accept_tree`` result: rows P + path[i] -> P + i.
        The caller sets ``cache.seq_len`` from the (host-read) path length."""
        ops.kv_compact(cache.k, cache.v, prefix_len, accept_out)

    # ------------------------------------------------------------ forward
    def _workspace(self, m: int, kv_len: int) -> torch.Tensor:
        need = self.model.workspace_bytes(m, kv_len)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.zeros(need + (1 << 20), dtype=torch.uint8, device=self.device)
        return self._ws

    def _tree_bits_from_parents(self, parents, prefix_len: int):
        t = len(parents)
        words = max(1, math.ceil(t / 64))
        if words > _lib.PE_TREE_MAX_WORDS:
            raise ValueError(f"tree of {t} nodes exceeds {64 * _lib.PE_TREE_MAX_WORDS}")
        par = torch.as_tensor(list(parents), dtype=torch.int32).to(self.device, non_blocking=True)
        bits, pos, _ = ops.tree_masks(par, prefix_len, words, self.status)
        return bits, pos

    def run_pass(self, ids: torch.Tensor, pos: torch.Tensor, cache: TreeKVCache, mask_mode: int,
                 bits: torch.Tensor | None, logits: torch.Tensor | None, fused: torch.Tensor | None) -> None:
        """Launch one pe_forward on the current stream (no host sync)."""
        m = ids.numel()
        prefix = cache.seq_len
        ws = self._workspace(m, prefix + m)
        a = _lib.PassArgs()
        a.input_ids, a.positions, a.M, a.mask_mode, a.prefix_len = ids.data_ptr(), pos.data_ptr(), m, mask_mode, prefix
        a.tree_bits = bits.data_ptr() if bits is not None else None
        a.bits_words = bits.shape[1] if bits is not None else 0
        fl = self.feature_layers
        a.num_features = len(fl) if fused is not None else 0
        for i, f in enumerate(fl[:4]):
            a.feature_layers[i] = f
        a.k_cache, a.v_cache, a.cache_capacity = cache.k.data_ptr(), cache.v.data_ptr(), cache.capacity
        a.logits = logits.data_ptr() if logits is not None else None
        a.fused = fused.data_ptr() if fused is not None else None
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        a.status = self.status.data_ptr()
        _lib.check(_lib.load().pe_forward(C.byref(self.model.desc()), C.byref(a), ops.stream_ptr()), "pe_forward")

    @torch.no_grad()
    def forward_cached(self, input_ids: torch.Tensor, past_key_values: TreeKVCache, position_ids: torch.Tensor,
                       attention_mask: torch.Tensor | None = None, *, parents=None):
        """Incremental forward over the new ``input_ids`` (1, T) attending to the cache.
        ``attention_mask``: 4-D additive bias (1, 1, T, P + T) for a tree, or None for
        causal continuation; ``parents`` (list) builds the tree mask on the device.
        Returns (logits (1, T, V), fused (1, T, F*H), cache)."""
        cache = past_key_values
        ids = torch.as_tensor(input_ids, device=self.device).reshape(-1).to(torch.int64).contiguous()
        pos = torch.as_tensor(position_ids, device=self.device).reshape(-1).to(torch.int64).contiguous()
        m = ids.numel()
        if pos.numel() != m:
            raise ValueError("position_ids must have one entry per input id")
        prefix = cache.seq_len
        cache.ensure_capacity(prefix + m)
        if parents is not None:
            if len(parents) != m:
                raise ValueError("parents must have one entry per input id")
            bits, _ = self._tree_bits_from_parents(parents, prefix)
            mode = _lib.PE_MASK_TREE
        elif attention_mask is not None:
            bias = attention_mask.reshape(attention_mask.shape[-2], attention_mask.shape[-1])
            if bias.shape != (m, prefix + m):
                raise ValueError(f"attention_mask must be (1, 1, {m}, {prefix + m})")
            words = max(1, math.ceil(m / 64))
            bits = ops.bias_to_bits(bias.to(self.device).contiguous(), prefix, words, self.status)
            mode = _lib.PE_MASK_TREE
        else:
            bits, mode = None, _lib.PE_MASK_CAUSAL
        logits = torch.empty((m, self.shape.vocab), dtype=self.dtype, device=self.device)
        fused = torch.empty((m, self.feature_dim), dtype=self.dtype, device=self.device)
        self.run_pass(ids, pos, cache, mode, bits, logits, fused)
        cache.seq_len = prefix + m
        if self.check_status:
            try:
                ops.read_status(self.status, "forward_cached")
            except _lib.PEError:
                cache.seq_len = prefix
                raise
        return logits.view(1, m, -1), fused.view(1, m, -1), cache

    def verify_step(self, cache: TreeKVCache, tree_nodes: int) -> "VerifyStep":
        """A device-resident verification step over ``cache`` at its current length."""
        return VerifyStep(self, cache, tree_nodes)

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None,
                position_ids: torch.Tensor | None = None) -> TargetOutput:
        """Recompute forward without a cache (src/pe/target.py:168-188). A 4-D bias
        must be the [prefix causal | tree] mask of tree_allow_mask: the leading
        causal rows run as a prefill and the rest as a tree pass over them."""
        ids = torch.as_tensor(input_ids, device=self.device).reshape(-1).to(torch.int64)
        s = ids.numel()
        pos = (torch.arange(s, device=self.device) if position_ids is None
               else torch.as_tensor(position_ids, device=self.device).reshape(-1).to(torch.int64))
        cache = self.make_cache(capacity=s)
        if attention_mask is None:
            lg, fu, _ = self.forward_cached(ids, cache, pos)
            return TargetOutput(lg, fu)
        bias = attention_mask.reshape(s, s).to(self.device)
        allow = bias == 0
        causal = torch.tril(torch.ones((s, s), dtype=torch.bool, device=self.device))
        row_causal = (allow == causal).all(dim=1)
        not_causal = (~row_causal).nonzero()
        p = int(not_causal[0]) if not_causal.numel() else s
        parts_l, parts_f = [], []
        if p > 0:
            lg, fu, _ = self.forward_cached(ids[:p], cache, pos[:p])
            parts_l.append(lg)
            parts_f.append(fu)
        if p < s:
            lg, fu, _ = self.forward_cached(ids[p:], cache, pos[p:], bias[p:, :].reshape(1, 1, s - p, s))
            parts_l.append(lg)
            parts_f.append(fu)
        return TargetOutput(torch.cat(parts_l, 1), torch.cat(parts_f, 1))


class VerifyStep:
    """One tree-verification step with every buffer preallocated, so it can be
    enqueued without a host synchronisation and captured in a HIP graph.

    It performs, on the device and in order, what one iteration of the
    reference's cached tree loop does between proposing the tree and emitting
    tokens (src/pe/serve.py:292-314):

    1. ``pe_tree_masks``: ancestor bitmasks and positions P + depth from the
       parent list (masks.py:118-156 without the dense (P+T)^2 matrix),
    2. ``pe_forward``: the masked verification forward over the cache with the
       in-place K/V append (target.py:203-224),
    3. ``pe_accept_tree_keys``: the greedy walk against the root logit
       (decode/verify.py:104-125), each node row's argmax taken from the keys
       the lm_head wrote with the logits (16-bit models; fp32 models re-read
       the rows with ``pe_accept_tree``),
    4. ``pe_kv_compact``: the accepted rows move to P, P+1, ... in place
       (target.py:194-201 with the keep index of serve.py:308-309).

    Inputs live in static device buffers (``load_tree`` fills them); ``result``
    reads back (path, bonus) and ``commit`` sets the cache length. The prefix
    length P is fixed at construction: a step replayed at the same P rewrites
    rows [P, P + T) and leaves [0, P) untouched.
    """

    def __init__(self, target: TargetModel, cache: TreeKVCache, tree_nodes: int):
        self.tm, self.cache, self.T = target, cache, int(tree_nodes)
        dev, s = target.device, target.shape
        self.P = cache.seq_len
        cache.ensure_capacity(self.P + self.T)
        self.words = max(1, math.ceil(self.T / 64))
        if self.words > _lib.PE_TREE_MAX_WORDS:
            raise ValueError(f"tree of {self.T} nodes exceeds {64 * _lib.PE_TREE_MAX_WORDS}")
        self.ids = torch.zeros(self.T, dtype=torch.int64, device=dev)
        self.parents = torch.full((self.T,), -1, dtype=torch.int32, device=dev)
        self.bits = torch.zeros((self.T, self.words), dtype=torch.int64, device=dev)
        self.pos = torch.zeros(self.T, dtype=torch.int64, device=dev)
        self.depth = torch.zeros(self.T, dtype=torch.int32, device=dev)
        self.root_logit = torch.zeros(s.vocab, dtype=target.dtype, device=dev)
        self.logits = torch.empty((self.T, s.vocab), dtype=target.dtype, device=dev)
        self.fused = torch.empty((self.T, target.feature_dim), dtype=target.dtype, device=dev)
        self.accept_out = torch.zeros(2 + self.T, dtype=torch.int32, device=dev)
        self.accept_scratch = torch.zeros(self.T + 2, dtype=torch.int32, device=dev)
        self.ws = torch.zeros(target.model.workspace_bytes(self.T, self.P + self.T), dtype=torch.uint8,
                              device=dev)
        # the lm_head's per-row argmax keys (16-bit models): [T][groups] uint64
        # (trees of more than 64 nodes run as a batch of one and walk the rows)
        self.key_groups = 0 if (target.dtype == torch.float32 or self.T > 64) else int(
            _lib.load().pe_dense_gemm_argmax_groups(self.T, s.vocab, s.hidden))
        self.node_keys = (torch.zeros((self.T, self.key_groups), dtype=torch.int64, device=dev)
                          if self.key_groups > 0 else None)
        self.graph = None
        a = _lib.PassArgs()
        a.input_ids, a.positions, a.M, a.mask_mode, a.prefix_len = (self.ids.data_ptr(), self.pos.data_ptr(),
                                                                     self.T, _lib.PE_MASK_TREE, self.P)
        a.tree_bits, a.bits_words = self.bits.data_ptr(), self.words
        fl = target.feature_layers
        a.num_features = len(fl)
        for i, f in enumerate(fl[:4]):
            a.feature_layers[i] = f
        a.k_cache, a.v_cache, a.cache_capacity = cache.k.data_ptr(), cache.v.data_ptr(), cache.capacity
        a.logits, a.fused = self.logits.data_ptr(), self.fused.data_ptr()
        a.workspace, a.workspace_bytes = self.ws.data_ptr(), self.ws.numel()
        a.status = target.status.data_ptr()
        a.node_keys = self.node_keys.data_ptr() if self.node_keys is not None else None
        self._args = a
        self._buffers = cache.buffers()

    def _check_cache(self) -> None:
        """The pass arguments hold the cache's K/V pointers and capacity from
        construction; a cache that has grown since (ensure_capacity replaced the
        buffers) would be written through freed memory."""
        if self.cache.buffers() != self._buffers:
            raise RuntimeError("the KV cache was reallocated after this VerifyStep was built; build a new step")

    def load_tree(self, node_tokens, parents, root_logit: torch.Tensor) -> None:
        """Copy a tree and the root logit into the static buffers (stream-ordered)."""
        if len(node_tokens) != self.T or len(parents) != self.T:
            raise ValueError(f"tree must have {self.T} nodes")
        self.ids.copy_(torch.as_tensor(list(node_tokens), dtype=torch.int64))
        self.parents.copy_(torch.as_tensor(list(parents), dtype=torch.int32))
        self.root_logit.copy_(root_logit.reshape(-1))

    def launch(self) -> None:
        """Enqueue masks -> forward -> acceptance -> compaction on the current stream."""
        self._check_cache()
        L, st = _lib.load(), ops.stream_ptr()
        c, s = self.cache, self.tm.shape
        _lib.check(L.pe_tree_masks(self.parents.data_ptr(), self.T, self.P, self.bits.data_ptr(), self.words,
                                   self.pos.data_ptr(), self.depth.data_ptr(), self.tm.status.data_ptr(), st),
                   "pe_tree_masks")
        _lib.check(L.pe_forward(C.byref(self.tm.model.desc()), C.byref(self._args), st), "pe_forward")
        if self.node_keys is not None:
            _lib.check(L.pe_accept_tree_keys(self.root_logit.data_ptr(), s.vocab, ops.dcode(self.tm.dtype),
                                             self.node_keys.data_ptr(), self.key_groups, self.T, self.ids.data_ptr(),
                                             self.parents.data_ptr(), self.accept_out.data_ptr(),
                                             self.accept_scratch.data_ptr(), st), "pe_accept_tree_keys")
        else:
            _lib.check(L.pe_accept_tree(self.root_logit.data_ptr(), self.logits.data_ptr(), s.vocab, self.T,
                                        s.vocab, ops.dcode(self.tm.dtype), self.ids.data_ptr(),
                                        self.parents.data_ptr(), self.accept_out.data_ptr(),
                                        self.accept_scratch.data_ptr(), st), "pe_accept_tree")
        _lib.check(L.pe_kv_compact(c.k.data_ptr(), c.v.data_ptr(), s.num_layers, s.num_kv_heads, c.capacity,
                                   s.head_dim, ops.dcode(self.tm.dtype), self.P, self.accept_out.data_ptr(), st),
                   "pe_kv_compact")

    def capture(self) -> None:
        """Record ``launch`` into a HIP graph (run it eagerly once first)."""
        self.launch()
        torch.cuda.synchronize(self.tm.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.launch()
        self.graph = g

    def run(self) -> None:
        self._check_cache()
        if self.graph is not None:
            self.graph.replay()
        else:
            self.launch()

    def result(self) -> tuple[list[int], int]:
        """(accepted node indices, bonus token); synchronises with the stream."""
        out = self.accept_out.cpu().tolist()
        ops.read_status(self.tm.status, "verify step")
        n = out[0]
        return out[2: 2 + n], out[1]

    def commit(self, path_len: int) -> None:
        self.cache.seq_len = self.P + path_len
