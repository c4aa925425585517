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

    def ensure_capacity(self, n: int) -> None:
        if n <= self.capacity:
            return
        cap = max(n, 2 * self.capacity)
        k = torch.zeros((self.k.shape[0], self.k.shape[1], cap, self.k.shape[3]), dtype=self.k.dtype,
                        device=self.k.device)
        v = torch.zeros_like(k)
        k[:, :, : self.seq_len] = self.k[:, :, : self.seq_len]
        v[:, :, : self.seq_len] = self.v[:, :, : self.seq_len]
        self.k, self.v, self.capacity = k, v, cap


class _Module:
    def __init__(self, weight):
        self.weight = weight


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

    def get_input_embeddings(self):
        return _Module(self.model.embed)

    def get_lm_head(self):
        return _Module(self.model.lm_head_logical)

    def get_final_norm(self):
        return _Module(self.model.final_norm)

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
