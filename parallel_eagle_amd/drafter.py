"""The drafter's forward on the device, with the API of ParallelDrafter.draft_logits
(src/pe/drafter.py:195-236).

The drafter's decoder layers are Llama layers (src/pe/nn.py:103-124), so its
forward is the target's pass (``pe_forward``) over a second layer stack: dense
layers in the target's dtype, the target's final norm and lm_head shared (the
same device tensors, as the reference shares the modules).

The reference's draft mask (real rows causal; the k - 1 mask slots see every
real row and the slots up to their own) and its positions (0..p-1, then
(p - 1) + d) are those of one causal pass over the p + k - 1 rows from an empty
cache, which is how it runs here (the p - 1 context rows without logits, then the k
rows whose logits are read as a causal continuation). The rows are the drafter's inputs, not token
embeddings: the layer stack's embedding table is a buffer of input rows that
the pass gathers with ids 0..m-1.

Inputs (drafter.py:126-138): ``in_proj([embed(token); feat_proj(feat_norm(feature
blocks))])`` for real positions, ``in_proj([mask_emb; h_shared])`` for mask
slots (computed once). The drafter's own norms (feat_norm and each layer's two)
multiply by the weight in fp32 and round once, as the reference's RMSNorm does
(src/pe/nn.py:22-26, PE_NORM_FP32_WEIGHT); the shared final norm is the
target's HF LlamaRMSNorm (the normalised row rounded, then the weight multiply).
Its attention is the reference drafter's explicit softmax (src/pe/nn.py:84-87,
PE_ATTN_EAGER): scores rounded to the dtype, probabilities normalised and
rounded before the PV product.
"""

from __future__ import annotations

from dataclasses import replace

import torch

from . import _lib, ops
from .model import DeviceModel
from .target import TargetModel, TreeKVCache


class DeviceDrafter:
    """``target``: the TargetModel whose embed, final norm and lm_head the drafter
    shares. ``weights``: {"feat_norm" [H], "feat_proj" [H][F], "in_proj" [H][2H],
    "mask_emb" [H], "h_shared" [H], "layers": [{"attn_norm", "mlp_norm", "q", "k",
    "v", "o", "gate", "up", "down"}]} (host or device tensors, logical [N][K]).
    ``capacity``: the most rows (context + k - 1) one call may run."""

    def __init__(self, target: TargetModel, weights: dict, max_depth: int, capacity: int = 4096):
        tm = target.model
        s = tm.shape
        dev, dt = tm.device, tm.dtype
        self.target = target
        self.max_depth = max_depth
        self.hidden = s.hidden
        self.eps = s.rms_eps
        self.dtype = dt
        self.device = dev
        n_layers = len(weights["layers"])
        self.shape = replace(s, name=f"{s.name}-drafter", num_layers=n_layers, weight_format="dense", qkv_bias=False,
                             feature_layers=(n_layers,))
        self.capacity = capacity

        def up(x):
            return torch.as_tensor(x).to(device=dev, dtype=dt).contiguous()

        def tile(x):
            x = up(x)
            return ops.dense_repack(x) if dt != torch.float32 else x

        self.feat_norm = up(weights["feat_norm"])
        self.feat_dim = int(weights["feat_proj"].shape[1])
        if self.feat_dim % s.hidden:
            raise ValueError("feat_proj's input width must be a multiple of hidden")
        self.feat_proj = tile(weights["feat_proj"])
        self.in_proj = tile(weights["in_proj"])
        mask_in = torch.cat([up(weights["mask_emb"]), up(weights["h_shared"])]).view(1, -1)
        self.mask_vec = ops.linear(mask_in, s.hidden, dense=self.in_proj).view(-1)

        core = DeviceModel(self.shape, dev)
        core.embed = torch.zeros((capacity, s.hidden), dtype=dt, device=dev)  # the call's input rows
        core.final_norm = tm.final_norm
        core.lm_head, core.lm_head_logical = tm.lm_head, tm.lm_head_logical
        core.logical = None
        for lw in weights["layers"]:
            core._add_layer({k: up(v) for k, v in lw.items()}, False)
        core.norm_mode = _lib.PE_NORM_FP32_WEIGHT
        core.attn_mode = _lib.PE_ATTN_EAGER
        core._finish()
        self.core = core
        self.runner = TargetModel(core, cache_capacity=capacity)
        self.cache = TreeKVCache(self.shape, dt, dev, capacity)
        self.rows = torch.arange(capacity, dtype=torch.int64, device=dev)
        self._valid = 0  # context rows of the last call whose K/V are in self.cache
        # False: calls leave their status word for the caller to read (a decode
        # loop folds it into its one read per step) instead of synchronising
        self.sync_status = True

    @property
    def status(self) -> torch.Tensor:
        """The device int32 status word the drafter's kernels report errors in."""
        return self.runner.status

    def reset(self) -> None:
        """Forget the cached context: the next ``draft_logits_extend`` runs its whole
        context (a new prompt is not an extension of the last one)."""
        self._valid = 0

    # nn.Module-style calls the reference's callers chain after load_drafter
    # (bench/run_bench.py:57: ``load_drafter(path, target).to(device, dtype).eval()``):
    # the weights already live on the target's device in its dtype, so these
    # check the request and return the drafter itself.
    def to(self, *args, **kwargs) -> "DeviceDrafter":
        dev, dt, _, _ = torch._C._nn._parse_to(*args, **kwargs)
        if dev is not None:
            want = torch.device(dev)
            if want.type != self.device.type or (want.index is not None and want.index != self.device.index):
                raise ValueError(f"the device drafter lives on {self.device}, not {want}")
        if dt is not None and dt != self.dtype:
            raise ValueError(f"the device drafter computes in its target's dtype {self.dtype}, not {dt}")
        return self

    def eval(self) -> "DeviceDrafter":
        return self

    def train(self, mode: bool = True) -> "DeviceDrafter":
        if mode:
            raise ValueError("the device drafter runs inference only")
        return self

    def real_input(self, token_ids: torch.Tensor, features: torch.Tensor) -> torch.Tensor:
        """in_proj([embed(token); feat_proj(feat_norm(features))]) (drafter.py:126-133)."""
        H = self.hidden
        ids = torch.as_tensor(token_ids, device=self.device).reshape(-1).to(torch.int64).contiguous()
        p = ids.numel()
        emb = ops.embed(ids, self.target.model.embed, self.runner.status)
        f = features.to(device=self.device, dtype=self.dtype).reshape(p * (self.feat_dim // H), H).contiguous()
        f = ops.rmsnorm(f, self.feat_norm, self.eps, mode=_lib.PE_NORM_FP32_WEIGHT).view(p, self.feat_dim)
        # pe_dense_gemm: more than 256 rows run the many-row kernel (each weight
        # read once per 256 rows)
        feat = ops.linear(f, H, dense=self.feat_proj)
        return ops.linear(torch.cat([emb, feat], dim=-1).contiguous(), H, dense=self.in_proj)

    @torch.no_grad()
    def draft_logits(self, context_ids: torch.Tensor, context_feats: torch.Tensor, k: int) -> torch.Tensor:
        """Logits (k, V) for the k tokens after ``context_ids``: row 0 from the last
        real slot, row d from mask slot d."""
        return self._draft(context_ids, context_feats, k, reuse=False)

    @torch.no_grad()
    def draft_logits_extend(self, context_ids: torch.Tensor, context_feats: torch.Tensor, k: int) -> torch.Tensor:
        """``draft_logits`` for a context that extends the previous call's (its
        tokens and features are the previous context's, followed by new ones, as
        in a decode loop): the K/V rows of the previous context stay in the
        drafter's cache (the attention is causal, so a row's K/V depend only on
        the rows before it) and only the new rows and the k query slots run. The
        caller guarantees the prefix (``reset`` before a context that does not
        extend the last one); the logits equal a full recomputation up to the
        rounding of the different launch shapes (exactly, in fp32)."""
        return self._draft(context_ids, context_feats, k, reuse=True)

    def _draft(self, context_ids, context_feats, k: int, reuse: bool) -> torch.Tensor:
        ids = torch.as_tensor(context_ids, device=self.device).reshape(-1)
        p = ids.numel()
        m = p + k - 1
        if p < 1 or k < 1:
            raise ValueError("draft_logits needs a context and k >= 1")
        if m > self.capacity:
            raise ValueError(f"{m} drafter rows exceed the capacity {self.capacity}")
        # rows [0, kept) of the cache hold this context's K/V from the previous call
        kept = min(self._valid, p - 1) if reuse else 0
        x = self.core.embed
        x[kept:p].copy_(self.real_input(ids[kept:], context_feats[kept:p]))
        if k > 1:
            x[p:m].copy_(self.mask_vec.expand(k - 1, -1))
        # rows [kept, p - 1) only fill the cache (no lm_head); the k rows whose
        # logits are read continue it causally: the same attention as one pass
        # over m rows
        rows = self.rows
        self.cache.seq_len = kept
        self._valid = 0  # until this call has written its rows
        if p - 1 > kept:
            self.runner.run_pass(rows[kept: p - 1], rows[kept: p - 1], self.cache, _lib.PE_MASK_CAUSAL, None, None,
                                 None)
            self.cache.seq_len = p - 1
        logits = torch.empty((k, self.shape.vocab), dtype=self.dtype, device=self.device)
        self.runner.run_pass(rows[p - 1: m], rows[p - 1: m], self.cache, _lib.PE_MASK_CAUSAL, None, logits, None)
        if self.sync_status:
            ops.read_status(self.runner.status, "draft_logits")
        self._valid = p  # rows [0, p) are this context's (the mask slots after it are not)
        return logits


_LAYER_KEYS = {"attn_norm": "input_norm.weight", "mlp_norm": "post_norm.weight", "q": "attn.q_proj.weight",
               "k": "attn.k_proj.weight", "v": "attn.v_proj.weight", "o": "attn.o_proj.weight",
               "gate": "mlp.gate_proj.weight", "up": "mlp.up_proj.weight", "down": "mlp.down_proj.weight"}


def weights_from_state_dict(sd: dict, num_layers: int) -> dict:
    """The drafter's weights by ParallelDrafter's parameter names (src/pe/drafter.py:62-76,
    src/pe/nn.py:59-117) in DeviceDrafter's layout."""
    def get(key):
        if key not in sd:
            raise KeyError(f"drafter state dict has no {key!r}")
        return sd[key]

    w = {"feat_norm": get("feat_norm.weight"), "feat_proj": get("feat_proj.weight"), "in_proj": get("in_proj.weight"),
         "mask_emb": get("mask_emb"), "h_shared": get("h_shared")}
    w["layers"] = [{ours: get(f"layers.{i}.{theirs}") for ours, theirs in _LAYER_KEYS.items()}
                   for i in range(num_layers)]
    return w


def load_drafter(path, target: TargetModel, capacity: int = 4096) -> DeviceDrafter:
    """load_drafter (src/pe/drafter.py:289-299) onto the device: the checkpoint's
    {"state_dict", "num_layers", "max_depth", ...} read without executing anything
    from the file (weights_only), sharing ``target``'s embed / final norm / lm_head."""
    from pathlib import Path
    if not Path(path).exists():
        raise FileNotFoundError(f"No drafter checkpoint at {path}")
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    w = weights_from_state_dict(ckpt["state_dict"], int(ckpt["num_layers"]))
    return DeviceDrafter(target, w, max_depth=int(ckpt["max_depth"]), capacity=capacity)
