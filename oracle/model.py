"""Llama / Qwen2 causal-LM forward on the CPU with the reference's numerics
(oracle; test infrastructure only).

TargetModel.forward_cached (src/pe/target.py:203-224) runs the HF model with a
DynamicCache, explicit position ids and an optional 4-D additive bias, and
returns (logits, fused features, cache). This module restates that forward op
for op, in the same dtype and the same order, so it reproduces transformers 5.x
bit for bit on the CPU:

- embeddings                       HF modeling_llama.py:381
- RoPE cos/sin (fp32, then dtype)   HF modeling_llama.py:93-127
- RMSNorm                          HF modeling_llama.py:62-67
- q/k/v/o (+ q/k/v bias for Qwen2)  HF modeling_llama.py:254-256,280; modeling_qwen2.py:189-192
- apply_rotary_pos_emb             HF modeling_llama.py:130-160
- KV append (torch.cat)            HF cache_utils.py:127-146
- SDPA dispatch                    HF integrations/sdpa_attention.py:79-154
- SwiGLU MLP, residual adds        HF modeling_llama.py:174-176,317,323
- final norm, lm_head, features    HF modeling_llama.py:413,477-480; utils/output_capturing.py:269-277;
                                   src/pe/target.py:161-162

NF4 linears are dequantised to bf16 on every call and multiplied with F.linear,
as bitsandbytes' Linear4bit does for inputs of more than one token.

Pinned by tests/test_oracle_model.py against transformers' LlamaForCausalLM and
Qwen2ForCausalLM built locally (no hub access) with the same weights.
"""

from __future__ import annotations

import time
from collections import defaultdict
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import nf4

DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


@dataclass
class StageTimer:
    seconds: dict = field(default_factory=lambda: defaultdict(float))
    enabled: bool = False

    def add(self, key: str, t0: float) -> float:
        t1 = time.perf_counter()
        if self.enabled:
            self.seconds[key] += t1 - t0
        return t1


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    dt = x.dtype
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return w * h.to(dt)


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_cos_sin(inv: torch.Tensor, position_ids: torch.Tensor, dtype: torch.dtype):
    inv_e = inv[None, :, None].float().expand(position_ids.shape[0], -1, 1)
    pos_e = position_ids[:, None, :].float()
    freqs = (inv_e.float() @ pos_e.float()).transpose(1, 2)
    emb = torch.cat((freqs, freqs), dim=-1)
    cos = emb.cos() * 1.0
    sin = emb.sin() * 1.0
    return cos.to(dtype=dtype), sin.to(dtype=dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    b, nkv, s, hd = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, nkv, n_rep, s, hd).reshape(b, nkv * n_rep, s, hd)


class OracleTarget:
    """CPU restatement of the target forward.

    ``weights``: {"embed", "final_norm", "lm_head", "layers": [{"attn_norm",
    "mlp_norm", "q", "k", "v", "o", "gate", "up", "down", optional "q_bias",
    "k_bias", "v_bias"}]}; each linear is a dense [N][K] tensor in the compute
    dtype or ("nf4", packed uint8 [N][K/2], absmax fp16 [N][K/64]).
    """

    def __init__(self, shape, weights: dict, timer: StageTimer | None = None):
        self.shape = shape
        self.w = weights
        self.dtype = DTYPES[shape.dtype]
        self.inv_freq = inv_freq(shape.head_dim, shape.rope_theta)
        self.feature_layers = shape.resolved_feature_layers()
        self.timer = timer or StageTimer()
        self._deq_cache: dict = {}
        self.cache_dequant = False

    # -- linears
    def _weight(self, spec) -> torch.Tensor:
        if isinstance(spec, tuple) and spec[0] == "nf4":
            key = id(spec)
            if self.cache_dequant and key in self._deq_cache:
                return self._deq_cache[key]
            t0 = time.perf_counter()
            w = nf4.dequantize_torch(spec[1], spec[2])
            self.timer.add("dequant", t0)
            if self.cache_dequant:
                self._deq_cache[key] = w
            return w
        return spec

    def linear(self, x: torch.Tensor, spec, bias=None) -> torch.Tensor:
        w = self._weight(spec)
        t0 = time.perf_counter()
        y = F.linear(x, w, bias)
        self.timer.add("matmul", t0)
        return y

    # -- forward
    @torch.no_grad()
    def forward(self, input_ids, position_ids, cache: list | None, attention_mask: torch.Tensor | None):
        """input_ids, position_ids: int64 [M] (or lists). cache: list of (K, V)
        tensors (1, nkv, S, hd) or None for an empty cache. attention_mask: 4-D
        additive bias (1, 1, M, S + M) or None (causal continuation).
        Returns logits (1, M, V), fused (1, M, nf*H), the new cache list."""
        s = self.shape
        ids = torch.as_tensor(input_ids, dtype=torch.long).reshape(1, -1)
        pos = torch.as_tensor(position_ids, dtype=torch.long).reshape(1, -1)
        M = ids.shape[1]
        L = s.num_layers
        if cache is None:
            cache = [None] * L
        hidden = self.w["embed"][ids]
        states = [hidden]
        cos, sin = rope_cos_sin(self.inv_freq, pos, self.dtype)
        cos_u, sin_u = cos.unsqueeze(1), sin.unsqueeze(1)
        scaling = s.head_dim ** -0.5
        new_cache = []
        for li in range(L):
            lw = self.w["layers"][li]
            residual = hidden
            x = rms_norm(hidden, lw["attn_norm"], s.rms_eps)
            q = self.linear(x, lw["q"], lw.get("q_bias")).view(1, M, -1, s.head_dim).transpose(1, 2)
            k = self.linear(x, lw["k"], lw.get("k_bias")).view(1, M, -1, s.head_dim).transpose(1, 2)
            v = self.linear(x, lw["v"], lw.get("v_bias")).view(1, M, -1, s.head_dim).transpose(1, 2)
            q = (q * cos_u) + (rotate_half(q) * sin_u)
            k = (k * cos_u) + (rotate_half(k) * sin_u)
            if cache[li] is not None:
                k = torch.cat([cache[li][0], k], dim=-2)
                v = torch.cat([cache[li][1], v], dim=-2)
            new_cache.append((k, v))
            t0 = time.perf_counter()
            attn = self._sdpa(q, k, v, attention_mask, scaling)
            self.timer.add("sdpa", t0)
            attn = attn.transpose(1, 2).contiguous().reshape(1, M, -1).contiguous()
            hidden = residual + self.linear(attn, lw["o"])
            residual = hidden
            x = rms_norm(hidden, lw["mlp_norm"], s.rms_eps)
            g = self.linear(x, lw["gate"])
            u = self.linear(x, lw["up"])
            hidden = residual + self.linear(F.silu(g) * u, lw["down"])
            states.append(hidden)
        hidden = rms_norm(hidden, self.w["final_norm"], s.rms_eps)
        states[-1] = hidden
        logits = self.linear(hidden, self.w["lm_head"])
        fused = torch.cat([states[i] for i in self.feature_layers], dim=-1)
        return logits, fused, new_cache

    def _sdpa(self, q, k, v, mask, scaling):
        """HF sdpa_attention_forward's dispatch (integrations/sdpa_attention.py:79-154):
        GQA through enable_gqa only without a mask, repeat_kv otherwise; is_causal
        only for a mask-less multi-token call (HF builds a boolean mask when a
        multi-token call continues a non-empty cache)."""
        groups = self.shape.num_heads // self.shape.num_kv_heads
        M, S = q.shape[2], k.shape[2]
        if mask is None and M > 1 and S != M:
            mask = (torch.arange(M)[:, None] + (S - M) >= torch.arange(S)[None, :]).view(1, 1, M, S)
        kw = {}
        if groups > 1:
            if mask is None:
                kw["enable_gqa"] = True
            else:
                k, v = repeat_kv(k, groups), repeat_kv(v, groups)
        is_causal = M > 1 and mask is None
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=0.0, scale=scaling,
                                              is_causal=is_causal, **kw)


def weights_from_hf(model, dtype: torch.dtype) -> dict:
    """Pull a weights dict out of a transformers Llama/Qwen2 model (tests)."""
    base = model.model
    layers = []
    for lyr in base.layers:
        a = lyr.self_attn
        d = {
            "attn_norm": lyr.input_layernorm.weight.data.to(dtype),
            "mlp_norm": lyr.post_attention_layernorm.weight.data.to(dtype),
            "q": a.q_proj.weight.data.to(dtype), "k": a.k_proj.weight.data.to(dtype),
            "v": a.v_proj.weight.data.to(dtype), "o": a.o_proj.weight.data.to(dtype),
            "gate": lyr.mlp.gate_proj.weight.data.to(dtype), "up": lyr.mlp.up_proj.weight.data.to(dtype),
            "down": lyr.mlp.down_proj.weight.data.to(dtype),
        }
        if a.q_proj.bias is not None:
            d["q_bias"] = a.q_proj.bias.data.to(dtype)
            d["k_bias"] = a.k_proj.bias.data.to(dtype)
            d["v_bias"] = a.v_proj.bias.data.to(dtype)
        layers.append(d)
    return {"embed": base.embed_tokens.weight.data.to(dtype), "final_norm": base.norm.weight.data.to(dtype),
            "lm_head": model.lm_head.weight.data.to(dtype), "layers": layers}
