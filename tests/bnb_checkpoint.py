"""Synthetic bitsandbytes 4-bit checkpoints for the import tests (test helper).

Writes the state-dict entries ``Params4bit`` saves through
``QuantState.as_dict(packed=True)`` (bitsandbytes >= 0.43): the uint8 codes as
``[N*K/2, 1]``, ``.absmax``, ``.quant_map``, the nested entries when the
statistics are double quantised, and the JSON record of the non-tensor fields
as a uint8 tensor under ``.quant_state.bitsandbytes__nf4``. bitsandbytes is not
installed, so no real checkpoint is read: the codes come from the oracle's NF4
quantiser, the fp32 absmax are perturbed away from fp16 values, and the nested
256-entry map is a synthetic sorted table (the importer takes the map from the
checkpoint and does not depend on how it was built).
"""
from __future__ import annotations

import json

import numpy as np
import torch

from oracle import nf4 as onf4

NESTED_BLOCK = 256


def nested_code() -> np.ndarray:
    """A sorted 256-entry signed map in [-1, 1] with 0 and +/-1 (like bitsandbytes'
    dynamic map in shape, not in values)."""
    vals = np.concatenate([-np.geomspace(1e-6, 1.0, 127), [0.0], np.geomspace(1e-6, 1.0, 128)]).astype(np.float32)
    vals = np.unique(vals)
    assert vals.size == 256
    return vals


def fp32_absmax(absmax16: np.ndarray, rng: np.random.Generator) -> np.ndarray:
    """fp32 absmax near the fp16 ones, but with mantissa bits fp16 does not hold."""
    a = np.asarray(absmax16, dtype=np.float32).reshape(-1)
    return (a * (np.float32(1.0) + np.float32(2.0 ** -12) * rng.uniform(1, 2, a.size).astype(np.float32))).astype(
        np.float32)


def double_quantise(absmax32: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray, float]:
    """(q uint8, code, nested_absmax, offset): offset = mean, blocks of 256 scaled by
    their max |absmax - offset|, nearest code (lowest index on ties)."""
    a = np.asarray(absmax32, dtype=np.float32).reshape(-1)
    offset = float(np.float32(a.mean()))
    c = (a - np.float32(offset)).astype(np.float32)
    nblk = -(-c.size // NESTED_BLOCK)
    padded = np.zeros(nblk * NESTED_BLOCK, dtype=np.float32)
    padded[: c.size] = c
    nested = np.abs(padded.reshape(nblk, NESTED_BLOCK)).max(axis=1).astype(np.float32)
    nested[nested == 0] = 1.0
    code = nested_code()
    scaled = c / nested[np.arange(c.size) // NESTED_BLOCK]
    q = np.abs(scaled[:, None] - code[None, :]).argmin(axis=1).astype(np.uint8)
    return q, code, nested, offset


def linear_entries(prefix: str, packed: np.ndarray, absmax32: np.ndarray, nested: bool) -> tuple[dict, np.ndarray]:
    """State-dict entries of one saved Params4bit and the fp32 absmax it decodes to."""
    n, kh = packed.shape
    k = kh * 2
    qs = {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": [n, k]}
    sd = {prefix + "weight": torch.from_numpy(np.ascontiguousarray(packed).reshape(-1, 1).copy()),
          prefix + "weight.quant_map": torch.from_numpy(onf4.NF4_TABLE.astype(np.float32).copy())}
    if nested:
        q, code, nest, offset = double_quantise(absmax32)
        sd[prefix + "weight.absmax"] = torch.from_numpy(q)
        sd[prefix + "weight.nested_absmax"] = torch.from_numpy(nest)
        sd[prefix + "weight.nested_quant_map"] = torch.from_numpy(code)
        qs.update({"nested_blocksize": NESTED_BLOCK, "nested_dtype": "float32", "nested_offset": offset})
        effective = onf4.absmax_from_double_quant(q, code, nest, NESTED_BLOCK, offset)
    else:
        sd[prefix + "weight.absmax"] = torch.from_numpy(np.asarray(absmax32, dtype=np.float32).reshape(-1).copy())
        effective = np.asarray(absmax32, dtype=np.float32).reshape(-1)
    sd[prefix + "weight.quant_state.bitsandbytes__nf4"] = torch.tensor(list(json.dumps(qs).encode("utf-8")),
                                                                      dtype=torch.uint8)
    return sd, effective.reshape(n, k // 64)


_NAMES = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
          "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}


def model_state_dict(shape, host_weights: dict, nested: bool, seed: int) -> dict:
    """An HF-named state dict of a model whose NF4 linears are saved as bitsandbytes
    Params4bit (fp32 absmax from the host weights' fp16 ones), the rest as bf16."""
    rng = np.random.default_rng(seed)
    sd = {"model.embed_tokens.weight": host_weights["embed"].to(torch.bfloat16),
          "model.norm.weight": host_weights["final_norm"].to(torch.bfloat16),
          "lm_head.weight": host_weights["lm_head"].to(torch.bfloat16)}
    for li, lw in enumerate(host_weights["layers"]):
        pre = f"model.layers.{li}."
        for name, path in _NAMES.items():
            _, packed, absmax16 = lw[name]
            entries, _ = linear_entries(pre + path + ".", packed, fp32_absmax(absmax16, rng), nested)
            sd.update(entries)
        sd[pre + "input_layernorm.weight"] = lw["attn_norm"].to(torch.bfloat16)
        sd[pre + "post_attention_layernorm.weight"] = lw["mlp_norm"].to(torch.bfloat16)
        for b in ("q", "k", "v"):
            if b + "_bias" in lw:
                sd[pre + f"self_attn.{b}_proj.bias"] = lw[b + "_bias"].to(torch.bfloat16)
    return sd
