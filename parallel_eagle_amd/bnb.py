"""Import of bitsandbytes 4-bit (NF4) checkpoints into the repacked kernel layout.

The reference loads pre-quantized checkpoints through transformers with a
bitsandbytes config (src/pe/target.py:32-38) and dequantises each linear as
``dequantize_4bit(weight, quant_state)`` (src/pe/target.py:55-62). A saved
``Params4bit`` weight is a set of state-dict entries under ``<linear>.weight``:

- ``weight``: uint8 ``[N*K/2, 1]``, two codes per byte (element 2j in the high
  nibble), row-major over ``W[N][K]``;
- ``weight.absmax``: fp32 ``[N*K/blocksize]``, or uint8 when the statistics are
  double quantised;
- ``weight.quant_map``: the 16 fp32 NF4 values;
- with double quantisation, ``weight.nested_absmax`` (fp32, one per
  ``nested_blocksize`` absmax) and ``weight.nested_quant_map`` (256 fp32);
- ``weight.quant_state.bitsandbytes__nf4``: uint8 bytes of a JSON object with
  ``quant_type``, ``blocksize``, ``dtype``, ``shape`` and, when nested,
  ``nested_blocksize``, ``nested_dtype`` and ``nested_offset``.

This is the layout bitsandbytes' ``QuantState.as_dict(packed=True)`` writes
(bitsandbytes >= 0.43, the reference's pin in pyproject.toml:25; the library
itself is not installed here). The fp32 absmax of block i is
``nested_quant_map[absmax[i]] * nested_absmax[i // nested_blocksize] +
nested_offset`` (``pe_nf4_absmax_dequant``), and the weight is
``bf16(NF4[c] * absmax)`` as for the quantiser's fp16 absmax, so a model built
from these tensors runs the fp32-absmax kernels (``PE_WFMT_NF4_F32ABS``).
"""
from __future__ import annotations

import json
from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from .config import ModelShape

# The published NF4 code book (QLoRA appendix; bitsandbytes' quant_map), fp32.
NF4_CODE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)

QUANT_STATE_KEY = "quant_state.bitsandbytes__nf4"


class CheckpointError(ValueError):
    """The state dict is not an NF4 bitsandbytes checkpoint this build can run."""


@dataclass
class Linear4bit:
    """One serialized ``Params4bit`` (host tensors, not yet on the device)."""
    n: int
    k: int
    packed: torch.Tensor            # uint8 [N][K/2]
    absmax: torch.Tensor            # fp32 [N*K/64], or uint8 when nested
    nested_absmax: torch.Tensor | None = None
    nested_code: torch.Tensor | None = None
    nested_blocksize: int = 0
    nested_offset: float = 0.0

    @property
    def nested(self) -> bool:
        return self.nested_absmax is not None


def _tensor(sd: dict, key: str) -> torch.Tensor:
    if key not in sd:
        raise CheckpointError(f"missing {key}")
    v = sd[key]
    return v if isinstance(v, torch.Tensor) else torch.as_tensor(np.asarray(v))


def decode_quant_state(t: torch.Tensor) -> dict:
    """The JSON record bitsandbytes packs into a uint8 tensor."""
    if t.dtype != torch.uint8:
        raise CheckpointError("the packed quant state must be a uint8 tensor")
    try:
        return json.loads(bytes(t.reshape(-1).cpu().tolist()).decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise CheckpointError(f"unreadable packed quant state: {e}") from None


def read_linear4bit(sd: dict, prefix: str) -> Linear4bit:
    """Parse the entries of one ``Params4bit`` saved as ``<prefix>weight*``."""
    w = _tensor(sd, prefix + "weight")
    qs = decode_quant_state(_tensor(sd, prefix + "weight." + QUANT_STATE_KEY))
    if qs.get("quant_type") != "nf4":
        raise CheckpointError(f"{prefix}weight: quant_type {qs.get('quant_type')!r}, only 'nf4' is supported")
    if int(qs.get("blocksize", -1)) != 64:
        raise CheckpointError(f"{prefix}weight: blocksize {qs.get('blocksize')}, the kernels take 64")
    # the compute dtype the checkpoint was quantised for (QuantState.dtype): the
    # NF4 kernels compute in bfloat16, and an fp16 model run in bf16 would give
    # other logits than the reference (target.py:89 takes the dtype from the model)
    cdt = str(qs.get("dtype", "")).replace("torch.", "")
    if cdt != "bfloat16":
        raise CheckpointError(f"{prefix}weight: compute dtype {qs.get('dtype')!r}; the NF4 kernels compute in bfloat16")
    shape = qs.get("shape")
    if not isinstance(shape, (list, tuple)) or len(shape) != 2:
        raise CheckpointError(f"{prefix}weight: shape {shape!r} is not 2-D")
    n, k = int(shape[0]), int(shape[1])
    if k % 64:
        raise CheckpointError(f"{prefix}weight: K = {k} is not a multiple of 64")
    if w.dtype != torch.uint8 or w.numel() * 2 != n * k:
        raise CheckpointError(f"{prefix}weight: expected {n * k // 2} uint8 codes, got {w.numel()} {w.dtype}")
    code = _tensor(sd, prefix + "weight.quant_map").to(torch.float32).reshape(-1).cpu().numpy()
    if code.shape != (16,) or not np.array_equal(code.view(np.uint32), NF4_CODE.view(np.uint32)):
        raise CheckpointError(f"{prefix}weight: quant_map is not the NF4 code book")
    absmax = _tensor(sd, prefix + "weight.absmax").reshape(-1)
    if absmax.numel() != n * k // 64:
        raise CheckpointError(f"{prefix}weight: {absmax.numel()} absmax for {n * k // 64} blocks")
    lin = Linear4bit(n, k, w.reshape(n, k // 2).contiguous(), absmax.contiguous())
    if "nested_blocksize" in qs:
        if absmax.dtype != torch.uint8:
            raise CheckpointError(f"{prefix}weight: double-quantised absmax must be uint8")
        nb = int(qs["nested_blocksize"])
        nested = _tensor(sd, prefix + "weight.nested_absmax").to(torch.float32).reshape(-1).contiguous()
        ncode = _tensor(sd, prefix + "weight.nested_quant_map").to(torch.float32).reshape(-1).contiguous()
        if nb <= 0 or nested.numel() * nb < absmax.numel() or ncode.numel() != 256:
            raise CheckpointError(f"{prefix}weight: inconsistent nested quant state")
        lin.nested_absmax, lin.nested_code, lin.nested_blocksize = nested, ncode, nb
        lin.nested_offset = float(qs.get("nested_offset", 0.0))
    elif absmax.dtype != torch.float32:
        raise CheckpointError(f"{prefix}weight: absmax must be fp32 (or uint8 with a nested state)")
    return lin


def to_device(lin: Linear4bit, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(packed uint8 [N][K/2], absmax fp32 [N][K/64]) on the device."""
    packed = lin.packed.to(device).contiguous()
    if lin.nested:
        absmax = ops.nf4_absmax_dequant(lin.absmax.to(device).contiguous(), lin.nested_code.to(device),
                                        lin.nested_absmax.to(device), lin.nested_blocksize, lin.nested_offset)
    else:
        absmax = lin.absmax.to(device=device, dtype=torch.float32).contiguous()
    return packed, absmax.reshape(lin.n, lin.k // 64)


# HF Llama / Qwen2 parameter names (modeling_llama.py) -> the oracle's layer keys
_LINEARS = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
            "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}


def weights_from_state_dict(shape: ModelShape, sd: dict, device="cuda") -> dict:
    """The weights dict of ``DeviceModel.from_weights`` from an HF state dict whose
    linears are bitsandbytes NF4 (embed, norms and lm_head in the compute dtype)."""
    if shape.weight_format != "nf4":
        raise CheckpointError("the model shape must name NF4 linears")

    def dense(key, rows, cols=None):
        t = _tensor(sd, key)
        want = (rows,) if cols is None else (rows, cols)
        if tuple(t.shape) != want:
            raise CheckpointError(f"{key}: shape {tuple(t.shape)}, expected {want}")
        if t.dtype not in (torch.bfloat16, torch.float32):
            # an fp16 embedding / norm / lm_head means an fp16 model (the reference
            # runs it in the embedding's dtype, target.py:89); bf16 here would not
            # reproduce its logits
            raise CheckpointError(f"{key}: {t.dtype}; the NF4 model computes in bfloat16")
        return t.to(device=device, dtype=torch.bfloat16).contiguous()

    s = shape
    lm_key = "lm_head.weight" if "lm_head.weight" in sd else "model.embed_tokens.weight"  # tied embeddings
    out = {"embed": dense("model.embed_tokens.weight", s.vocab, s.hidden),
           "final_norm": dense("model.norm.weight", s.hidden),
           "lm_head": dense(lm_key, s.vocab, s.hidden), "layers": []}
    for li in range(s.num_layers):
        pre = f"model.layers.{li}."
        lw = {}
        for name, n, k in s.linear_shapes():
            lin = read_linear4bit(sd, pre + _LINEARS[name] + ".")
            if (lin.n, lin.k) != (n, k):
                raise CheckpointError(f"{pre}{_LINEARS[name]}: shape {(lin.n, lin.k)}, expected {(n, k)}")
            lw[name] = ("nf4",) + to_device(lin, device)
        lw["attn_norm"] = dense(pre + "input_layernorm.weight", s.hidden)
        lw["mlp_norm"] = dense(pre + "post_attention_layernorm.weight", s.hidden)
        if s.qkv_bias:
            lw["q_bias"] = dense(pre + "self_attn.q_proj.bias", s.q_dim)
            lw["k_bias"] = dense(pre + "self_attn.k_proj.bias", s.kv_dim)
            lw["v_bias"] = dense(pre + "self_attn.v_proj.bias", s.kv_dim)
        out["layers"].append(lw)
    return out
