"""NF4 weight format restated in numpy (oracle; test infrastructure only).

The reference loads bitsandbytes NF4 checkpoints (src/pe/target.py:32-38) and
its multi-token Linear4bit path dequantises the whole weight to bf16 before the
GEMM (dequantize as at src/pe/target.py:55-62). bitsandbytes (>=0.43,<1,
pyproject.toml:25) is not installed here; its published behaviour is restated:

- code book: the 16 NF4 values of QLoRA / bitsandbytes (fp32),
- blocks of 64 consecutive elements of the row-major [N][K] weight share one
  absmax (stored fp16 here),
- packing: byte j holds element 2j in the high nibble, 2j+1 in the low nibble,
- dequant: bf16_rne(fp32(NF4[c]) * fp32(absmax)),
- quantise (fixture generation): absmax = max|x| rounded to fp16, code =
  argmin_c |x / absmax - NF4[c]| with the lowest index on ties.

Pinned by: code 7 == 0, codes 0/15 == -/+1 (so dequant gives -/+absmax), the
table's monotonicity and its closed-form reconstruction from normal quantiles
(scipy, agreement to ~1e-7: a sanity check, not the definition), pack/unpack
round trips and quantise-dequantise-quantise idempotence.
"""

from __future__ import annotations

import numpy as np
import torch

NF4_TABLE = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
     -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
     0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
     0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0],
    dtype=np.float32,
)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [N][K] (0..15) -> packed uint8 [N][K/2]."""
    c = np.asarray(codes, dtype=np.uint8)
    return ((c[..., 0::2] << 4) | c[..., 1::2]).astype(np.uint8)


def unpack(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p >> 4
    out[..., 1::2] = p & 15
    return out


def quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp32 W[N][K] -> (packed uint8 [N][K/2], absmax fp16 [N][K/64])."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blocks = w.reshape(n, k // 64, 64)
    amax = np.abs(blocks).max(axis=-1).astype(np.float16)
    sc = amax.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        xn = np.where(sc > 0, blocks / np.where(sc > 0, sc, 1.0).astype(np.float32), np.float32(0.0))
    xn = xn.astype(np.float32)
    d = np.abs(xn[..., None] - NF4_TABLE)  # fp32 differences
    codes = np.argmin(d, axis=-1).astype(np.uint8)  # first minimum on ties
    return pack(codes.reshape(n, k)), amax


def dequantize(packed: np.ndarray, absmax: np.ndarray) -> np.ndarray:
    """-> bf16 bit patterns uint16 [N][K]."""
    codes = unpack(packed)
    n, k = codes.shape
    vals = NF4_TABLE[codes].reshape(n, k // 64, 64) * np.asarray(absmax).astype(np.float32)[..., None]
    return f32_to_bf16_bits(vals.reshape(n, k).astype(np.float32))


_TABLE_T = torch.from_numpy(NF4_TABLE)


def dequantize_torch(packed: np.ndarray, absmax: np.ndarray) -> torch.Tensor:
    """The same dequantisation as ``dequantize`` in torch ops (multi-threaded on the
    host cores) -> bf16 tensor [N][K]. Bit-identical to ``dequantize``: one fp32
    product per element, then one round-to-nearest-even cast."""
    p = torch.from_numpy(np.ascontiguousarray(packed, dtype=np.uint8))
    n, kh = p.shape
    codes = torch.stack([p >> 4, p & 15], dim=-1).reshape(n, kh * 2).long()
    scale = torch.from_numpy(np.ascontiguousarray(absmax)).float().unsqueeze(-1)
    vals = _TABLE_T[codes].view(n, kh * 2 // 64, 64) * scale
    return vals.view(n, kh * 2).to(torch.bfloat16)


def absmax_from_double_quant(q: np.ndarray, code: np.ndarray, nested_absmax: np.ndarray, nested_blocksize: int,
                             offset: float) -> np.ndarray:
    """bitsandbytes' double-quantised absmax back to fp32: dequantize_blockwise
    (out = code[q[i]] * nested_absmax[i // nested_blocksize], one fp32 product)
    followed by ``absmax += offset`` (one fp32 sum), as dequantize_4bit does with
    a nested quant state (bitsandbytes functional.py; the reference reaches it
    through Linear4bit / dequantize_4bit, src/pe/target.py:55-62).

    Pinned in tests/test_bnb_import.py: exact on products and sums that fp32
    represents, within half an ulp of the exact two-step value elsewhere, and
    different from a fused multiply-add on inputs where the two differ."""
    q = np.asarray(q, dtype=np.uint8).reshape(-1)
    idx = np.arange(q.size) // int(nested_blocksize)
    prod = np.asarray(code, dtype=np.float32)[q] * np.asarray(nested_absmax, dtype=np.float32)[idx]
    return (prod.astype(np.float32) + np.float32(offset)).astype(np.float32)
