"""Thin torch-tensor wrappers over the C ABI of libpe_hip.so.

Every function takes device tensors, validates shapes and dtypes on the host,
launches on torch's current HIP stream and raises ``PEError`` on a non-zero
status. They are registered as torch custom ops under the ``pe`` namespace
(``torch.ops.pe.*``) where a functional form exists; in-place cache updates
stay plain functions. There is no CPU implementation behind any of them.
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from ._lib import check

DTYPE_CODE = {torch.float32: _lib.PE_DTYPE_F32, torch.bfloat16: _lib.PE_DTYPE_BF16, torch.float16: _lib.PE_DTYPE_F16}


def lib():
    return _lib.load()


def stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("parallel_eagle_amd kernels take HIP device tensors")
    return t.data_ptr()


def dcode(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError as e:
        raise TypeError(f"unsupported dtype {dtype}") from e


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


# ------------------------------------------------------------------ synthetic / formats
def fill_normal(out: torch.Tensor, seed: int, stream_id: int, std: float) -> torch.Tensor:
    _req(out.is_contiguous(), "out must be contiguous")
    check(lib().pe_fill_normal(ptr(out), out.numel(), dcode(out.dtype), seed, stream_id, std, stream_ptr()),
          "pe_fill_normal")
    return out


def fill_uniform_int(out: torch.Tensor, hi: int, seed: int, stream_id: int) -> torch.Tensor:
    _req(out.dtype == torch.int64 and out.is_contiguous(), "out must be contiguous int64")
    check(lib().pe_fill_uniform_int(ptr(out), out.numel(), hi, seed, stream_id, stream_ptr()), "pe_fill_uniform_int")
    return out


def nf4_quantize(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    _req(w.dtype == torch.float32 and w.dim() == 2 and w.is_contiguous(), "w must be contiguous fp32 [N][K]")
    n, k = w.shape
    _req(k % 64 == 0, "K must be a multiple of 64")
    packed = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    absmax = torch.empty((n, k // 64), dtype=torch.float16, device=w.device)
    check(lib().pe_nf4_quantize(ptr(w), n, k, ptr(packed), ptr(absmax), stream_ptr()), "pe_nf4_quantize")
    return packed, absmax


def nf4_repack(packed: torch.Tensor, absmax: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Logical NF4 (packed uint8 [N][K/2], absmax fp16 or fp32 [N][K/64]) -> tiled;
    the tiled absmax keeps the absmax dtype."""
    n, kh = packed.shape
    k = kh * 2
    _req(packed.dtype == torch.uint8 and packed.is_contiguous(), "packed must be contiguous uint8 [N][K/2]")
    _req(absmax.dtype in (torch.float16, torch.float32) and absmax.shape == (n, k // 64) and absmax.is_contiguous(),
         "absmax must be contiguous fp16 or fp32 [N][K/64]")
    _req(n % 32 == 0 and k % 128 == 0, "N % 32 == 0 and K % 128 == 0 required")
    tiled = torch.empty(n * k // 2, dtype=torch.uint8, device=packed.device)
    tabs = torch.empty(n * k // 64, dtype=absmax.dtype, device=packed.device)
    fn = "pe_nf4_repack_f32abs" if absmax.dtype == torch.float32 else "pe_nf4_repack"
    check(getattr(lib(), fn)(ptr(packed), ptr(absmax), n, k, ptr(tiled), ptr(tabs), stream_ptr()), fn)
    return tiled, tabs


def nf4_dequant(tiled: torch.Tensor, tabs: torch.Tensor, n: int, k: int) -> torch.Tensor:
    _req(tabs.dtype in (torch.float16, torch.float32), "tiled absmax must be fp16 or fp32")
    out = torch.empty((n, k), dtype=torch.bfloat16, device=tiled.device)
    fn = "pe_nf4_dequant_f32abs" if tabs.dtype == torch.float32 else "pe_nf4_dequant"
    check(getattr(lib(), fn)(ptr(tiled), ptr(tabs), n, k, ptr(out), stream_ptr()), fn)
    return out


def nf4_absmax_dequant(q: torch.Tensor, code: torch.Tensor, nested_absmax: torch.Tensor, nested_blocksize: int,
                       offset: float) -> torch.Tensor:
    """bitsandbytes double-quantised absmax -> fp32: code[q[i]] * nested_absmax[i // bs] + offset."""
    _req(q.dtype == torch.uint8 and q.is_contiguous(), "q must be contiguous uint8")
    _req(code.dtype == torch.float32 and code.numel() == 256 and code.is_contiguous(), "code must be 256 fp32")
    n = q.numel()
    _req(nested_absmax.dtype == torch.float32 and nested_absmax.is_contiguous()
         and nested_absmax.numel() * nested_blocksize >= n, "nested_absmax must cover every block")
    out = torch.empty(n, dtype=torch.float32, device=q.device)
    check(lib().pe_nf4_absmax_dequant(ptr(q), n, ptr(code), ptr(nested_absmax), nested_blocksize, float(offset),
                                      ptr(out), stream_ptr()), "pe_nf4_absmax_dequant")
    return out


def dense_repack(w: torch.Tensor) -> torch.Tensor:
    _req(w.dim() == 2 and w.is_contiguous(), "w must be contiguous [N][K]")
    n, k = w.shape
    out = torch.empty(n * k, dtype=w.dtype, device=w.device)
    check(lib().pe_dense_repack(ptr(w), n, k, dcode(w.dtype), ptr(out), stream_ptr()), "pe_dense_repack")
    return out


# ------------------------------------------------------------------ GEMMs
def gemm_workspace_bytes(m: int, n: int, k: int, nf4: bool, dtype: torch.dtype, epilogue: int) -> int:
    return int(lib().pe_gemm_workspace_bytes(m, n, k, _lib.PE_WFMT_NF4 if nf4 else _lib.PE_WFMT_DENSE,
                                             dcode(dtype), epilogue))


def _workspace(nbytes: int, device) -> torch.Tensor:
    return torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)


def linear(x: torch.Tensor, n: int, *, nf4: tuple | None = None, dense: torch.Tensor | None = None,
           epilogue: int = _lib.PE_EPI_STORE, bias: torch.Tensor | None = None, resid: torch.Tensor | None = None,
           out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Y = X . W^T with W given as nf4=(tiled, tabs) or dense (tiled/row-major)."""
    _req(x.dim() == 2 and x.stride(1) == 1, "x must be [M][K] with unit column stride")
    m, k = x.shape
    n_out = n // 2 if epilogue == _lib.PE_EPI_SWIGLU else n
    if out is None:
        out = torch.empty((m, n_out), dtype=x.dtype, device=x.device)
    _req(out.shape == (m, n_out) and out.stride(1) == 1 and out.dtype == x.dtype, "bad out")
    if resid is not None:
        _req(resid.shape == (m, n_out) and resid.dtype == x.dtype, "bad resid")
    if workspace is None:
        workspace = _workspace(gemm_workspace_bytes(m, n, k, nf4 is not None, x.dtype, epilogue), x.device)
    L = lib()
    if nf4 is not None:
        _req(x.dtype == torch.bfloat16, "NF4 linears compute in bf16")
        fn = L.pe_nf4_gemm_f32abs if nf4[1].dtype == torch.float32 else L.pe_nf4_gemm
        rc = fn(ptr(x), x.stride(0), m, k, ptr(nf4[0]), ptr(nf4[1]), n, epilogue, ptr(bias), ptr(resid),
                resid.stride(0) if resid is not None else 0, ptr(out), out.stride(0), ptr(workspace),
                workspace.numel(), stream_ptr())
    else:
        rc = L.pe_dense_gemm(ptr(x), x.stride(0), m, k, ptr(dense), dcode(x.dtype), n, epilogue, ptr(bias),
                             ptr(resid), resid.stride(0) if resid is not None else 0, ptr(out), out.stride(0),
                             ptr(workspace), workspace.numel(), stream_ptr())
    check(rc, "linear")
    return out


def xtile_index(m: int, k: int, device=None) -> torch.Tensor:
    """[m][k] -> flat position of each element in the A-tiled activation layout
    (the order the NF4 GEMM reads X as its MFMA A operand; k % 128 == 0)."""
    _req(k % 128 == 0, "A-tiled activations need K % 128 == 0")
    row = torch.arange(m, device=device).view(m, 1)
    col = torch.arange(k, device=device).view(1, k)
    units = k // 128
    mt, ln = row // 32, row % 32
    p, c = col // 128, col % 128
    return ((((mt * units + p) * 8 + (c % 64) // 8) * 64 + ln + 32 * (c // 64)) * 8 + c % 8)


def to_xtile(x: torch.Tensor) -> torch.Tensor:
    """Row-major [M][K] -> A-tiled flat buffer (rows past M of the last 32-row
    tile are zero)."""
    m, k = x.shape
    out = torch.zeros(((m + 31) // 32) * 32 * k, dtype=x.dtype, device=x.device)
    out[xtile_index(m, k, x.device).flatten()] = x.flatten()
    return out


def from_xtile(t: torch.Tensor, m: int, k: int) -> torch.Tensor:
    return t[xtile_index(m, k, t.device).flatten()].view(m, k)


def linear_tiled(xt: torch.Tensor, m: int, k: int, n: int, nf4: tuple, *, epilogue: int = _lib.PE_EPI_STORE,
                 resid: torch.Tensor | None = None, out: torch.Tensor | None = None, out_tiled: bool = False,
                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """pe_nf4_gemm_tiled: X given A-tiled (to_xtile); the output row-major, or
    A-tiled when out_tiled."""
    n_out = n // 2 if epilogue == _lib.PE_EPI_SWIGLU else n
    if out is None:
        out = (torch.zeros(((m + 31) // 32) * 32 * n_out, dtype=xt.dtype, device=xt.device) if out_tiled
               else torch.empty((m, n_out), dtype=xt.dtype, device=xt.device))
    if workspace is None:
        workspace = _workspace(gemm_workspace_bytes(m, n, k, True, xt.dtype, epilogue), xt.device)
    _req(nf4[1].dtype == torch.float16, "the A-tiled and split-partial NF4 entry points take fp16 absmax")
    check(lib().pe_nf4_gemm_tiled(ptr(xt), m, k, ptr(nf4[0]), ptr(nf4[1]), n, epilogue, None, ptr(resid),
                                  resid.stride(0) if resid is not None else 0, ptr(out),
                                  0 if out_tiled else out.stride(0), n_out // 128 if out_tiled else 0,
                                  ptr(workspace), workspace.numel(), stream_ptr()), "linear_tiled")
    return out


# ------------------------------------------------------------------ elementwise
def nf4_linear_partials(x: torch.Tensor, m: int, k: int, n: int, nf4: tuple, *, x_tiled: bool = False,
                        partials: torch.Tensor | None = None) -> tuple[torch.Tensor, int]:
    """pe_nf4_gemm_partials: fp32 split partials [S][m][n] of X . deq(W)^T (X
    row-major [m][k] or A-tiled); returns (partials, S)."""
    nbytes = int(lib().pe_nf4_gemm_partials_bytes(m, n, k))
    _req(nbytes > 0, "unsupported shape for split partials")
    if partials is None:
        partials = torch.empty(nbytes // 4, dtype=torch.float32, device=x.device)
    s = C.c_int(0)
    _req(nf4[1].dtype == torch.float16, "the A-tiled and split-partial NF4 entry points take fp16 absmax")
    check(lib().pe_nf4_gemm_partials(ptr(x), k if x_tiled else x.stride(0), int(x_tiled), m, k, ptr(nf4[0]),
                                     ptr(nf4[1]), n, ptr(partials), partials.numel() * 4, C.byref(s), stream_ptr()),
          "nf4_linear_partials")
    return partials[: s.value * m * n].view(s.value, m, n), s.value


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, mode: int = _lib.PE_NORM_HF) -> torch.Tensor:
    """RMSNorm of the rows of x [M][H]; ``mode`` PE_NORM_HF (HF LlamaRMSNorm) or
    PE_NORM_FP32_WEIGHT (the drafter's RMSNorm, one rounding)."""
    _req(x.dim() == 2 and x.stride(1) == 1 and w.dtype == x.dtype, "bad rmsnorm args")
    out = torch.empty_like(x)
    check(lib().pe_rmsnorm_ex(ptr(x), x.stride(0), x.shape[0], x.shape[1], ptr(w), eps, dcode(x.dtype), int(mode),
                              ptr(out), out.stride(0), stream_ptr()), "pe_rmsnorm_ex")
    return out


def embed(ids: torch.Tensor, table: torch.Tensor, status: torch.Tensor) -> torch.Tensor:
    m = ids.numel()
    v, h = table.shape
    out = torch.empty((m, h), dtype=table.dtype, device=table.device)
    check(lib().pe_embed(ptr(ids), m, ptr(table), v, h, dcode(table.dtype), ptr(out), h, ptr(status),
                         stream_ptr()), "pe_embed")
    return out


def rope_qkv(qkv, nh, nkv, hd, positions, cos_sin, k_cache, v_cache, row0, status):
    m = qkv.shape[0]
    q = torch.empty((m, nh, hd), dtype=qkv.dtype, device=qkv.device)
    check(lib().pe_rope_qkv(ptr(qkv), qkv.stride(0), m, nh, nkv, hd, ptr(positions), ptr(cos_sin),
                            cos_sin.shape[1], dcode(qkv.dtype), ptr(q), ptr(k_cache), ptr(v_cache), k_cache.shape[1],
                            row0, ptr(status), stream_ptr()), "pe_rope_qkv")
    return q


# ------------------------------------------------------------------ masks
def tree_masks(parents: torch.Tensor, prefix_len: int, words: int, status: torch.Tensor):
    """parents int32 device [T] -> (bits u64 [T][words] as int64, positions int64 [T], depths int32 [T])."""
    t = parents.numel()
    bits = torch.empty((t, words), dtype=torch.int64, device=parents.device)
    pos = torch.empty(t, dtype=torch.int64, device=parents.device)
    dep = torch.empty(t, dtype=torch.int32, device=parents.device)
    check(lib().pe_tree_masks(ptr(parents), t, prefix_len, ptr(bits), words, ptr(pos), ptr(dep), ptr(status),
                              stream_ptr()), "pe_tree_masks")
    return bits, pos, dep


def tree_allow_dense(bits: torch.Tensor, prefix_len: int) -> torch.Tensor:
    t, words = bits.shape
    n = prefix_len + t
    allow = torch.empty((n, n), dtype=torch.bool, device=bits.device)
    check(lib().pe_tree_allow_dense(ptr(bits), t, words, prefix_len, ptr(allow), stream_ptr()), "pe_tree_allow_dense")
    return allow


def bias_to_bits(bias: torch.Tensor, prefix_len: int, words: int, status: torch.Tensor) -> torch.Tensor:
    _req(bias.dim() == 2 and bias.stride(1) == 1, "bias must be [T][P+T] with unit column stride")
    t = bias.shape[0]
    bits = torch.empty((t, words), dtype=torch.int64, device=bias.device)
    check(lib().pe_bias_to_bits(ptr(bias), bias.stride(0), dcode(bias.dtype), t, prefix_len, ptr(bits), words,
                                ptr(status), stream_ptr()), "pe_bias_to_bits")
    return bits


# ------------------------------------------------------------------ attention
def tree_attention(q, k_cache, v_cache, prefix_len, mask_mode, bits, scale, workspace=None):
    """q [T][nh][hd]; caches [nkv][cap][hd] (one layer)."""
    t, nh, hd = q.shape
    nkv, cap, _ = k_cache.shape
    words = bits.shape[1] if bits is not None else 0
    need = int(lib().pe_attention_workspace_bytes(t, nh, nkv, hd, prefix_len + t, dcode(q.dtype)))
    if workspace is None:
        workspace = _workspace(need, q.device)
    out = torch.empty((t, nh * hd), dtype=q.dtype, device=q.device)
    check(lib().pe_tree_attention(ptr(q), ptr(k_cache), ptr(v_cache), cap, nh, nkv, hd, t, prefix_len, mask_mode,
                                  ptr(bits), words, scale, dcode(q.dtype), ptr(out), out.stride(0), ptr(workspace),
                                  workspace.numel(), stream_ptr()), "pe_tree_attention")
    return out


def tree_attention_batch(q, k_cache, v_cache, seq_row0, seq_prefix, bits, scale, max_rows, max_prefix,
                         workspace=None):
    """q [M][nh][128]; caches [B][nkv][cap][128] (one layer per sequence);
    seq_row0 int32 [B + 1], seq_prefix int64 [B] and bits int64 [M][words] on
    the device."""
    m, nh, hd = q.shape
    b, nkv, cap, _ = k_cache.shape
    _req(hd == 128 and q.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous(),
         "q and the caches must be contiguous with 128-dim heads")
    need = int(lib().pe_attention_batch_workspace_bytes(max_rows, nh, nkv, max_prefix + max_rows, b))
    if workspace is None:
        workspace = torch.zeros(need, dtype=torch.uint8, device=q.device)
    out = torch.empty((m, nh * hd), dtype=q.dtype, device=q.device)
    check(lib().pe_tree_attention_batch(ptr(q), ptr(k_cache), ptr(v_cache), cap, nkv * cap * hd, nh, nkv, max_rows,
                                        max_prefix, b, ptr(seq_row0), ptr(seq_prefix), ptr(bits), bits.shape[1],
                                        scale, dcode(q.dtype), ptr(out), out.stride(0), ptr(workspace),
                                        workspace.numel(), stream_ptr()), "pe_tree_attention_batch")
    return out


# ------------------------------------------------------------------ acceptance / cache
def argmax_rows(x: torch.Tensor) -> torch.Tensor:
    _req(x.dim() == 2 and x.stride(1) == 1, "x must be [rows][V]")
    out = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
    check(lib().pe_argmax_rows(ptr(x), x.stride(0), x.shape[0], x.shape[1], dcode(x.dtype), ptr(out), stream_ptr()),
          "pe_argmax_rows")
    return out


def accept_tree(root_logit: torch.Tensor, node_logits: torch.Tensor, node_tokens: torch.Tensor,
                parents: torch.Tensor, out: torch.Tensor | None = None, scratch: torch.Tensor | None = None):
    """Device result int32 [2 + T]: (|path|, bonus, path...)."""
    t = node_tokens.numel()
    v = root_logit.shape[-1]
    _req(root_logit.stride(-1) == 1 and (t == 0 or node_logits.stride(1) == 1), "logit rows must be contiguous")
    if out is None:
        out = torch.empty(2 + max(t, 1), dtype=torch.int32, device=root_logit.device)
    if scratch is None:
        scratch = torch.zeros(t + 2, dtype=torch.int32, device=root_logit.device)
    _req(scratch.dtype == torch.int32 and scratch.numel() >= t + 2, "scratch must hold T + 2 int32")
    ld = node_logits.stride(0) if t > 0 else v
    check(lib().pe_accept_tree(ptr(root_logit), ptr(node_logits) if t > 0 else None, ld, t, v,
                               dcode(root_logit.dtype), ptr(node_tokens) if t > 0 else None,
                               ptr(parents) if t > 0 else None, ptr(out), ptr(scratch), stream_ptr()), "pe_accept_tree")
    return out


def propose_tree(logits: torch.Tensor, widths, top_k: int, status: torch.Tensor | None = None,
                 scratch: torch.Tensor | None = None):
    """Beam tree proposal over k draft-logit rows [k][V] on the device.

    Returns (node_tokens int64 [n], parents int32 [n], status int32 [1]) as device
    tensors; n is known on the host, so nothing here waits for the GPU.
    PE_ERR_VALUE in ``status`` marks a row with a NaN or no finite value.
    ``scratch`` (k * PE_PROPOSE_SCRATCH_PER_DEPTH bytes) receives, per depth, 64
    fp32 log-probabilities and then (after all k of those) 64 int32 tokens."""
    _req(logits.dim() == 2 and logits.stride(1) == 1, "logits must be [k][V] with contiguous rows")
    k, v = logits.shape
    widths = [int(w) for w in widths]
    _req(len(widths) == k, "one width per depth row")
    dev = logits.device
    cap = k * _lib.PE_PROPOSE_MAX_WIDTH
    tokens = torch.empty(cap, dtype=torch.int64, device=dev)
    parents = torch.empty(cap, dtype=torch.int32, device=dev)
    if scratch is None:
        scratch = torch.empty(k * _lib.PE_PROPOSE_SCRATCH_PER_DEPTH, dtype=torch.uint8, device=dev)
    _req(scratch.numel() * scratch.element_size() >= k * _lib.PE_PROPOSE_SCRATCH_PER_DEPTH and scratch.is_contiguous(),
         "scratch must hold k * PE_PROPOSE_SCRATCH_PER_DEPTH bytes")
    if status is None:
        status = torch.zeros(1, dtype=torch.int32, device=dev)
    w = (C.c_int32 * k)(*widths)
    n = C.c_int32(0)
    check(lib().pe_propose_tree(ptr(logits), logits.stride(0), k, v, dcode(logits.dtype), w, int(top_k), ptr(tokens),
                                ptr(parents), C.byref(n), ptr(scratch), ptr(status), stream_ptr()), "pe_propose_tree")
    return tokens[: n.value], parents[: n.value], status


def kv_compact(k_cache, v_cache, prefix_len: int, accept_out: torch.Tensor) -> None:
    """Caches [L][nkv][cap][hd]."""
    L, nkv, cap, hd = k_cache.shape
    check(lib().pe_kv_compact(ptr(k_cache), ptr(v_cache), L, nkv, cap, hd, dcode(k_cache.dtype), prefix_len,
                              ptr(accept_out), stream_ptr()), "pe_kv_compact")


def kv_gather(k_cache, v_cache, keep: torch.Tensor, status4: torch.Tensor) -> None:
    L, nkv, cap, hd = k_cache.shape
    _req(keep.dtype == torch.int64 and keep.is_contiguous(), "keep must be contiguous int64")
    _req(status4.dtype == torch.int32 and status4.numel() >= 4, "status must be int32[4]")
    check(lib().pe_kv_gather(ptr(k_cache), ptr(v_cache), L, nkv, cap, hd, dcode(k_cache.dtype), ptr(keep),
                             keep.numel(), ptr(status4), stream_ptr()), "pe_kv_gather")


def read_status(status: torch.Tensor, where: str) -> None:
    s = int(status[0].item())
    if s:
        status.zero_()
        raise _lib.PEError(s, where)


# ------------------------------------------------------------------ torch custom ops
# A target registered here is named by an integer handle in torch.ops.pe.verify_pass
# (a torch op takes tensors and scalars only; the pass reads the model's weights
# through its pe_model_desc).
_MODELS: dict[int, object] = {}


def register_model(target) -> int:
    """Handle of ``target`` (a TargetModel) for ``torch.ops.pe.verify_pass``; the same
    target gets the same handle."""
    for h, t in _MODELS.items():
        if t is target:
            return h
    h = len(_MODELS) + 1
    _MODELS[h] = target
    return h


def _model(handle: int):
    try:
        return _MODELS[handle]
    except KeyError as e:
        raise ValueError(f"no target registered under handle {handle} (ops.register_model)") from e


def verify_pass(target, input_ids: torch.Tensor, positions: torch.Tensor, tree_bits: torch.Tensor,
                k_cache: torch.Tensor, v_cache: torch.Tensor, prefix_len: int, workspace: torch.Tensor,
                status: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """TargetModel.forward_cached (src/pe/target.py:203-224) as one pe_forward over
    preallocated caches [L][nkv][cap][hd]: rows input_ids at positions, their K/V
    appended at [prefix_len, prefix_len + M), attention over the prefix plus the
    tree rows of tree_bits [M][words] (empty: a causal continuation). Returns
    (logits [M][V], fused [M][F]) in the model dtype; device errors go to status."""
    s = target.shape
    m = input_ids.numel()
    _req(positions.numel() == m and input_ids.dtype == torch.int64 and positions.dtype == torch.int64,
         "input_ids and positions: int64, one position per id")
    _req(k_cache.shape == v_cache.shape and k_cache.dim() == 4 and k_cache.dtype == target.dtype
         and k_cache.is_contiguous() and v_cache.is_contiguous(), "caches [L][nkv][cap][hd] in the model dtype")
    _req(status.dtype == torch.int32 and workspace.dtype == torch.uint8, "status int32, workspace uint8")
    tree = tree_bits.numel() > 0
    logits = torch.empty((m, s.vocab), dtype=target.dtype, device=input_ids.device)
    fused = torch.empty((m, target.feature_dim), dtype=target.dtype, device=input_ids.device)
    a = _lib.PassArgs()
    a.input_ids, a.positions, a.M, a.prefix_len = ptr(input_ids), ptr(positions), m, prefix_len
    a.mask_mode = _lib.PE_MASK_TREE if tree else _lib.PE_MASK_CAUSAL
    a.tree_bits, a.bits_words = (ptr(tree_bits), tree_bits.shape[1]) if tree else (None, 0)
    fl = target.feature_layers
    a.num_features = len(fl)
    for i, f in enumerate(fl[:4]):
        a.feature_layers[i] = f
    a.k_cache, a.v_cache, a.cache_capacity = ptr(k_cache), ptr(v_cache), k_cache.shape[2]
    a.logits, a.fused = ptr(logits), ptr(fused)
    a.workspace, a.workspace_bytes = ptr(workspace), workspace.numel()
    a.status = ptr(status)
    check(lib().pe_forward(C.byref(target.model.desc()), C.byref(a), stream_ptr()), "pe_forward")
    return logits, fused


_REGISTERED = False


def register_torch_ops() -> None:
    """Register the pass and its steps as torch custom ops (``torch.ops.pe.*``),
    each with a fake (meta) implementation for tracing and the cache / scratch /
    status mutations declared in its schema:

    - ``verify_pass(model, input_ids, positions, tree_bits, k_cache!, v_cache!,
      prefix_len, workspace!, status!) -> (logits, fused)``: the masked
      verification forward (src/pe/target.py:203-224), ``model`` from
      ``register_model``;
    - ``tree_masks(parents, prefix_len, words, status!) -> (bits, positions,
      depths)``: src/pe/masks.py:118-156;
    - ``accept_tree(root, node_logits, node_tokens, parents, scratch!) -> out``:
      src/pe/decode/verify.py:104-125, out = [|path|, bonus, path...];
    - ``kv_compact(k_cache!, v_cache!, prefix_len, accept_out)`` and
      ``kv_gather(k_cache!, v_cache!, keep, status!)``: gather_cache
      (src/pe/target.py:194-201);
    - ``rmsnorm``, ``argmax_rows``, ``nf4_linear``, ``dense_linear``: the pass's
      building blocks.
    """
    global _REGISTERED
    if _REGISTERED:
        return
    lib_def = torch.library.custom_op

    def op(name, schema, mutates=()):
        return lambda fn: lib_def(f"pe::{name}", fn, mutates_args=mutates, schema=schema)

    @op("verify_pass", "(int model, Tensor input_ids, Tensor positions, Tensor tree_bits, Tensor(a!) k_cache, "
        "Tensor(b!) v_cache, int prefix_len, Tensor(c!) workspace, Tensor(d!) status) -> (Tensor, Tensor)",
        ("k_cache", "v_cache", "workspace", "status"))
    def _verify_pass(model, input_ids, positions, tree_bits, k_cache, v_cache, prefix_len, workspace, status):
        return verify_pass(_model(model), input_ids, positions, tree_bits, k_cache, v_cache, prefix_len, workspace,
                           status)

    @_verify_pass.register_fake
    def _(model, input_ids, positions, tree_bits, k_cache, v_cache, prefix_len, workspace, status):
        t = _model(model)
        m = input_ids.numel()
        return (input_ids.new_empty((m, t.shape.vocab), dtype=t.dtype),
                input_ids.new_empty((m, t.feature_dim), dtype=t.dtype))

    @op("tree_masks", "(Tensor parents, int prefix_len, int words, Tensor(a!) status) -> (Tensor, Tensor, Tensor)",
        ("status",))
    def _tree_masks(parents, prefix_len, words, status):
        return tree_masks(parents, prefix_len, words, status)

    @_tree_masks.register_fake
    def _(parents, prefix_len, words, status):
        t = parents.numel()
        return (parents.new_empty((t, words), dtype=torch.int64), parents.new_empty(t, dtype=torch.int64),
                parents.new_empty(t, dtype=torch.int32))

    @op("accept_tree", "(Tensor root, Tensor node_logits, Tensor node_tokens, Tensor parents, Tensor(a!) scratch) "
        "-> Tensor", ("scratch",))
    def _accept(root, node_logits, node_tokens, parents, scratch):
        return accept_tree(root, node_logits, node_tokens, parents, scratch=scratch)

    @_accept.register_fake
    def _(root, node_logits, node_tokens, parents, scratch):
        return root.new_empty(2 + max(node_tokens.numel(), 1), dtype=torch.int32)

    @op("kv_compact", "(Tensor(a!) k_cache, Tensor(b!) v_cache, int prefix_len, Tensor accept_out) -> ()",
        ("k_cache", "v_cache"))
    def _kv_compact(k_cache, v_cache, prefix_len, accept_out):
        kv_compact(k_cache, v_cache, prefix_len, accept_out)

    @_kv_compact.register_fake
    def _(k_cache, v_cache, prefix_len, accept_out):
        return None

    @op("kv_gather", "(Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor keep, Tensor(c!) status) -> ()",
        ("k_cache", "v_cache", "status"))
    def _kv_gather(k_cache, v_cache, keep, status):
        kv_gather(k_cache, v_cache, keep, status)

    @_kv_gather.register_fake
    def _(k_cache, v_cache, keep, status):
        return None

    @op("rmsnorm", "(Tensor x, Tensor w, float eps) -> Tensor")
    def _rmsnorm(x, w, eps):
        return rmsnorm(x, w, eps)

    @_rmsnorm.register_fake
    def _(x, w, eps):
        return torch.empty_like(x)

    @op("argmax_rows", "(Tensor x) -> Tensor")
    def _argmax(x):
        return argmax_rows(x)

    @_argmax.register_fake
    def _(x):
        return x.new_empty(x.shape[0], dtype=torch.int32)

    @op("nf4_linear", "(Tensor x, Tensor tiled, Tensor tabs, int n) -> Tensor")
    def _nf4_linear(x, tiled, tabs, n):
        return linear(x, n, nf4=(tiled, tabs))

    @_nf4_linear.register_fake
    def _(x, tiled, tabs, n):
        return x.new_empty((x.shape[0], n))

    @op("dense_linear", "(Tensor x, Tensor w, int n) -> Tensor")
    def _dense_linear(x, w, n):
        return linear(x, n, dense=w)

    @_dense_linear.register_fake
    def _(x, w, n):
        return x.new_empty((x.shape[0], n))

    _REGISTERED = True
