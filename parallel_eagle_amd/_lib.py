"""ctypes binding of libpe_hip.so (declarations in include/pe_hip.h).

torch is imported first so its HIP runtime is the one the library resolves
against: there must be exactly one libamdhip64 in the process. The loader fails
loudly when the library has not been built; nothing here has a CPU fallback.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "libpe_hip.so"

PE_OK = 0
PE_ERR_ARG = 1
PE_ERR_LAUNCH = 2
PE_ERR_TREE = 4
PE_ERR_CAPACITY = 8
PE_ERR_MASK = 16
PE_ERR_TOKEN = 32
PE_ERR_INDEX = 64
PE_ERR_WORKSPACE = 128
PE_ERR_VALUE = 256

PE_DTYPE_F32, PE_DTYPE_BF16, PE_DTYPE_F16 = 0, 1, 2
PE_WFMT_DENSE, PE_WFMT_NF4, PE_WFMT_NF4_F32ABS = 0, 1, 2
PE_EPI_STORE, PE_EPI_RESIDUAL, PE_EPI_SWIGLU = 0, 1, 2
PE_MASK_TREE, PE_MASK_CAUSAL = 0, 1
PE_QKV_PLAIN, PE_QKV_ROPE_PAIRED = 0, 1
PE_NORM_HF, PE_NORM_FP32_WEIGHT = 0, 1
PE_ATTN_SDPA, PE_ATTN_EAGER = 0, 1
PE_TREE_MAX_WORDS = 4
PE_PROPOSE_MAX_DEPTH, PE_PROPOSE_MAX_WIDTH, PE_PROPOSE_SCRATCH_PER_DEPTH = 16, 64, 512
PE_ACCEPT_NOALLOC_MAX_NODES = 64 * PE_TREE_MAX_WORDS
PE_LOOP_REC_HEAD = 4

_ERR_NAMES = {
    PE_ERR_ARG: "invalid argument",
    PE_ERR_LAUNCH: "kernel launch failed",
    PE_ERR_TREE: "parents are not a topologically ordered tree (or tree too large)",
    PE_ERR_CAPACITY: "KV cache capacity or position table exceeded",
    PE_ERR_MASK: "attention bias is not a prefix + ancestor tree mask",
    PE_ERR_TOKEN: "token id outside the vocabulary",
    PE_ERR_INDEX: "keep index not strictly increasing or out of range",
    PE_ERR_WORKSPACE: "workspace too small",
    PE_ERR_VALUE: "NaN in a logit row, or a row with no finite value",
}


class PEError(RuntimeError):
    def __init__(self, status: int, where: str = ""):
        names = [v for k, v in _ERR_NAMES.items() if status & k] or [f"status {status}"]
        super().__init__(f"{where}: " + "; ".join(names) if where else "; ".join(names))
        self.status = status


vp = C.c_void_p
i32 = C.c_int32
i64 = C.c_int64
u64 = C.c_uint64
f32 = C.c_float
f64 = C.c_double


class ModelDesc(C.Structure):
    _fields_ = [
        ("num_layers", i32), ("hidden", i32), ("num_heads", i32), ("num_kv_heads", i32),
        ("head_dim", i32), ("intermediate", i32), ("vocab", i32), ("intermediate_padded", i32),
        ("dtype", i32), ("weight_format", i32), ("qkv_layout", i32), ("rms_eps", f32), ("norm_mode", i32),
        ("embed_rows", i32), ("attn_mode", i32), ("_reserved", i32), ("max_positions", i64),
        ("embed", vp), ("final_norm", vp), ("lm_head", vp), ("rope_cos_sin", vp),
        ("attn_norm", C.POINTER(vp)), ("mlp_norm", C.POINTER(vp)),
        ("w_qkv", C.POINTER(vp)), ("a_qkv", C.POINTER(vp)), ("b_qkv", C.POINTER(vp)),
        ("w_o", C.POINTER(vp)), ("a_o", C.POINTER(vp)),
        ("w_gu", C.POINTER(vp)), ("a_gu", C.POINTER(vp)),
        ("w_down", C.POINTER(vp)), ("a_down", C.POINTER(vp)),
    ]


class PassArgs(C.Structure):
    _fields_ = [
        ("input_ids", vp), ("positions", vp), ("M", i32), ("mask_mode", i32), ("prefix_len", i64),
        ("tree_bits", vp), ("bits_words", i32), ("num_features", i32), ("feature_layers", i32 * 4),
        ("_pad", i32), ("k_cache", vp), ("v_cache", vp), ("cache_capacity", i64), ("logits", vp),
        ("fused", vp), ("workspace", vp), ("workspace_bytes", i64), ("status", vp),
        ("batch", i32), ("max_seq_rows", i32), ("seq_row0", vp), ("seq_prefix", vp), ("cache_seq_stride", i64),
        ("node_keys", vp),
    ]


# name -> (restype, argtypes); must list every function declared in include/pe_hip.h
SIGNATURES: dict[str, tuple] = {
    "pe_status_string": (C.c_char_p, [C.c_int]),
    "pe_version": (C.c_int, []),
    "pe_fill_normal": (C.c_int, [vp, i64, C.c_int, u64, u64, f64, vp]),
    "pe_fill_uniform_int": (C.c_int, [vp, i64, i64, u64, u64, vp]),
    "pe_nf4_quantize": (C.c_int, [vp, i64, i64, vp, vp, vp]),
    "pe_nf4_repack": (C.c_int, [vp, vp, i64, i64, vp, vp, vp]),
    "pe_nf4_dequant": (C.c_int, [vp, vp, i64, i64, vp, vp]),
    "pe_nf4_repack_f32abs": (C.c_int, [vp, vp, i64, i64, vp, vp, vp]),
    "pe_nf4_dequant_f32abs": (C.c_int, [vp, vp, i64, i64, vp, vp]),
    "pe_nf4_absmax_dequant": (C.c_int, [vp, i64, vp, vp, C.c_int, C.c_float, vp, vp]),
    "pe_dense_repack": (C.c_int, [vp, i64, i64, C.c_int, vp, vp]),
    "pe_gemm_workspace_bytes": (i64, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "pe_nf4_gemm": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, i64, vp, i64,
                              vp, i64, vp]),
    "pe_nf4_gemm_f32abs": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, i64, vp, i64,
                                     vp, i64, vp]),
    "pe_nf4_gemm_tiled": (C.c_int, [vp, C.c_int, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp, i64, vp, i64, C.c_int,
                                    vp, i64, vp]),
    "pe_nf4_gemm_partials_bytes": (i64, [C.c_int, C.c_int, C.c_int]),
    "pe_nf4_gemm_partials": (C.c_int, [vp, i64, C.c_int, C.c_int, C.c_int, vp, vp, C.c_int, vp, i64,
                                       C.POINTER(C.c_int), vp]),
    "pe_dense_gemm": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, C.c_int, C.c_int, C.c_int, vp, vp, i64, vp,
                                i64, vp, i64, vp]),
    "pe_embed": (C.c_int, [vp, C.c_int, vp, i64, C.c_int, C.c_int, vp, i64, vp, vp]),
    "pe_rmsnorm": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, f32, C.c_int, vp, i64, vp]),
    "pe_rmsnorm_ex": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, f32, C.c_int, C.c_int, vp, i64, vp]),
    "pe_rope_qkv": (C.c_int, [vp, i64, C.c_int, C.c_int, C.c_int, C.c_int, vp, vp, i64, C.c_int, vp, vp, vp,
                              i64, i64, vp, vp]),
    "pe_copy_rows": (C.c_int, [vp, i64, C.c_int, i64, vp, i64, vp]),
    "pe_tree_masks": (C.c_int, [vp, C.c_int, i64, vp, C.c_int, vp, vp, vp, vp]),
    "pe_tree_allow_dense": (C.c_int, [vp, C.c_int, C.c_int, i64, vp, vp]),
    "pe_bias_to_bits": (C.c_int, [vp, i64, C.c_int, C.c_int, i64, vp, C.c_int, vp, vp]),
    "pe_attention_workspace_bytes": (i64, [C.c_int, C.c_int, C.c_int, C.c_int, i64, C.c_int]),
    "pe_tree_attention": (C.c_int, [vp, vp, vp, i64, C.c_int, C.c_int, C.c_int, C.c_int, i64, C.c_int, vp,
                                    C.c_int, f32, C.c_int, vp, i64, vp, i64, vp]),
    "pe_attention_batch_workspace_bytes": (i64, [C.c_int, C.c_int, C.c_int, i64, C.c_int]),
    "pe_tree_attention_batch": (C.c_int, [vp, vp, vp, i64, i64, C.c_int, C.c_int, C.c_int, i64, C.c_int, vp, vp,
                                          vp, C.c_int, f32, C.c_int, vp, i64, vp, i64, vp]),
    "pe_argmax_rows": (C.c_int, [vp, i64, C.c_int, i64, C.c_int, vp, vp]),
    "pe_accept_tree": (C.c_int, [vp, vp, i64, C.c_int, i64, C.c_int, vp, vp, vp, vp, vp]),
    "pe_accept_tree_keys": (C.c_int, [vp, i64, C.c_int, vp, C.c_int, C.c_int, vp, vp, vp, vp, vp]),
    "pe_dense_gemm_argmax_groups": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "pe_dense_gemm_argmax": (C.c_int, [vp, i64, C.c_int, C.c_int, vp, C.c_int, C.c_int, vp, i64, vp, vp, i64, vp]),
    "pe_accept_tree_noalloc": (C.c_int, [vp, vp, i64, C.c_int, i64, C.c_int, vp, vp, vp, vp]),
    "pe_propose_tree": (C.c_int, [vp, i64, C.c_int, i64, C.c_int, C.POINTER(C.c_int32), C.c_int, vp, vp,
                                  C.POINTER(C.c_int32), vp, vp, vp]),
    "pe_kv_compact": (C.c_int, [vp, vp, C.c_int, C.c_int, i64, C.c_int, C.c_int, i64, vp, vp]),
    "pe_kv_gather": (C.c_int, [vp, vp, C.c_int, C.c_int, i64, C.c_int, C.c_int, vp, i64, vp, vp]),
    "pe_forward_workspace_bytes": (i64, [C.POINTER(ModelDesc), C.c_int, i64]),
    "pe_forward": (C.c_int, [C.POINTER(ModelDesc), C.POINTER(PassArgs), vp]),
    "pe_forward_batch_workspace_bytes": (i64, [C.POINTER(ModelDesc), C.c_int, C.c_int, i64, C.c_int]),
    "pe_tree_masks_batch": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, vp, C.c_int, vp, vp, vp, vp]),
    "pe_accept_tree_batch": (C.c_int, [vp, i64, vp, i64, i64, C.c_int, vp, C.c_int, C.c_int, vp, vp, vp, vp, vp]),
    "pe_kv_compact_batch": (C.c_int, [vp, vp, C.c_int, i64, C.c_int, C.c_int, i64, C.c_int, C.c_int, vp, vp,
                                      C.c_int, vp]),
    "pe_loop_commit": (C.c_int, [vp, C.c_int, vp, vp, C.c_int, vp, i64, C.c_int, vp, vp, vp, i64, vp, vp, C.c_int,
                                 vp, vp, vp, vp]),
    "pe_loop_miss_commit": (C.c_int, [vp, C.c_int, vp, C.c_int, vp, C.c_int, vp, vp, i64, vp, vp, vp, vp, vp, vp]),
}

_lib = None


def load(path: Path | str | None = None):
    """Load (once) and return the configured ctypes library."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"{p} is missing: build it with `python -m parallel_eagle_amd.build` "
            "(parallel_eagle_amd has no CPU fallback)"
        )
    lib = C.CDLL(str(p), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def hip_runtime_mappings() -> list[str]:
    """Distinct libamdhip64 files mapped into this process."""
    seen = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[5]:
                seen.add(os.path.realpath(parts[5]))
    return sorted(seen)


def check(status: int, where: str) -> None:
    if status != PE_OK:
        raise PEError(status, where)
