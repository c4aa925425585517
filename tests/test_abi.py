"""The C ABI library (CPU checks, no kernel launches): it loads, exports every
function include/pe_hip.h declares, binds to a single HIP runtime, and its host-
side argument validation rejects bad calls before launching anything."""

import ctypes as C
import re
from pathlib import Path

import pytest
import torch

from parallel_eagle_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pe_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libpe_hip.so not built")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), f"{n} missing from libpe_hip.so"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_single_hip_runtime(lib):
    maps = _lib.hip_runtime_mappings()
    assert len(maps) == 1, maps


def test_version_and_status_strings(lib):
    assert lib.pe_version() == 1
    assert lib.pe_status_string(0) == b"ok"
    assert b"topolog" in lib.pe_status_string(_lib.PE_ERR_TREE)


def test_host_validation_rejects_bad_arguments(lib):
    # null pointers and impossible shapes are refused before any launch
    assert lib.pe_nf4_gemm(None, 0, 26, 4096, None, None, 4096, 0, None, None, 0, None, 0, None, 0, None) \
        == _lib.PE_ERR_ARG
    assert lib.pe_nf4_repack(C.c_void_p(8), C.c_void_p(8), 32, 100, C.c_void_p(8), C.c_void_p(8), None) \
        == _lib.PE_ERR_ARG  # K not a multiple of 128
    assert lib.pe_tree_masks(C.c_void_p(8), 300, 0, C.c_void_p(8), 4, None, None, None, None) == _lib.PE_ERR_TREE
    assert lib.pe_tree_attention(C.c_void_p(8), C.c_void_p(8), C.c_void_p(8), 10, 4, 4, 128, 8, 5, 0,
                                 C.c_void_p(8), 1, 0.1, 1, C.c_void_p(8), 512, C.c_void_p(8), 1 << 20, None) \
        == _lib.PE_ERR_CAPACITY  # P + T > capacity
    assert lib.pe_rope_qkv(C.c_void_p(8), 0, 4, 6, 4, 128, C.c_void_p(8), C.c_void_p(8), 100, 1, C.c_void_p(8),
                           C.c_void_p(8), C.c_void_p(8), 10, 8, None, None) == _lib.PE_ERR_ARG  # nh % nkv
    assert lib.pe_dense_gemm(C.c_void_p(8), 0, 26, 4096, C.c_void_p(8), 1, 96, 2, None, None, 0,
                             C.c_void_p(8), 0, None, 0, None) == _lib.PE_ERR_ARG  # SwiGLU needs N % 64
    # a split-K shape without workspace is refused, not launched
    assert lib.pe_dense_gemm(C.c_void_p(8), 0, 26, 4096, C.c_void_p(8), 1, 4096, 2, None, None, 0,
                             C.c_void_p(8), 0, None, 0, None) == _lib.PE_ERR_WORKSPACE


@pytest.mark.parametrize("m,k", [(26, 128), (33, 256), (64, 4096), (1, 11008)])
def test_xtile_index_is_a_permutation_of_the_padded_tile(m, k):
    """The A-tiled activation order covers each element of the 32-row padded
    tile exactly once, keeps a lane's 8 columns contiguous, and puts 64
    consecutive lanes (one wave load) in 1 KiB of consecutive memory."""
    from parallel_eagle_amd import ops
    idx = ops.xtile_index(m, k).flatten()
    assert idx.unique().numel() == m * k
    assert idx.min().item() >= 0 and idx.max().item() < ((m + 31) // 32) * 32 * k
    # a lane's 8 consecutive columns are 8 consecutive elements
    full = ops.xtile_index(32, k)
    assert torch.equal(full[:, 8:16] - full[:, 8:9], torch.arange(8).expand(32, 8))
    # k-step s of unit 0: lanes (row r, half g) at ((s * 64) + r + 32 g) * 8
    for s in (0, 5):
        for g in (0, 1):
            col = 64 * g + 8 * s
            assert torch.equal(full[:, col], (s * 64 + torch.arange(32) + 32 * g) * 8)


def test_xtile_round_trip():
    from parallel_eagle_amd import ops
    x = torch.randn(40, 256)
    t = ops.to_xtile(x)
    assert t.numel() == 64 * 256
    assert torch.equal(ops.from_xtile(t, 40, 256), x)


@pytest.mark.parametrize("m", [1, 26, 33, 64])
@pytest.mark.parametrize("n,k", [(4096, 4096), (4096, 11008), (5120, 13824), (5120, 5120), (32000, 4096)])
def test_nf4_split_partials_fill_one_round(lib, m, n, k):
    """Split count of an NF4 split-partial launch, read from its workspace size:
    as many K splits as one round of one workgroup per CU holds (256 CUs, also
    the count the library assumes without a device) while every wave keeps at
    least two 128-wide units; with more 64-column groups than CUs, at least one
    split."""
    s, rem = divmod(int(lib.pe_nf4_gemm_partials_bytes(m, n, k)), m * n * 4)
    assert rem == 0
    groups, units = n // 64, k // 128
    if groups <= 256:
        assert s == max(1, min(256 // groups, units // 8))
    else:
        assert 1 <= s <= 16


def _desc_7b_nf4() -> _lib.ModelDesc:
    """A 7B-shaped NF4 model description (dimensions only: no weight is read
    by the checks below)."""
    d = _lib.ModelDesc()
    d.num_layers, d.hidden, d.num_heads, d.num_kv_heads, d.head_dim = 2, 4096, 32, 32, 128
    d.intermediate, d.intermediate_padded, d.vocab = 11008, 11008, 32000
    d.dtype, d.weight_format, d.qkv_layout = _lib.PE_DTYPE_BF16, _lib.PE_WFMT_NF4, _lib.PE_QKV_ROPE_PAIRED
    d.rms_eps, d.norm_mode, d.attn_mode, d.max_positions = 1e-5, _lib.PE_NORM_HF, _lib.PE_ATTN_SDPA, 4096
    return d


def _wide_tree_args(M: int, P: int, words: int, ws_bytes: int) -> _lib.PassArgs:
    a = _lib.PassArgs()
    a.input_ids = a.positions = a.tree_bits = a.k_cache = a.v_cache = a.workspace = 8
    a.M, a.mask_mode, a.prefix_len, a.bits_words = M, _lib.PE_MASK_TREE, P, words
    a.cache_capacity, a.workspace_bytes = P + M + 64, ws_bytes
    return a


def test_wide_tree_passes_are_validated_before_any_launch(lib):
    """A tree pass of 65-256 nodes runs as a batch of one sequence: its workspace
    (pe_forward_workspace_bytes) covers the batched layout plus the sequence
    table, and argument errors are refused before anything is launched."""
    d = _desc_7b_nf4()
    M, P = 100, 300
    need = lib.pe_forward_workspace_bytes(C.byref(d), M, P + M)
    batch = lib.pe_forward_batch_workspace_bytes(C.byref(d), M, M, P + M, 1)
    assert batch > 0 and need >= batch + 256
    a = _wide_tree_args(M, P, 2, need)
    a.node_keys = 8  # argmax keys are for passes of one chunk
    assert lib.pe_forward(C.byref(d), C.byref(a), None) == _lib.PE_ERR_ARG
    a = _wide_tree_args(M, P, 1, need)  # one word of ancestor bits cannot name 100 nodes
    assert lib.pe_forward(C.byref(d), C.byref(a), None) == _lib.PE_ERR_TREE
    a = _wide_tree_args(M, P, 2, batch)  # no room for the sequence table
    assert lib.pe_forward(C.byref(d), C.byref(a), None) == _lib.PE_ERR_WORKSPACE
    a = _wide_tree_args(300, P, 4, need)  # beyond the 256 nodes the bitmasks hold
    assert lib.pe_forward(C.byref(d), C.byref(a), None) == _lib.PE_ERR_TREE
