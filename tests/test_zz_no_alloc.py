"""pe_accept_tree_noalloc, the acceptance walk with a library-owned scratch
array instead of a caller's buffer, against pe_accept_tree through the C ABI:
two calls in a row on the same GPU (the second over a smaller tree, so the
array holds the first call's contents when the second starts), on random and
planted trees, bf16 and fp32; and the size limit is refused."""

import ctypes as C

import pytest
import torch

from oracle import verify as ov
from parallel_eagle_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, depth, widths, top_k, V, dtype):
    g = torch.Generator().manual_seed(seed)
    tokens, parents = synth.tree_for_seed(seed, V, depth, widths, top_k)
    T = len(tokens)
    root = torch.randn(V, generator=g)
    nodes = torch.randn(T, V, generator=g)
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))[: 1 + seed % depth]
    row = root
    for node in chain:
        row[tokens[node]] = 9.0
        row = nodes[node]
    return (root.to(dtype).to(DEV), nodes.to(dtype).to(DEV), torch.tensor(tokens, device=DEV),
            torch.tensor(parents, dtype=torch.int32, device=DEV), tokens, parents)


def _noalloc(root, nodes, tok, par, out):
    T, V = tok.numel(), root.numel()
    return _lib.load().pe_accept_tree_noalloc(root.data_ptr(), nodes.data_ptr(), nodes.stride(0), T, V,
                                              ops.dcode(root.dtype), tok.data_ptr(), par.data_ptr(), out.data_ptr(),
                                              ops.stream_ptr())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_walk_equals_the_scratch_walk_on_two_calls(dtype):
    cases = [(3, 6, (8, 11, 11, 11, 11, 12), 8, 32000), (4, 4, (2, 2, 2, 2), 2, 1024)]  # 64 nodes, then 8
    for seed, depth, widths, top_k, V in cases:
        root, nodes, tok, par, tokens, parents = _case(seed, depth, widths, top_k, V, dtype)
        T = tok.numel()
        want = ops.accept_tree(root, nodes, tok, par).cpu().tolist()
        out = torch.full((2 + T,), -7, dtype=torch.int32, device=DEV)
        assert _noalloc(root, nodes, tok, par, out) == _lib.PE_OK
        got = out.cpu().tolist()
        n = want[0]
        assert got[:2 + n] == want[:2 + n], (seed, got, want)
        # and both equal the oracle's walk
        assert (got[2:2 + n], got[1]) == ov.accept_tree_cached(root.cpu(), nodes.cpu(), tokens, parents)
        assert n >= 1 + seed % depth


def test_noalloc_refuses_trees_beyond_its_array():
    V, T = 64, _lib.PE_ACCEPT_NOALLOC_MAX_NODES + 1
    root = torch.zeros(V, dtype=torch.bfloat16, device=DEV)
    nodes = torch.zeros(T, V, dtype=torch.bfloat16, device=DEV)
    tok = torch.zeros(T, dtype=torch.int64, device=DEV)
    par = torch.full((T,), -1, dtype=torch.int32, device=DEV)
    out = torch.zeros(2 + T, dtype=torch.int32, device=DEV)
    assert _noalloc(root, nodes, tok, par, out) == _lib.PE_ERR_TREE
    assert _lib.load().pe_accept_tree_noalloc(None, None, 0, 1, V, _lib.PE_DTYPE_BF16, None, None, None,
                                              ops.stream_ptr()) == _lib.PE_ERR_ARG
    _ = C
