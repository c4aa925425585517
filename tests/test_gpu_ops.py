"""The torch custom-op layer (torch.ops.pe.*) on the GPU.

Each op is the ctypes path it wraps, called through the torch dispatcher: the
masks (src/pe/masks.py:118-156), the verification pass (src/pe/target.py:
203-224), the walk (src/pe/decode/verify.py:104-125) and the compaction of
gather_cache (src/pe/target.py:194-201) give the same results bit for bit as
the library called directly, eagerly and captured in a HIP graph (replayed
several times with eager work in between); opcheck verifies each schema's
declared mutations and its fake implementation against the real one.
"""

import pytest
import torch

from parallel_eagle_amd import _lib, ops, synth
from parallel_eagle_amd.config import LLAMA2_7B_NF4, WORKLOADS
from parallel_eagle_amd.target import TargetModel

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(P=300):
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    tm = TargetModel.synthetic(shape, seed=5, device=DEV, cache_capacity=P + 64)
    cache = tm.make_cache()
    prompt = synth.uniform_int(5, synth.STREAM_PROMPT, P, shape.vocab).tolist()
    pl, _, cache = tm.forward_cached(torch.tensor([prompt]), cache, torch.arange(P)[None])
    tokens, parents = synth.tree_for_seed(5, shape.vocab, wl.depth, wl.widths, wl.top_k)
    # the device's own greedy token at the chain's first node, so the walk accepts it
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))
    synth.set_token(tokens, parents, chain[0], int(pl[0, -1].float().argmax()), shape.vocab)
    return tm, cache, pl[0, -1].contiguous(), tokens, parents


def _eager_ctypes(tm, cache, root, tok, par, P):
    """The same step through ops' ctypes wrappers (no dispatcher)."""
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    bits, pos, dep = ops.tree_masks(par, P, 1, status)
    ws = torch.zeros(tm.model.workspace_bytes(tok.numel(), P + tok.numel()), dtype=torch.uint8, device=DEV)
    lg, fu = ops.verify_pass(tm, tok, pos, bits, cache.k, cache.v, P, ws, status)
    out = ops.accept_tree(root, lg, tok, par)
    ops.kv_compact(cache.k, cache.v, P, out)
    torch.cuda.synchronize()
    assert int(status[0]) == 0
    return bits, pos, dep, lg, fu, out


def _same(got, want):
    """(bits, positions, depths, logits, fused, walk result) equal; of the walk's
    result only [|path|, bonus, path] is written."""
    for a, b in zip(got[:5], want[:5]):
        assert torch.equal(a, b)
    n = int(want[5][0])
    assert torch.equal(got[5][: 2 + n], want[5][: 2 + n])


def _through_ops(h, cache, root, tok, par, P, ws, status, scratch):
    bits, pos, dep = torch.ops.pe.tree_masks(par, P, 1, status)
    lg, fu = torch.ops.pe.verify_pass(h, tok, pos, bits, cache.k, cache.v, P, ws, status)
    out = torch.ops.pe.accept_tree(root, lg, tok, par, scratch)
    torch.ops.pe.kv_compact(cache.k, cache.v, P, out)
    return bits, pos, dep, lg, fu, out


def test_torch_ops_equal_the_ctypes_path_eagerly_and_in_a_graph():
    ops.register_torch_ops()
    P = 300
    tm, cache, root, tokens, parents = _setup(P)
    tok = torch.tensor(tokens, dtype=torch.int64, device=DEV)
    par = torch.tensor(parents, dtype=torch.int32, device=DEV)
    k0, v0 = cache.k.clone(), cache.v.clone()
    want = _eager_ctypes(tm, cache, root, tok, par, P)
    k_want, v_want = cache.k.clone(), cache.v.clone()
    assert int(want[5][0]) >= 1  # the planted node is accepted, so the compaction moves rows
    h = ops.register_model(tm)
    assert ops.register_model(tm) == h
    ws = torch.zeros(tm.model.workspace_bytes(len(tokens), P + len(tokens)), dtype=torch.uint8, device=DEV)
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    scratch = torch.zeros(len(tokens) + 2, dtype=torch.int32, device=DEV)
    # eager, through the dispatcher
    cache.k.copy_(k0)
    cache.v.copy_(v0)
    got = _through_ops(h, cache, root, tok, par, P, ws, status, scratch)
    torch.cuda.synchronize()
    _same(got, want)
    assert torch.equal(cache.k, k_want) and torch.equal(cache.v, v_want)
    assert int(status[0]) == 0
    # captured in a HIP graph, replayed with eager work in between
    cache.k.copy_(k0)
    cache.v.copy_(v0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = _through_ops(h, cache, root, tok, par, P, ws, status, scratch)
    for rep in range(3):
        cache.k.copy_(k0)
        cache.v.copy_(v0)
        g.replay()
        torch.cuda.synchronize()
        _same(outs, want)
        assert torch.equal(cache.k, k_want) and torch.equal(cache.v, v_want), rep
        outs[3].zero_()
        cache.k[:, :, P:].normal_()
        torch.cuda.synchronize()
    assert int(status[0]) == 0


def test_opcheck_schemas_and_fake_implementations():
    """torch.library.opcheck: the declared mutations match what each op writes and
    the fake implementations give the real outputs' shapes, dtypes and devices."""
    ops.register_torch_ops()
    P = 100
    tm, cache, root, tokens, parents = _setup(P)
    tok = torch.tensor(tokens, dtype=torch.int64, device=DEV)
    par = torch.tensor(parents, dtype=torch.int32, device=DEV)
    h = ops.register_model(tm)
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    bits, pos, _ = ops.tree_masks(par, P, 1, status)
    ws = torch.zeros(tm.model.workspace_bytes(len(tokens), P + len(tokens)), dtype=torch.uint8, device=DEV)
    lg, _ = ops.verify_pass(tm, tok, pos, bits, cache.k, cache.v, P, ws, status)
    out = ops.accept_tree(root, lg, tok, par)
    utils = ("test_schema", "test_faketensor")
    cases = [
        (torch.ops.pe.tree_masks.default, (par, P, 1, status)),
        (torch.ops.pe.verify_pass.default, (h, tok, pos, bits, cache.k, cache.v, P, ws, status)),
        (torch.ops.pe.accept_tree.default, (root, lg, tok, par, torch.zeros(len(tokens) + 2, dtype=torch.int32,
                                                                             device=DEV))),
        (torch.ops.pe.kv_compact.default, (cache.k, cache.v, P, out)),
        (torch.ops.pe.argmax_rows.default, (lg,)),
        (torch.ops.pe.rmsnorm.default, (lg[:, :4096].contiguous(), tm.model.final_norm, 1e-5)),
    ]
    for op, args in cases:
        torch.library.opcheck(op, args, test_utils=utils)
    assert int(status[0]) == 0


def test_a_bad_tree_through_the_op_reports_in_status():
    ops.register_torch_ops()
    par = torch.tensor([-1, 2, 0], dtype=torch.int32, device=DEV)  # not topological
    status = torch.zeros(4, dtype=torch.int32, device=DEV)
    torch.ops.pe.tree_masks(par, 10, 1, status)
    torch.cuda.synchronize()
    assert int(status[0]) & _lib.PE_ERR_TREE
