"""Batched ragged verification on the GPU against batch-1 oracle runs.

The batched workload: B independent sequences, each with its own seeded tree
over its own cached prefix (lengths drawn from [512, 4096]), verified in one
pass (forward_tree_batch), walked in one launch (accept_tree_batch) and
committed in one launch (commit_batch: each sequence moves its own accepted
rows at its own prefix). Each sequence is checked against the oracle's
batch-1 restatement of the reference step (src/pe/target.py:203-224,
src/pe/decode/verify.py:104-125, src/pe/target.py:194-201 with the keep index
of src/pe/serve.py:308-309): logits, fused features and appended K/V rows
within the parity bound, acceptance exact (or a near tie of the deciding
row), committed rows bit-exact. Ragged tree sizes (up to 64 nodes) and the
graph-replayed step are checked too.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import verify as ov
from oracle.model import OracleTarget
from parallel_eagle_amd import batch as pb
from parallel_eagle_amd import ops, synth
from parallel_eagle_amd.config import LLAMA2_7B_NF4, QWEN25_14B_FP16, QWEN25_14B_NF4, WORKLOADS
from parallel_eagle_amd.target import TargetModel
from tests.test_gpu_target import _check_acceptance, _close, _fp32_oracle

pytestmark = pytest.mark.gpu
DEV = "cuda"
STREAM_BATCH_PREFIX = 8


def _batch_case(shape, seed, prefixes, trees_spec, plant, device_kv=False):
    """trees_spec: per sequence (depth, widths, top_k). Returns everything the
    checks need, after the batched pass, walk and commit. device_kv: the prefix
    K/V drawn on the device (no host copy for an oracle; property tests)."""
    B = len(prefixes)
    cap = max(prefixes) + 80
    tm = TargetModel.synthetic(shape, seed=seed, device=DEV, keep_logical=not device_kv, norm_noise=0.1,
                               cache_capacity=cap)
    V = shape.vocab
    cache = pb.BatchKVCache(tm, B, cap)
    kv_host = []
    if device_kv:
        ops.fill_normal(cache.k, seed, synth.STREAM_KV, 1.0)
        ops.fill_normal(cache.v, seed, synth.STREAM_KV_V, 1.0)
    for b, P in enumerate(prefixes):
        cache.seq(b).seq_len = P
        if device_kv:
            continue
        g = torch.Generator().manual_seed(1000 * seed + b)
        k = torch.randn(shape.num_layers, shape.num_kv_heads, P, shape.head_dim, generator=g).to(tm.dtype)
        v = torch.randn(shape.num_layers, shape.num_kv_heads, P, shape.head_dim, generator=g).to(tm.dtype)
        cache.k[b, :, :, :P] = k.to(DEV)
        cache.v[b, :, :, :P] = v.to(DEV)
        kv_host.append((k, v))
    g = torch.Generator().manual_seed(seed)
    roots = torch.randn(B, V, generator=g).to(tm.dtype)
    tokens, parents = [], []
    for b, (depth, widths, top_k) in enumerate(trees_spec):
        t, p = synth.tree_for_seed(16 * seed + b, V, depth, widths, top_k)
        tokens.append(t)
        parents.append(p)
    # plant each sequence's greedy chain (its root row's argmax, then the pass's own
    # node argmaxes) to a sequence-dependent depth
    chains = [synth.chain_nodes(parents[b], synth.deepest_first_leaf(parents[b]))[: plant(b)] for b in range(B)]
    for b in range(B):
        if chains[b]:
            synth.set_token(tokens[b], parents[b], chains[b][0], ov.first_argmax(roots[b]), V)
    for d in range(1, max(len(c) for c in chains)):
        lg, _, trees = pb.forward_tree_batch(tm, tokens, parents, cache)
        for b in range(B):
            if d < len(chains[b]):
                row = lg[trees.row0[b] + chains[b][d - 1]]
                synth.set_token(tokens[b], parents[b], chains[b][d], int(row.float().argmax()), V)
    lg, fu, trees = pb.forward_tree_batch(tm, tokens, parents, cache)
    if device_kv:  # pre-commit rows kept on the device
        pre_k = [cache.k[b, :, :, : prefixes[b] + trees.rows[b]].clone() for b in range(B)]
        pre_v = [cache.v[b, :, :, : prefixes[b] + trees.rows[b]].clone() for b in range(B)]
    else:
        pre_k = [cache.k[b, :, :, : prefixes[b] + trees.rows[b]].float().cpu().numpy() for b in range(B)]
        pre_v = [cache.v[b, :, :, : prefixes[b] + trees.rows[b]].float().cpu().numpy() for b in range(B)]
    out = pb.accept_batch_device(roots.to(DEV), lg, trees)
    pb.commit_batch(tm, cache, trees, out)
    res = [(row[2: 2 + row[0]], row[1]) for row in out.cpu().tolist()]
    return dict(tm=tm, cache=cache, kv=kv_host, roots=roots, tokens=tokens, parents=parents, chains=chains, lg=lg,
                fu=fu, trees=trees, pre_k=pre_k, pre_v=pre_v, res=res, prefixes=prefixes)


def _check_sequences(shape, c, tol=2e-2):
    hw = c["tm"].model.host_weights()
    orc = OracleTarget(shape, hw)
    orc.cache_dequant = True
    o32 = _fp32_oracle(shape, hw, orc)
    verdicts = []
    for b, P in enumerate(c["prefixes"]):
        tokens, parents = c["tokens"][b], c["parents"][b]
        T = len(tokens)
        r0 = c["trees"].row0[b]
        pos = [P + d for d in om.tree_depths(parents)]
        k, v = c["kv"][b]
        o_cache = [(k[li].unsqueeze(0), v[li].unsqueeze(0)) for li in range(shape.num_layers)]
        allow = om.tree_allow_mask(parents, P)[P:, :]
        o_lg, o_fu, o_new = orc.forward(tokens, pos, o_cache, om.to_additive_bias(allow, orc.dtype))
        c32 = [(a.float(), bb.float()) for a, bb in o_cache]
        r_lg, r_fu, r_new = o32.forward(tokens, pos, c32, om.to_additive_bias(allow, torch.float32))
        ok_l, lerr = _close(c["lg"][r0: r0 + T], o_lg[0], tol, r_lg[0])
        ok_f, ferr = _close(c["fu"][r0: r0 + T], o_fu[0], tol, r_fu[0])
        assert ok_l and ok_f, f"sequence {b} (P={P}): logits {lerr:.3g} / features {ferr:.3g} outside the bound"
        for li in range(shape.num_layers):
            got_k = torch.from_numpy(c["pre_k"][b][li, :, P:P + T])
            got_v = torch.from_numpy(c["pre_v"][b][li, :, P:P + T])
            ok_k, kerr = _close(got_k, o_new[li][0][0, :, P:], tol, r_new[li][0][0, :, P:])
            ok_v, verr = _close(got_v, o_new[li][1][0, :, P:], tol, r_new[li][1][0, :, P:])
            assert ok_k and ok_v, f"sequence {b} layer {li} K/V rows: {kerr:.3g} / {verr:.3g}"
        ref = ov.accept_tree_cached(c["roots"][b], o_lg[0], tokens, parents)
        verdict = _check_acceptance(c["res"][b], ref, c["roots"][b], o_lg[0], c["roots"][b], c["lg"][r0: r0 + T])
        verdicts.append(verdict)
        # ragged commit: rows [0, P) kept, P + i <- P + path[i], in every layer and head
        path = c["res"][b][0]
        assert c["cache"].seq(b).seq_len == P + len(path)
        n = P + len(path)
        assert np.array_equal(c["cache"].k[b, :, :, :n].float().cpu().numpy(), ov.compact_rows(c["pre_k"][b], P, path))
        assert np.array_equal(c["cache"].v[b, :, :, :n].float().cpu().numpy(), ov.compact_rows(c["pre_v"][b], P, path))
    return verdicts


def test_batched_ragged_qwen14b_nf4_width():
    """The batched workload's shape at one layer: Qwen2.5-14B width NF4 (GQA
    40/8, q/k/v bias), eight sequences of 26-node depth-5 trees over prefixes
    drawn from [512, 4096] (208 rows through every GEMM); the vocabulary cut to
    16384 bounds the CPU oracle."""
    wl = WORKLOADS["qwen2.5-14b-nf4-B8-T26"]
    shape = QWEN25_14B_NF4.reduced(1, feature_layers=(0, 1, 1), vocab=16384)
    prefixes = (synth.uniform_int(3, STREAM_BATCH_PREFIX, wl.batch, wl.prefix_len - wl.prefix_min + 1)
                + wl.prefix_min).tolist()
    spec = [(wl.depth, wl.widths, wl.top_k)] * wl.batch
    c = _batch_case(shape, 3, prefixes, spec, plant=lambda b: 1 + b % 4)
    assert c["trees"].M == 208
    verdicts = _check_sequences(shape, c)
    print("prefixes", prefixes, "verdicts", verdicts, "accepted", [len(r[0]) for r in c["res"]])
    assert sum(len(r[0]) for r in c["res"]) >= sum(1 + b % 4 for b in range(wl.batch)) - 2


def test_batched_ragged_tree_sizes_7b_width():
    """Trees of different sizes in one batch (26, 7 and 64 nodes: one and two
    32-row tiles) over prefixes of 100, 2048 and 300 rows, at the 7B width."""
    shape = LLAMA2_7B_NF4.reduced(1, feature_layers=(1, 1, 1))
    spec = [(5, (4, 5, 5, 6, 6), 4), (3, (2, 2, 3), 2), (6, (8, 11, 11, 11, 11, 12), 8)]
    c = _batch_case(shape, 5, [100, 2048, 300], spec, plant=lambda b: (3, 2, 5)[b])
    assert c["trees"].rows == [26, 7, 64]
    verdicts = _check_sequences(shape, c)
    print("verdicts", verdicts, "accepted", [len(r[0]) for r in c["res"]])


def test_batched_ragged_gqa_tree_sizes():
    """GQA rows of different counts in one batch at the 14B width (trees of 26, 7
    and 40 nodes: 130, 35 and 200 rows per KV head, seven row tiles of which the
    short tree fills two) over prefixes of 0, 900 and 2500 rows: the first
    sequence attends to its own node keys only, the others over several key
    splits combined by the last workgroup to arrive."""
    shape = QWEN25_14B_NF4.reduced(1, feature_layers=(0, 1, 1), vocab=16384)
    spec = [(5, (4, 5, 5, 6, 6), 4), (3, (2, 2, 3), 2), (5, (8, 8, 8, 8, 8), 8)]
    c = _batch_case(shape, 11, [0, 900, 2500], spec, plant=lambda b: (2, 1, 3)[b])
    assert c["trees"].rows == [26, 7, 40]
    verdicts = _check_sequences(shape, c)
    print("verdicts", verdicts, "accepted", [len(r[0]) for r in c["res"]])


def _graph_replays_equal_eager(c, prefixes):
    cache, tm = c["cache"], c["tm"]
    want = c["res"]
    k_e = [cache.k[b, :, :, : cache.seq(b).seq_len].clone() for b in range(len(prefixes))]
    # restore the pre-commit caches and lengths, then run the step
    for b, P in enumerate(prefixes):
        T = c["trees"].rows[b]
        cache.k[b, :, :, : P + T] = torch.as_tensor(c["pre_k"][b]).to(tm.dtype).to(DEV)
        cache.v[b, :, :, : P + T] = torch.as_tensor(c["pre_v"][b]).to(tm.dtype).to(DEV)
        cache.seq(b).seq_len = P
    step = pb.BatchVerifyStep(tm, cache, c["tokens"], c["parents"])
    step.root.copy_(c["roots"].to(DEV))
    step.capture()
    for rep in range(3):
        step.run()
        assert step.results() == want, f"replay {rep}"
        assert torch.equal(step.logits, c["lg"]) and torch.equal(step.fused, c["fu"])
        for b, P in enumerate(prefixes):
            n = P + len(want[b][0])
            assert torch.equal(cache.k[b, :, :, :n], k_e[b])
        cache.k[:, :, :, max(prefixes):].normal_()
        step.logits.zero_()
        torch.cuda.synchronize()


def test_batch_verify_step_graph_replays_match_eager():
    """BatchVerifyStep (masks -> batched pass -> walk -> ragged compaction), eager
    and replayed from a HIP graph, equals the eager batch API bit for bit, with
    eager work between the replays."""
    shape = QWEN25_14B_NF4.reduced(2, feature_layers=(1, 2, 2), vocab=16384)
    prefixes = [700, 1500, 3100, 520]
    spec = [(5, (4, 5, 5, 6, 6), 4)] * len(prefixes)
    c = _batch_case(shape, 7, prefixes, spec, plant=lambda b: 2 + b % 3)
    _graph_replays_equal_eager(c, prefixes)


def test_batched_workload_at_full_depth():
    """The batched workload itself: the 48-layer Qwen2.5-14B-shaped NF4 model
    with its 152064-token vocabulary, eight sequences over the workload's
    prefixes (drawn from [512, 4096]), 26-node trees. Held to properties: every
    logit finite, each sequence's planted chain of the device's own greedy
    tokens (1 to 5 deep) accepted to its depth, the ragged commit moving exactly
    the accepted rows, and the recorded step's replays equal to the eager batch
    API bit for bit."""
    wl = WORKLOADS["qwen2.5-14b-nf4-B8-T26"]
    prefixes = (synth.uniform_int(3, STREAM_BATCH_PREFIX, wl.batch, wl.prefix_len - wl.prefix_min + 1)
                + wl.prefix_min).tolist()
    spec = [(wl.depth, wl.widths, wl.top_k)] * wl.batch
    plant = lambda b: 1 + b % 5  # noqa: E731
    c = _batch_case(wl.model, 3, prefixes, spec, plant=plant, device_kv=True)
    assert c["trees"].M == 208
    assert bool(torch.isfinite(c["lg"].float()).all()) and bool(torch.isfinite(c["fu"].float()).all())
    for b, P in enumerate(prefixes):
        path = c["res"][b][0]
        assert path[: len(c["chains"][b])] == c["chains"][b], f"sequence {b}: {path} vs {c['chains'][b]}"
        n = P + len(path)
        got = c["cache"].k[b, :, :, :n]
        assert torch.equal(got[:, :, :P], c["pre_k"][b][:, :, :P])
        for i, t in enumerate(path):
            assert torch.equal(got[:, :, P + i], c["pre_k"][b][:, :, P + t])
    print("prefixes", prefixes, "accepted", [len(r[0]) for r in c["res"]])
    _graph_replays_equal_eager(c, prefixes)


@pytest.mark.parametrize("case", ["nf4-2x26", "dense-bf16-3x26"])
def test_row_major_batched_branch(case):
    """Batched passes that take the row-major branch (64-row launches over all
    sequences' rows, each row's K/V at its own sequence's slot): an NF4 batch of
    52 rows (two 26-node trees) and a dense bf16 batch (three trees, 78 rows,
    the GQA 40/8 width with q/k/v bias); each sequence against the oracle's
    batch-1 step, the ragged commit bit-exact."""
    spec7 = (5, (4, 5, 5, 6, 6), 4)
    if case == "nf4-2x26":
        shape = LLAMA2_7B_NF4.reduced(1, feature_layers=(1, 1, 1))
        prefixes = [300, 700]
    else:
        shape = replace(QWEN25_14B_FP16.reduced(1, feature_layers=(0, 1, 1), vocab=16384), dtype="bfloat16")
        prefixes = [100, 513, 1024]
    c = _batch_case(shape, 9, prefixes, [spec7] * len(prefixes), plant=lambda b: 1 + b % 3)
    assert c["trees"].M == 26 * len(prefixes)
    verdicts = _check_sequences(shape, c)
    print(case, "verdicts", verdicts, "accepted", [len(r[0]) for r in c["res"]])
