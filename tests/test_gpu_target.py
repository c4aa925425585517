"""End-to-end parity of the verification pass on the GPU against the CPU oracle.

For each workload shape (full size for the tiny fp32 model, full width with
fewer layers for the 7B / 14B shapes) and each seed: the same synthetic
weights, the same cached prefix and the same seeded tree (with a planted
accepted chain) go through

    TargetModel.forward_cached  ->  accept_tree_cached  ->  gather_cache

on the GPU and through the oracle restatement of the reference path on the CPU.
Checked: logits and fused features within tolerance (fp32 1e-4, bf16/fp16
2e-2), acceptance decisions and committed tokens equal (for bf16/fp16 a
mismatch is allowed only where the oracle's top-1/top-2 margin at the deciding
row is below the measured logit error, and is reported), and the compacted
cache equal to the oracle's gather of the GPU's own K/V rows.
"""

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import verify as ov
from oracle.model import OracleTarget
from parallel_eagle_amd import synth
from parallel_eagle_amd.config import LLAMA2_7B_NF4, QWEN25_14B_FP16, QWEN25_14B_NF4, WORKLOADS
from parallel_eagle_amd.target import TargetModel
from parallel_eagle_amd.verify import accept_tree_cached

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _plant(orc, cache, prompt_logit, tokens, parents, a, vocab, P):
    """Overwrite the first ``a`` nodes of the deepest first chain with the oracle's
    greedy tokens (siblings kept distinct)."""
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))[:a]
    pos = [P + d for d in om.tree_depths(parents)]
    bias = om.to_additive_bias(om.tree_allow_mask(parents, P)[P:, :], orc.dtype)
    row = prompt_logit
    for node in chain:
        synth.set_token(tokens, parents, node, ov.first_argmax(row), vocab)
        lg, _, _ = orc.forward(tokens, pos, cache, bias)
        row = lg[0, node]
    return tokens


def _margin(row: torch.Tensor) -> float:
    v = row.float().topk(2).values
    return float(v[0] - v[1])


def _check_acceptance(gpu, ref, o_root, o_nodes, tokens, parents, tol):
    if gpu == ref:
        return "exact"
    # walk the oracle's decisions: the first row where the GPU path diverges must be a near tie
    path_g, bonus_g = gpu
    path_r, bonus_r = ref
    i = 0
    while i < min(len(path_g), len(path_r)) and path_g[i] == path_r[i]:
        i += 1
    row = o_root if i == 0 else o_nodes[path_r[i - 1]]
    m = _margin(row)
    assert m <= 2 * tol, f"acceptance differs at depth {i} with oracle margin {m:.4g} > {2 * tol:.4g}"
    return f"near-tie at depth {i} (margin {m:.3g})"


def _run_case(shape, seed, P, depth, widths, top_k, plant, tol, random_kv=False):
    torch.manual_seed(0)
    tm = TargetModel.synthetic(shape, seed=seed, device=DEV, keep_logical=True, norm_noise=0.1,
                               cache_capacity=P + 128)
    orc = OracleTarget(shape, tm.model.host_weights())
    orc.cache_dequant = True  # dequantise each NF4 matrix once; values are the same every call
    V = shape.vocab
    cache = tm.make_cache()
    if random_kv:
        # identical random prefix K/V for both paths
        g = torch.Generator().manual_seed(seed)
        kk = (torch.randn(cache.k[:, :, :P].shape, generator=g)).to(tm.dtype)
        vv = (torch.randn(cache.v[:, :, :P].shape, generator=g)).to(tm.dtype)
        cache.k[:, :, :P] = kk.to(DEV)
        cache.v[:, :, :P] = vv.to(DEV)
        cache.seq_len = P
        o_cache = [(kk[li].unsqueeze(0), vv[li].unsqueeze(0)) for li in range(shape.num_layers)]
        last = int(synth.uniform_int(seed, synth.STREAM_PROMPT, 1, V)[0])
        # root logit: one causal token on both sides at position P - 1 is not defined here;
        # use a 1-token continuation from the random prefix instead
        root_g, _, cache = tm.forward_cached(torch.tensor([[last]]), cache, torch.tensor([[P]]))
        root_o, _, o_cache = orc.forward([last], [P], o_cache, None)
        P = P + 1
    else:
        prompt = synth.uniform_int(seed, synth.STREAM_PROMPT, P, V).tolist()
        root_g, _, cache = tm.forward_cached(torch.tensor([prompt]), cache, torch.arange(P).unsqueeze(0))
        root_o, _, o_cache = orc.forward(prompt, list(range(P)), None, None)
    perr = (root_g[0, -1].float().cpu() - root_o[0, -1].float()).abs().max().item()
    assert perr <= tol, f"prefix logits differ by {perr}"
    # the oracle continues from its own prefix cache; the GPU from its own
    tokens, parents = synth.tree_for_seed(seed, V, depth, widths, top_k)
    a = plant(seed)
    tokens = _plant(orc, o_cache, root_o[0, -1], tokens, parents, a, V, P)
    pos = [P + d for d in om.tree_depths(parents)]
    bias_o = om.to_additive_bias(om.tree_allow_mask(parents, P)[P:, :], orc.dtype)
    o_lg, o_fu, o_cache2 = orc.forward(tokens, pos, o_cache, bias_o)
    lg, fu, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
    lerr = (lg.float().cpu() - o_lg.float()).abs().max().item()
    ferr = (fu.float().cpu() - o_fu.float()).abs().max().item()
    assert lerr <= tol and ferr <= tol, f"logits {lerr:.3g} / features {ferr:.3g} exceed {tol}"
    # node K/V rows written by the pass
    for li in range(shape.num_layers):
        kerr = (cache.k[li, :, P:P + len(tokens)].float().cpu() - o_cache2[li][0][0, :, P:].float()).abs().max()
        assert kerr.item() <= tol
    gpu = accept_tree_cached(root_g[0, -1], lg[0], tokens, parents)
    ref = ov.accept_tree_cached(root_o[0, -1], o_lg[0], tokens, parents)
    verdict = _check_acceptance(gpu, ref, root_o[0, -1], o_lg[0], tokens, parents, lerr)
    # the acceptance kernel on the oracle's own logits must be bit-exact
    same = accept_tree_cached(root_o[0, -1].to(DEV), o_lg[0].to(DEV), tokens, parents)
    assert same == ref
    # commit: gather on the GPU vs the oracle's gather of the GPU's pre-commit rows
    path = gpu[0]
    before_k = cache.k[:, :, : P + len(tokens)].float().cpu().numpy()
    keep = torch.tensor(list(range(P)) + [P + t for t in path], device=DEV)
    tm.gather_cache(cache, keep)
    assert cache.seq_len == P + len(path)
    ref_k = ov.compact_rows(before_k, P, path)
    assert np.array_equal(cache.k[:, :, : cache.seq_len].float().cpu().numpy(), ref_k)
    return verdict, len(path), lerr


def test_tiny_fp32_full_workload():
    wl = WORKLOADS["tiny-fp32-T8-P64"]
    accepted = []
    for seed in wl.seeds:
        v, n, _ = _run_case(wl.model, seed, wl.prefix_len, wl.depth, wl.widths, wl.top_k,
                            plant=lambda s: s % (wl.depth + 1), tol=1e-4)
        assert v == "exact"
        accepted.append(n)
    assert max(accepted) >= 3  # the planted chains are accepted


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_llama7b_nf4_width_two_layers(seed):
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    v, n, err = _run_case(shape, seed, 48, wl.depth, wl.widths, wl.top_k, plant=lambda s: 1 + s % wl.depth,
                          tol=2e-2)
    print(f"seed {seed}: {v}, accepted {n}, max |dlogit| {err:.3g}")


def test_llama7b_nf4_width_long_random_prefix():
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    v, n, err = _run_case(shape, 5, 2047, wl.depth, wl.widths, wl.top_k, plant=lambda s: 3, tol=2e-2,
                          random_kv=True)
    print(f"P=2048: {v}, accepted {n}, max |dlogit| {err:.3g}")


def test_llama7b_nf4_width_wide_tree():
    wl = WORKLOADS["llama2-7b-nf4-T64-P8192"]
    shape = LLAMA2_7B_NF4.reduced(1, feature_layers=(1, 1, 1))
    v, n, err = _run_case(shape, 2, 300, wl.depth, wl.widths, wl.top_k, plant=lambda s: 4, tol=2e-2,
                          random_kv=True)
    print(f"T=64: {v}, accepted {n}, max |dlogit| {err:.3g}")


@pytest.mark.parametrize("shape", [QWEN25_14B_FP16.reduced(1, feature_layers=(0, 1, 1), vocab=16384),
                                   QWEN25_14B_NF4.reduced(1, feature_layers=(0, 1, 1), vocab=16384)],
                         ids=["fp16", "nf4"])
def test_qwen14b_width_one_layer(shape):
    """Qwen2.5-14B width (GQA 40/8, q/k/v bias); vocabulary cut to 16384 to bound
    the CPU oracle's lm_head time."""
    wl = WORKLOADS["qwen2.5-14b-fp16-T26-P4096"]
    v, n, err = _run_case(shape, 1, 40, wl.depth, wl.widths, wl.top_k, plant=lambda s: 2, tol=2e-2)
    print(f"{shape.name}: {v}, accepted {n}, max |dlogit| {err:.3g}")
