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

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import nf4 as onf4
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


def _close(a: torch.Tensor, b: torch.Tensor, tol: float, ref32: torch.Tensor | None = None,
           min_frac: float = 0.95) -> tuple[bool, float]:
    """Parity of a GPU tensor ``a`` with the oracle's ``b``; returns (ok, max |a - b|).

    fp32 (``ref32`` None): every element within rtol = atol = tol.
    bf16/fp16: the oracle itself deviates from an fp32 evaluation of the same
    weights by more than 2e-2 on some logits (its own rounding: torch's CPU
    flash attention uses its own approximate exp, so no other implementation
    reproduces its bf16 roundings), so the check is (i) at least ``min_frac`` of
    the elements within rtol = atol = tol and (ii) the GPU no farther from the
    fp32 evaluation than the oracle is (relative L2, 10% slack)."""
    a, b = a.float().cpu(), b.float().cpu()
    d = (a - b).abs()
    inside = (d <= tol + tol * b.abs()).float().mean().item()
    if ref32 is None:
        return inside == 1.0, float(d.max())
    r = ref32.float().cpu()
    e_gpu = ((a - r).norm() / r.norm()).item()
    e_orc = ((b - r).norm() / r.norm()).item()
    ok = inside >= min_frac and e_gpu <= 1.1 * e_orc + 1e-6
    if not ok:
        print(f"parity: inside {inside:.5f} (need {min_frac}), relL2 gpu-vs-fp32 {e_gpu:.4g}, "
              f"oracle-vs-fp32 {e_orc:.4g}, max|gpu-oracle| {float(d.max()):.4g}")
    return ok, float(d.max())


def _margin(row: torch.Tensor) -> float:
    v = row.float().topk(2).values
    return float(v[0] - v[1])


def _check_acceptance(gpu, ref, o_root, o_nodes, g_root, g_nodes):
    """"exact" when the device's (path, bonus) equals the oracle's. Otherwise the
    first row where the two walks decide differently must be a near tie of that
    row: the oracle's top-1 / top-2 margin there at most twice the largest
    |device - oracle| difference of that same row (two logits moving by that
    much in opposite directions swap the order); anything else fails."""
    if gpu == ref:
        return "exact"
    path_g, bonus_g = gpu
    path_r, bonus_r = ref
    i = 0
    while i < min(len(path_g), len(path_r)) and path_g[i] == path_r[i]:
        i += 1
    node = None if i == 0 else path_r[i - 1]
    o_row = o_root if node is None else o_nodes[node]
    g_row = g_root if node is None else g_nodes[node]
    row_err = float((g_row.float().cpu() - o_row.float()).abs().max())
    m = _margin(o_row)
    assert m <= 2 * row_err, (f"acceptance differs at depth {i}: oracle margin {m:.4g} > twice the deciding "
                              f"row's logit error {row_err:.4g}")
    return f"near-tie at depth {i} (margin {m:.3g}, row error {row_err:.3g})"


def _fp32_oracle(shape, host_weights):
    """The same model evaluated in fp32 (NF4 weights dequantised to the bf16 operands
    the reference multiplies, then upcast): the yardstick for bf16/fp16 rounding."""
    def up(x):
        if isinstance(x, tuple):
            return onf4.dequantize_torch(x[1], x[2]).float()
        return x.float()

    hw32 = {"embed": up(host_weights["embed"]), "final_norm": up(host_weights["final_norm"]),
            "lm_head": up(host_weights["lm_head"]),
            "layers": [{k: up(v) for k, v in lw.items()} for lw in host_weights["layers"]]}
    return OracleTarget(replace(shape, dtype="float32", weight_format="dense"), hw32)


def _run_case(shape, seed, P, depth, widths, top_k, plant, tol, random_kv=False, tm=None):
    """tm: a model built with keep_logical=True (default: the seeded synthetic one)."""
    torch.manual_seed(0)
    if tm is None:
        tm = TargetModel.synthetic(shape, seed=seed, device=DEV, keep_logical=True, norm_noise=0.1,
                                   cache_capacity=P + 128)
    hw = tm.model.host_weights()
    orc = OracleTarget(shape, hw)
    orc.cache_dequant = True  # dequantise each NF4 matrix once; values are the same every call
    o32 = _fp32_oracle(shape, hw) if shape.dtype != "float32" else None
    V = shape.vocab
    cache = tm.make_cache()
    c32 = None
    if random_kv:
        # identical random prefix K/V for both paths
        g = torch.Generator().manual_seed(seed)
        kk = (torch.randn(cache.k[:, :, :P].shape, generator=g)).to(tm.dtype)
        vv = (torch.randn(cache.v[:, :, :P].shape, generator=g)).to(tm.dtype)
        cache.k[:, :, :P] = kk.to(DEV)
        cache.v[:, :, :P] = vv.to(DEV)
        cache.seq_len = P
        o_cache = [(kk[li].unsqueeze(0), vv[li].unsqueeze(0)) for li in range(shape.num_layers)]
        if o32 is not None:
            c32 = [(a.float(), b.float()) for a, b in o_cache]
        last = int(synth.uniform_int(seed, synth.STREAM_PROMPT, 1, V)[0])
        # the root logit comes from a 1-token continuation of the random prefix
        root_g, _, cache = tm.forward_cached(torch.tensor([[last]]), cache, torch.tensor([[P]]))
        root_o, _, o_cache = orc.forward([last], [P], o_cache, None)
        root32 = None
        if o32 is not None:
            root32, _, c32 = o32.forward([last], [P], c32, None)
        P = P + 1
    else:
        prompt = synth.uniform_int(seed, synth.STREAM_PROMPT, P, V).tolist()
        root_g, _, cache = tm.forward_cached(torch.tensor([prompt]), cache, torch.arange(P).unsqueeze(0))
        root_o, _, o_cache = orc.forward(prompt, list(range(P)), None, None)
        root32 = None
        if o32 is not None:
            root32, _, c32 = o32.forward(prompt, list(range(P)), None, None)
    ok, perr = _close(root_g[0, -1], root_o[0, -1], tol, None if root32 is None else root32[0, -1])
    assert ok, f"prefix logits differ by {perr}"
    # the oracle continues from its own prefix cache; the GPU from its own
    tokens, parents = synth.tree_for_seed(seed, V, depth, widths, top_k)
    a = plant(seed)
    tokens = _plant(orc, o_cache, root_o[0, -1], tokens, parents, a, V, P)
    pos = [P + d for d in om.tree_depths(parents)]
    bias_o = om.to_additive_bias(om.tree_allow_mask(parents, P)[P:, :], orc.dtype)
    o_lg, o_fu, o_cache2 = orc.forward(tokens, pos, o_cache, bias_o)
    r_lg = r_fu = r_cache = None
    if o32 is not None:
        bias32 = om.to_additive_bias(om.tree_allow_mask(parents, P)[P:, :], torch.float32)
        r_lg, r_fu, r_cache = o32.forward(tokens, pos, c32, bias32)
    lg, fu, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
    ok_l, lerr = _close(lg, o_lg, tol, r_lg)
    ok_f, ferr = _close(fu, o_fu, tol, r_fu)
    assert ok_l and ok_f, f"logits {lerr:.3g} / features {ferr:.3g} outside the parity bound (tol {tol})"
    # node K/V rows written by the pass
    for li in range(shape.num_layers):
        rk = None if r_cache is None else r_cache[li][0][0, :, P:]
        rv = None if r_cache is None else r_cache[li][1][0, :, P:]
        ok_k, kerr = _close(cache.k[li, :, P:P + len(tokens)], o_cache2[li][0][0, :, P:], tol, rk)
        ok_v, verr = _close(cache.v[li, :, P:P + len(tokens)], o_cache2[li][1][0, :, P:], tol, rv)
        assert ok_k and ok_v, f"layer {li} K/V rows differ: {kerr:.3g} / {verr:.3g}"
    gpu = accept_tree_cached(root_g[0, -1], lg[0], tokens, parents)
    ref = ov.accept_tree_cached(root_o[0, -1], o_lg[0], tokens, parents)
    verdict = _check_acceptance(gpu, ref, root_o[0, -1], o_lg[0], root_g[0, -1], lg[0])
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


@pytest.mark.parametrize("seed", WORKLOADS["llama2-7b-nf4-T26-P2048"].seeds)
def test_llama7b_nf4_width_two_layers(seed):
    """All ten workload seeds; a planted chain of 1..5 accepted nodes each. The
    committed path must equal the oracle's, except at a near tie of the deciding
    row (reported, and bounded by that row's own logit error)."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    v, n, err = _run_case(shape, seed, 48, wl.depth, wl.widths, wl.top_k, plant=lambda s: 1 + s % wl.depth,
                          tol=2e-2)
    print(f"seed {seed}: {v}, accepted {n}, max |dlogit| {err:.3g}")
    assert v == "exact" or v.startswith("near-tie")


@pytest.mark.parametrize("P", [130, 300])
def test_llama7b_nf4_width_prefill_longer_than_a_chunk(P):
    """A causal prefill of more than 64 tokens: 130 runs as 64-row fused chunks,
    300 (more than 256) takes the prefill path (each weight dequantised once, one
    bf16 GEMM over all rows, attention over all rows at once). Its logits, the K/V
    rows it appends and the tree pass on top match the oracle."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    v, n, err = _run_case(shape, 7, P, wl.depth, wl.widths, wl.top_k, plant=lambda s: 1 + s % wl.depth, tol=2e-2)
    print(f"P={P}: {v}, accepted {n}, max |dlogit| {err:.3g}")


@pytest.mark.parametrize("shape", [LLAMA2_7B_NF4.reduced(2),
                                   replace(QWEN25_14B_FP16.reduced(1, vocab=16384), dtype="bfloat16")],
                         ids=["nf4", "dense-bf16"])
def test_prefill_weight_copy_gives_the_same_prefill(shape):
    """pe_prefill_weights_fill keeps every linear as a row-major 16-bit copy and
    the prefill multiplies it instead of dequantising (NF4) or untiling (dense)
    per call: the same bf16 / fp16 operands, so the logits and the K/V rows the
    prefill appends are bit-identical to a prefill without the copy."""
    P = 300
    tm = TargetModel.synthetic(shape, seed=3, device=DEV, cache_capacity=P + 8)
    ids = torch.tensor([synth.uniform_int(3, synth.STREAM_PROMPT, P, shape.vocab).tolist()])
    pos = torch.arange(P).unsqueeze(0)
    c1 = tm.make_cache(P + 8)
    l1, _, c1 = tm.forward_cached(ids, c1, pos)
    nbytes = tm.model.enable_prefill_weights()
    s = shape
    per_weight = ((s.num_heads + 2 * s.num_kv_heads) * s.head_dim + s.num_heads * s.head_dim) * s.hidden \
        + 3 * tm.model.ipad * s.hidden
    assert nbytes == 2 * per_weight * s.num_layers
    c2 = tm.make_cache(P + 8)
    l2, _, c2 = tm.forward_cached(ids, c2, pos)
    assert torch.equal(l1, l2)
    assert torch.equal(c1.k[..., :P, :], c2.k[..., :P, :]) and torch.equal(c1.v[..., :P, :], c2.v[..., :P, :])


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


@pytest.mark.parametrize("shape,P,plant", [(WORKLOADS["tiny-fp32-T8-P64"].model, 64, 2),
                                           (LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2)), 300, 2),
                                           (LLAMA2_7B_NF4, 2048, 5),
                                           (QWEN25_14B_FP16.reduced(1, vocab=16384), 1200, 2)],
                         ids=["tiny-fp32", "llama7b-nf4-2layers", "llama7b-nf4-32layers-P2048",
                              "qwen14b-fp16-1layer-P1200"])
def test_verify_step_graph_replays_match_eager_api(shape, P, plant):
    """The device-resident step (masks -> forward -> acceptance -> compaction),
    eager and replayed from a HIP graph, equals forward_cached + accept_tree_cached
    + gather_cache on the same inputs, bit for bit, on every replay with eager
    work in between (the GQA case: two row tiles per KV head in 5 key splits,
    whose arrival counters return to zero after every launch). The full 32-layer 7B model (the benchmark's workload, too
    deep for the CPU oracle) is held to properties: every logit finite, and a
    chain of the device's own greedy tokens planted to the tree's full depth is
    accepted to that depth with the greedy bonus."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"] if shape.weight_format == "nf4" else WORKLOADS["tiny-fp32-T8-P64"]
    tm = TargetModel.synthetic(shape, seed=3, device=DEV, cache_capacity=P + 64)
    V = shape.vocab
    prompt = synth.uniform_int(3, synth.STREAM_PROMPT, P, V).tolist()
    cache = tm.make_cache()
    pl, _, cache = tm.forward_cached(torch.tensor([prompt]), cache, torch.arange(P).unsqueeze(0))
    root = pl[0, -1].clone()
    tokens, parents = synth.tree_for_seed(3, V, wl.depth, wl.widths, wl.top_k)
    # plant the device's greedy chain so the walk and the compaction move rows
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))[:plant]
    pos = [P + d for d in om.tree_depths(parents)]
    row = root
    for node in chain:
        synth.set_token(tokens, parents, node, int(row.float().argmax()), V)
        lg, _, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
        cache.crop(P)
        row = lg[0, node]
    k0 = cache.k.clone()
    v0 = cache.v.clone()
    # eager reference through the reference-shaped API
    lg_e, fu_e, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
    path_e, bonus_e = accept_tree_cached(root, lg_e[0], tokens, parents)
    tm.gather_cache(cache, torch.tensor(list(range(P)) + [P + t for t in path_e], device=DEV))
    k_e = cache.k[:, :, : cache.seq_len].clone()
    v_e = cache.v[:, :, : cache.seq_len].clone()
    assert path_e[: len(chain)] == chain
    assert bonus_e == int(lg_e[0, chain[-1]].float().argmax()) or len(path_e) > len(chain)
    assert bool(torch.isfinite(lg_e.float()).all()) and bool(torch.isfinite(fu_e.float()).all())
    # device-resident step over the same starting cache
    cache.k.copy_(k0)
    cache.v.copy_(v0)
    cache.seq_len = P
    step = tm.verify_step(cache, len(tokens))
    step.load_tree(tokens, parents, root)
    step.capture()
    for rep in range(3):
        step.run()
        got = step.result()
        assert got == (path_e, bonus_e), f"replay {rep}: {got} vs {(path_e, bonus_e)}"
        assert torch.equal(step.logits, lg_e[0]) and torch.equal(step.fused, fu_e[0])
        n = P + len(path_e)
        assert torch.equal(cache.k[:, :, :n], k_e) and torch.equal(cache.v[:, :, :n], v_e)
        # eager work between replays: scribble over the node rows and the outputs
        cache.k[:, :, P:P + len(tokens)].normal_()
        step.logits.zero_()
        torch.cuda.synchronize()
