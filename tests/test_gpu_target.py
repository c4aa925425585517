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

import ctypes as C
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import nf4 as onf4
from oracle import verify as ov
from oracle.model import OracleTarget
from parallel_eagle_amd import _lib, ops, synth
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
           info: dict | None = None) -> tuple[bool, float]:
    """Parity of a GPU tensor ``a`` with the oracle's ``b``; returns (ok, max |a - b|).

    fp32 (``ref32`` None): every element within rtol = atol = tol of the oracle.

    bf16/fp16: the tensor passes if every element is within rtol = atol = tol
    of the oracle (the bound itself), or if its relative L2 distance from an
    fp32 evaluation of the same weights is at most 1.1 times the oracle's and
    either (a) at least 99.9% of its elements are within the bound of the
    oracle, or (b) the count of its elements outside rtol = atol = tol of the
    fp32 evaluation is at most 1.25 times the oracle's count plus three times
    that count's square root.
    Why not the bound alone: over many bf16 layers the oracle itself deviates
    from the fp32 evaluation by more than ``tol`` on some elements (its own
    bf16 roundings; torch's CPU flash attention uses its own approximate exp,
    so no other implementation reproduces them), and the device, a second
    16-bit evaluation whose roundings fall independently, then differs from
    the oracle by up to twice that. So the device is held to the oracle's own
    distance from the fp32 evaluation. A rule that it be at least as close on
    every tensor fails about half the time with nothing wrong. The errors are
    correlated (one hidden row's error moves that row's every logit, and one
    layer's K or V rows), so the outside counts of small tensors and single
    rows fluctuate far beyond counting noise: (a) covers the fp16 14B model at
    full depth, where one to five of a deep layer's 26624 K or V elements fall
    just outside while L2 is equal, and the 1.25 of (b) its single root logit
    rows (outside counts 1.22 times the oracle's at an L2 ratio of 1.04).
    ``info`` receives the measured fractions and distances."""
    a, b = a.float().cpu(), b.float().cpu()
    d = (a - b).abs()
    inside_orc = (d <= tol + tol * b.abs()).float().mean().item()
    if info is not None:
        info.update(inside_vs_oracle=inside_orc, max_vs_oracle=float(d.max()))
    if ref32 is None:
        return inside_orc == 1.0, float(d.max())
    r = ref32.float().cpu()
    frac_dev = ((a - r).abs() <= tol + tol * r.abs()).float().mean().item()
    frac_orc = ((b - r).abs() <= tol + tol * r.abs()).float().mean().item()
    e_gpu = ((a - r).norm() / r.norm()).item()
    e_orc = ((b - r).norm() / r.norm()).item()
    n = a.numel()
    out_dev, out_orc = (1.0 - frac_dev) * n, (1.0 - frac_orc) * n
    count_ok = out_dev <= 1.25 * out_orc + 3.0 * out_orc ** 0.5 + 0.5
    ok = inside_orc == 1.0 or (e_gpu <= 1.1 * e_orc + 1e-6 and (inside_orc >= 0.999 or count_ok))
    if info is not None:
        info.update(inside_fp32_device=frac_dev, inside_fp32_oracle=frac_orc, rel_l2_device=e_gpu,
                    rel_l2_oracle=e_orc)
    if not ok:
        print(f"parity: within {tol} of fp32: device {frac_dev:.6f}, oracle {frac_orc:.6f}; relL2 vs fp32: device "
              f"{e_gpu:.4g}, oracle {e_orc:.4g}; max|gpu-oracle| {float(d.max()):.4g}, inside vs oracle "
              f"{inside_orc:.5f}")
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


def _fp32_oracle(shape, host_weights, orc=None):
    """The same model evaluated in fp32 (NF4 weights dequantised to the bf16 operands
    the reference multiplies, then upcast): the yardstick for bf16/fp16 rounding.
    With ``orc`` (cache_dequant on) each NF4 matrix is dequantised once for both."""
    def up(x):
        if isinstance(x, tuple):
            return (orc._weight(x) if orc is not None else onf4.dequantize_torch(x[1], x[2])).float()
        return x.float()

    hw32 = {"embed": up(host_weights["embed"]), "final_norm": up(host_weights["final_norm"]),
            "lm_head": up(host_weights["lm_head"]),
            "layers": [{k: up(v) for k, v in lw.items()} for lw in host_weights["layers"]]}
    return OracleTarget(replace(shape, dtype="float32", weight_format="dense"), hw32)


class Prepared:
    """A model on the device, its oracle (and fp32 evaluator) on the CPU, and
    optionally one random KV prefix shared by several seeds' cases (rows
    [0, P) are never written by a case, so they stay valid across cases)."""

    def __init__(self, shape, model_seed, P=None, kv_seed=None, cache_capacity=None, fp32=True, tm=None):
        torch.manual_seed(0)
        self.shape = shape
        if tm is None:
            tm = TargetModel.synthetic(shape, seed=model_seed, device=DEV, keep_logical=True, norm_noise=0.1,
                                       cache_capacity=cache_capacity or (P or 0) + 128)
        self.tm = tm
        hw = tm.model.host_weights()
        self.orc = OracleTarget(shape, hw)
        self.orc.cache_dequant = True  # dequantise each NF4 matrix once; values are the same every call
        self.o32 = _fp32_oracle(shape, hw, self.orc) if (shape.dtype != "float32" and fp32) else None
        self.cache = tm.make_cache()
        self.P = P
        self.o_cache = self.c32 = None
        if kv_seed is not None:
            # one random prefix K/V for both paths
            g = torch.Generator().manual_seed(kv_seed)
            kk = torch.randn(self.cache.k[:, :, :P].shape, generator=g).to(tm.dtype)
            vv = torch.randn(self.cache.v[:, :, :P].shape, generator=g).to(tm.dtype)
            self.cache.k[:, :, :P] = kk.to(DEV)
            self.cache.v[:, :, :P] = vv.to(DEV)
            self.o_cache = [(kk[li].unsqueeze(0), vv[li].unsqueeze(0)) for li in range(shape.num_layers)]
            if self.o32 is not None:
                self.c32 = [(a.float(), b.float()) for a, b in self.o_cache]


    def with_prefix(self, P, kv_seed, cache_capacity):
        """The same model, oracle and fp32 evaluator over another random prefix of P
        rows (a cache of its own)."""
        other = Prepared.__new__(Prepared)
        other.shape, other.tm, other.orc, other.o32, other.P = self.shape, self.tm, self.orc, self.o32, P
        other.cache = self.tm.make_cache(cache_capacity)
        g = torch.Generator().manual_seed(kv_seed)
        kk = torch.randn(other.cache.k[:, :, :P].shape, generator=g).to(self.tm.dtype)
        vv = torch.randn(other.cache.v[:, :, :P].shape, generator=g).to(self.tm.dtype)
        other.cache.k[:, :, :P] = kk.to(DEV)
        other.cache.v[:, :, :P] = vv.to(DEV)
        other.o_cache = [(kk[li].unsqueeze(0), vv[li].unsqueeze(0)) for li in range(self.shape.num_layers)]
        other.c32 = [(a.float(), b.float()) for a, b in other.o_cache] if self.o32 is not None else None
        return other


def _run_case(shape, seed, P, depth, widths, top_k, plant, tol, random_kv=False, tm=None, prep=None, details=None):
    """One seed's tree through forward_cached -> accept_tree_cached -> gather_cache
    on the device and through the oracle. ``prep``: a Prepared context (its random
    prefix of prep.P rows is shared; the root logit comes from a one-token
    continuation of it); otherwise one is made here (random_kv: a random prefix of
    P rows, else a prefill of P random tokens). ``details`` (dict) receives the
    per-seed measurements. Returns (verdict, accepted length, max |dlogit|)."""
    if prep is None:
        prep = Prepared(shape, seed, P=P, kv_seed=seed if random_kv else None, tm=tm, cache_capacity=P + 128)
        random_kv = random_kv
    else:
        random_kv, P = True, prep.P
    tm, orc, o32 = prep.tm, prep.orc, prep.o32
    V = shape.vocab
    cache = prep.cache
    c32 = None
    if random_kv:
        cache.seq_len = P
        o_cache = prep.o_cache
        c32 = prep.c32
        last = int(synth.uniform_int(seed, synth.STREAM_PROMPT, 1, V)[0])
        # the root logit comes from a 1-token continuation of the random prefix
        root_g, _, cache = tm.forward_cached(torch.tensor([[last]]), cache, torch.tensor([[P]]))
        root_o, _, o_cache = orc.forward([last], [P], o_cache, None)
        root32 = None
        if o32 is not None:
            root32, _, c32 = o32.forward([last], [P], c32, None)
        P = P + 1
    else:
        cache.seq_len = 0
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
    linfo = {}
    ok_l, lerr = _close(lg, o_lg, tol, r_lg, info=linfo)
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
    if details is not None:
        # the oracle's top-1 / top-2 margin at the row that decided the walk's end
        dec_row = root_o[0, -1] if not ref[0] else o_lg[0][ref[0][-1]]
        details.update(linfo, seed=seed, verdict=verdict, accepted=len(path), planted=a,
                       path_equal=gpu == ref, deciding_margin=_margin(dec_row), max_dlogit=lerr)
        if r_lg is not None:
            # the same walk on the fp32 evaluation's logits: which bf16 walk agrees with it
            w32 = ov.accept_tree_cached(root32[0, -1], r_lg[0], tokens, parents)
            details.update(device_walk_equals_fp32=gpu == w32, oracle_walk_equals_fp32=ref == w32)
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


@pytest.fixture(scope="module")
def two_layer_7b():
    """The 7B width at two layers over one random 2047-row prefix (the
    workload's P = 2048 once the root token is appended)."""
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    return Prepared(shape, 11, P=2047, kv_seed=2048, cache_capacity=2048 + 64)


@pytest.mark.parametrize("seed", WORKLOADS["llama2-7b-nf4-T26-P2048"].seeds)
def test_llama7b_nf4_width_two_layers(two_layer_7b, seed):
    """All ten workload seeds at the workload's P = 2048 (a shared random prefix
    plus each seed's root token); a planted chain of 1..5 accepted nodes each.
    The committed path must equal the oracle's, except at a near tie of the
    deciding row (reported, and bounded by that row's own logit error)."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    det = {}
    v, n, err = _run_case(two_layer_7b.shape, seed, None, wl.depth, wl.widths, wl.top_k,
                          plant=lambda s: 1 + s % wl.depth, tol=2e-2, prep=two_layer_7b, details=det)
    _report("7b-2layer-P2048", det)
    assert v == "exact" or v.startswith("near-tie")


def _report(case: str, det: dict) -> None:
    """Print one seed's parity record (and append it to $PE_PARITY_LOG as a JSON line)."""
    import json
    import os

    line = json.dumps({"case": case, **{k: (round(v, 6) if isinstance(v, float) else v) for k, v in det.items()}})
    print(line)
    path = os.environ.get("PE_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(line + "\n")


@pytest.fixture(scope="module")
def full_7b():
    """The whole 32-layer 7B NF4 workload model over one random 2047-row prefix:
    the oracle's weights dequantised once (bf16, about 13 GB of host memory) and
    an fp32 evaluator (about 26 GB)."""
    return Prepared(LLAMA2_7B_NF4, 0, P=2047, kv_seed=2048, cache_capacity=2048 + 64)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("seed", WORKLOADS["llama2-7b-nf4-T26-P2048"].seeds)
def test_llama7b_nf4_full_depth_against_the_oracle(full_7b, seed):
    """The benchmark's workload at full depth: 32 layers, P = 2048, T = 26, every
    workload seed with a planted chain of 1..5 nodes, through forward_cached ->
    accept_tree_cached -> gather_cache against the oracle restatement of
    target.py:203-224 and verify.py:104-125. Logits, features and every layer's
    appended K/V rows within the parity rule of _close; the committed path equal
    to the oracle's or a bounded near tie; the compaction bit-exact."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    det = {}
    v, n, err = _run_case(LLAMA2_7B_NF4, seed, None, wl.depth, wl.widths, wl.top_k,
                          plant=lambda s: 1 + s % wl.depth, tol=2e-2, prep=full_7b, details=det)
    _report("7b-32layer-P2048", det)
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


@pytest.fixture(scope="module")
def full_7b_p8192(full_7b):
    """The same model over a random 8191-row prefix (P = 8192 with the root token)."""
    return full_7b.with_prefix(8191, 8192, 8192 + 128)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("seed", [4, 5, 6])
def test_llama7b_nf4_T64_P8192_full_depth_against_the_oracle(full_7b_p8192, seed):
    """The long-context wide-tree workload at full depth: the 32-layer 7B NF4
    model, a 64-node depth-6 tree (widths [8,11,11,11,11,12]) over a random
    8191-row prefix plus the root token (P = 8192), a planted chain to the full
    depth, against the oracle: logits, features and K/V rows within the parity
    rule, acceptance exact or a bounded near tie, the compaction bit-exact."""
    wl = WORKLOADS["llama2-7b-nf4-T64-P8192"]
    det = {}
    v, n, err = _run_case(LLAMA2_7B_NF4, seed, None, wl.depth, wl.widths, wl.top_k, plant=lambda s: wl.depth,
                          tol=2e-2, prep=full_7b_p8192, details=det)
    _report("7b-32layer-T64-P8192", det)
    assert v == "exact" or v.startswith("near-tie")


@pytest.mark.parametrize("case", ["nf4-P2048", "dense-bf16-P300", "dense-fp16-P600"])
def test_prefill_through_the_many_row_kernels(case):
    """Causal prefills of more than 256 rows run every linear once over all rows
    on the library's many-row MFMA kernels (NF4: each weight dequantised once per
    256-row block inside the GEMM; dense 16-bit: tiled weights) and attention
    once over all rows: the 7B width at 2048 prompt tokens, and the 14B width
    (GQA 40/8, q/k/v bias) as a dense bf16 and a dense fp16 model. The prefill's
    last logit row (the root of the first tree), the tree pass on top and the
    K/V rows it appends match the oracle; acceptance exact or a bounded near tie."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    if case == "nf4-P2048":
        shape, P, seed = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2)), 2048, 8
    else:
        dt = "bfloat16" if "bf16" in case else "float16"
        shape = replace(QWEN25_14B_FP16.reduced(1, feature_layers=(0, 1, 1), vocab=16384), dtype=dt)
        P, seed = (300, 9) if dt == "bfloat16" else (600, 10)
    det = {}
    v, n, err = _run_case(shape, seed, P, wl.depth, wl.widths, wl.top_k, plant=lambda s: 3, tol=2e-2, details=det)
    _report(f"prefill-{case}", det)


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


@pytest.mark.parametrize("case", ["nf4-T100", "nf4-T200", "fp16-gqa-T100"])
def test_trees_wider_than_one_chunk(case):
    """Trees of more than 64 nodes (up to the 256 the bitmasks hold) through
    forward_cached: the pass runs as a batch of one sequence on the batched
    kernels (the many-row NF4 GEMM, the tree attention over row-tile pairs).
    Logits, features and K/V rows against the oracle, acceptance and the
    compaction as for every other case."""
    if case.startswith("nf4"):
        shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    else:
        shape = QWEN25_14B_FP16.reduced(1, feature_layers=(0, 1, 1), vocab=16384)
    if case.endswith("T200"):
        depth, widths, top_k = 6, [8, 32, 40, 40, 40, 40], 8
    else:
        depth, widths, top_k = 5, [8, 16, 24, 26, 26], 8
    det = {}
    v, n, err = _run_case(shape, 3, 300, depth, widths, top_k, plant=lambda s: depth, tol=2e-2, random_kv=True,
                          details=det)
    _report(f"wide-tree-{case}", det)
    assert v == "exact" or v.startswith("near-tie")


def test_verify_step_with_a_wide_tree_replays_the_eager_api():
    """VerifyStep over a 100-node tree (the pass as a batch of one, the walk
    from the node rows): eager and three graph replays, with eager work in
    between, equal forward_cached -> accept_tree_cached -> gather_cache bit for
    bit, a planted greedy chain accepted to full depth."""
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    P, depth, widths, top_k = 300, 5, [8, 16, 24, 26, 26], 8
    tm = TargetModel.synthetic(shape, seed=4, device=DEV, cache_capacity=P + 128)
    V = shape.vocab
    prompt = synth.uniform_int(4, synth.STREAM_PROMPT, P, V).tolist()
    cache = tm.make_cache()
    pl, _, cache = tm.forward_cached(torch.tensor([prompt]), cache, torch.arange(P).unsqueeze(0))
    root = pl[0, -1].clone()
    tokens, parents = synth.tree_for_seed(4, V, depth, widths, top_k)
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))
    pos = [P + d for d in om.tree_depths(parents)]
    row = root
    for node in chain:
        synth.set_token(tokens, parents, node, int(row.float().argmax()), V)
        lg, _, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
        cache.crop(P)
        row = lg[0, node]
    k0, v0 = cache.k.clone(), cache.v.clone()
    lg_e, fu_e, cache = tm.forward_cached(torch.tensor([tokens]), cache, torch.tensor([pos]), parents=parents)
    path_e, bonus_e = accept_tree_cached(root, lg_e[0], tokens, parents)
    assert path_e == chain
    tm.gather_cache(cache, torch.tensor(list(range(P)) + [P + t for t in path_e], device=DEV))
    n = cache.seq_len
    k_e, v_e = cache.k[:, :, :n].clone(), cache.v[:, :, :n].clone()
    cache.k.copy_(k0)
    cache.v.copy_(v0)
    cache.seq_len = P
    step = tm.verify_step(cache, len(tokens))
    step.load_tree(tokens, parents, root)
    step.capture()
    for rep in range(3):
        step.run()
        assert step.result() == (path_e, bonus_e), rep
        assert torch.equal(step.logits, lg_e[0]) and torch.equal(step.fused, fu_e[0])
        assert torch.equal(cache.k[:, :, :n], k_e) and torch.equal(cache.v[:, :, :n], v_e)
        cache.k[:, :, P:P + len(tokens)].normal_()
        step.logits.zero_()
        torch.cuda.synchronize()


@pytest.mark.parametrize("shape", [QWEN25_14B_FP16.reduced(1, feature_layers=(0, 1, 1), vocab=16384),
                                   QWEN25_14B_NF4.reduced(1, feature_layers=(0, 1, 1), vocab=16384)],
                         ids=["fp16", "nf4"])
def test_qwen14b_width_one_layer(shape):
    """Qwen2.5-14B width (GQA 40/8, q/k/v bias); vocabulary cut to 16384 to bound
    the CPU oracle's lm_head time."""
    wl = WORKLOADS["qwen2.5-14b-fp16-T26-P4096"]
    v, n, err = _run_case(shape, 1, 40, wl.depth, wl.widths, wl.top_k, plant=lambda s: 2, tol=2e-2)
    print(f"{shape.name}: {v}, accepted {n}, max |dlogit| {err:.3g}")


def _attention_splits(shape, T: int, S: int) -> int:
    """Key splits the library's attention plan gives T tree rows over S keys."""
    tiles = (T * shape.group + 31) // 32
    want = ((S + 31) // 32 + 7) // 8
    return max(1, min(want, min(256 // (shape.num_kv_heads * tiles), 16)))


def _device_prefix_pass(tm, cache, step, P: int, bound: int):
    """The step's pass (masks and forward) as a batch of one whose prefix P is
    read on the device and whose launches are sized for prefixes up to
    ``bound``; returns (logits, fused, K/V rows [P, P + T) of every layer)."""
    L = _lib.load()
    T = step.T
    dev = tm.device
    state = torch.tensor([P], dtype=torch.int64, device=dev)
    row0 = torch.tensor([0, T], dtype=torch.int32, device=dev)
    bits = torch.zeros_like(step.bits)
    pos = torch.zeros_like(step.pos)
    dep = torch.zeros_like(step.depth)
    st = ops.stream_ptr()
    _lib.check(L.pe_tree_masks_batch(step.parents.data_ptr(), row0.data_ptr(), state.data_ptr(), 1, T,
                                     bits.data_ptr(), step.words, pos.data_ptr(), dep.data_ptr(),
                                     tm.status.data_ptr(), st), "pe_tree_masks_batch")
    logits = torch.empty_like(step.logits)
    fused = torch.empty_like(step.fused)
    keys = torch.empty_like(step.node_keys)
    desc = tm.model.desc()
    ws = torch.zeros(int(L.pe_forward_batch_workspace_bytes(C.byref(desc), T, T, bound + T, 1)), dtype=torch.uint8,
                     device=dev)
    a = _lib.PassArgs.from_buffer_copy(step._args)
    a.positions, a.tree_bits = pos.data_ptr(), bits.data_ptr()
    a.logits, a.fused, a.node_keys = logits.data_ptr(), fused.data_ptr(), keys.data_ptr()
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    a.batch, a.max_seq_rows, a.prefix_len = 1, T, bound
    a.seq_row0, a.seq_prefix, a.cache_seq_stride = row0.data_ptr(), state.data_ptr(), cache.k.numel()
    _lib.check(L.pe_forward(C.byref(desc), C.byref(a), st), "pe_forward (device prefix)")
    ops.read_status(tm.status, "device prefix pass")
    return logits, fused, cache.k[:, :, P:P + T].clone(), cache.v[:, :, P:P + T].clone(), keys


@pytest.mark.parametrize("wl_name,shape,P,plant", [
    ("tiny-fp32-T8-P64", WORKLOADS["tiny-fp32-T8-P64"].model, 64, 2),
    ("llama2-7b-nf4-T26-P2048", LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2)), 300, 2),
    ("llama2-7b-nf4-T26-P2048", LLAMA2_7B_NF4, 2048, 5),
    ("qwen2.5-14b-fp16-T26-P4096", QWEN25_14B_FP16.reduced(1, vocab=16384), 1200, 2),
    ("qwen2.5-14b-fp16-T26-P4096", QWEN25_14B_FP16, 4096, 5),
    ("llama2-7b-nf4-T64-P8192", LLAMA2_7B_NF4, 8192, 6)],
    ids=["tiny-fp32", "llama7b-nf4-2layers", "llama7b-nf4-32layers-P2048", "qwen14b-fp16-1layer-P1200",
         "qwen14b-fp16-48layers-P4096", "llama7b-nf4-32layers-T64-P8192"])
def test_verify_step_graph_replays_match_eager_api(wl_name, shape, P, plant):
    """The device-resident step (masks -> forward -> acceptance -> compaction),
    eager and replayed from a HIP graph, equals forward_cached + accept_tree_cached
    + gather_cache on the same inputs, bit for bit, on every replay with eager
    work in between (the GQA case: two row tiles per KV head in 5 key splits,
    whose arrival counters return to zero after every launch). The full-depth
    workload models (the 32-layer 7B at P = 2048 and with 64-node trees at
    P = 8192, the 48-layer 14B fp16 with its 152064-token vocabulary at P = 4096)
    are also held to properties: every logit finite, and a chain of the device's
    own greedy tokens planted to the tree's full depth is accepted to that depth
    with the greedy bonus. For the 16-bit models the same pass with P read on
    the device (a batch of one, the launches sized for P and for P + 40) gives
    the same logits, features and K/V rows: bit for bit where the attention's
    key splits are the same."""
    wl = WORKLOADS[wl_name]
    tm = TargetModel.synthetic(shape, seed=3, device=DEV, cache_capacity=P + 128)
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
    T = len(tokens)
    kv_rows_e = (cache.k[:, :, P:P + T].clone(), cache.v[:, :, P:P + T].clone())
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
    step = tm.verify_step(cache, T)
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
    if shape.dtype == "float32":
        return
    for bound in (P, P + 40):
        cache.k.copy_(k0)
        cache.v.copy_(v0)
        lg_d, fu_d, k_d, v_d, keys_d = _device_prefix_pass(tm, cache, step, P, bound)
        same_plan = _attention_splits(shape, T, bound + T) == _attention_splits(shape, T, P + T)
        if same_plan:
            assert torch.equal(lg_d, lg_e[0]) and torch.equal(fu_d, fu_e[0]), bound
            assert torch.equal(k_d, kv_rows_e[0]) and torch.equal(v_d, kv_rows_e[1]), bound
        else:
            ok, err = _close(lg_d, lg_e[0].cpu(), 2e-2)
            assert (lg_d.float() - lg_e[0].float()).abs().max() < 0.25, (bound, err)
