"""Beam tree proposal on the device (pe_propose_tree) against the oracle's
restatement of propose_tree (src/pe/decode/tree.py:34-55).

Three layers: each depth's candidates (tokens exactly, log-probabilities within
a few fp32 ulps of torch.log_softmax), the beam over the device's own
candidates (bit-exact: the same float64 sums and the same stable order), and the
whole proposal on fp32 logits (exact; random fp32 logits leave no near-ties).
"""
import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import tree as otree
from parallel_eagle_amd import _lib, ops, synth
from parallel_eagle_amd import tree as ptree

pytestmark = pytest.mark.gpu
DEV = "cuda"
W = _lib.PE_PROPOSE_MAX_WIDTH

CASES = [
    # (k, V, widths, top_k)
    (5, 32000, (3,) * 5, 3),            # the reference's rule at top_k 3, max_nodes 24
    (5, 32000, (4, 5, 5, 6, 6), 4),     # the 26-node tree of the verification workload
    (1, 7, (5,), 5),
    (3, 1000, (2, 8, 16), 3),           # widths above what the parents can fill
    (16, 1000, (2,) * 16, 2),           # deepest tree
    (4, 4096, (64,) * 4, 64),           # 4096 candidates per depth
]


def _logits(k, v, dtype, seed, scale=3.0):
    x = torch.from_numpy(synth.normal(seed, synth.STREAM_DRAFT, k * v, scale).reshape(k, v))
    return x.to(dtype)


def _run(lg, widths, top_k):
    k = lg.shape[0]
    scratch = torch.zeros(k * _lib.PE_PROPOSE_SCRATCH_PER_DEPTH, dtype=torch.uint8, device=DEV)
    tok, par, st = ops.propose_tree(lg.to(DEV), widths, top_k, scratch=scratch)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    lp = scratch[: k * W * 4].view(torch.float32).view(k, W).cpu()
    ids = scratch[k * W * 4: k * W * 8].view(torch.int32).view(k, W).cpu()
    return tok.cpu().tolist(), par.cpu().tolist(), lp, ids


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_candidates_and_beam_match_oracle(case, dtype):
    k, v, widths, top_k = CASES[case]
    lg = _logits(k, v, dtype, seed=case + 11)
    tokens, parents, lp, ids = _run(lg, widths, top_k)
    ref_lp = torch.log_softmax(lg.float(), dim=-1)
    topv, topi = [], []
    for d in range(k):
        c = min(top_k, widths[d])
        x = lg[d].float().numpy()
        want = np.lexsort((np.arange(v), -x))[:c]
        assert ids[d, :c].tolist() == want.tolist(), f"depth {d}"
        got = lp[d, :c]
        exp = ref_lp[d, want]
        assert torch.all((got - exp).abs() <= 4e-7 * (1 + exp.abs())), (got - exp).abs().max()
        topv.append([float(t) for t in got])
        topi.append(ids[d, :c].tolist())
    # the beam over the device's candidates, bit-exact
    assert (tokens, parents) == otree.beam_from_candidates(topv, topi, list(widths))
    assert om.is_topological(parents)
    # the whole proposal; the narrow trees' best sums are far apart next to the
    # few-ulp difference of the device's log-sum-exp
    if dtype == torch.float32 and max(widths) <= 16:
        assert (tokens, parents) == otree.propose_tree_beam(lg, list(widths), top_k)


@pytest.mark.parametrize("k,top_k,max_nodes,pending", [(5, 3, 24, 0), (4, 3, 48, 2), (6, 10, 24, 1), (3, 2, 2, 0)])
def test_reference_rule_and_pending(k, top_k, max_nodes, pending):
    lg = _logits(k + pending, 32000, torch.float32, seed=k * 7 + pending)
    got = ptree.propose_tree_from_logits(lg.to(DEV), k, top_k, max_nodes, pending)
    assert got == otree.reference_constant_width(lg[pending:], k, top_k, max_nodes)


def test_drop_in_propose_tree_calls_the_drafter():
    lg = _logits(7, 32000, torch.bfloat16, seed=5).to(DEV)
    calls = []

    class Drafter:
        def draft_logits(self, ids, feats, n):
            calls.append(n)
            return lg[:n]

    tokens, parents = ptree.propose_tree(Drafter(), None, None, 5, 3, 24, pending=2)
    assert calls == [7]
    w = ptree.beam_width(5, 3, 24)
    _, _, lp, ids = _run(lg[2:7].cpu(), [w] * 5, w)
    topv = [[float(t) for t in lp[d, :w]] for d in range(5)]
    topi = [ids[d, :w].tolist() for d in range(5)]
    assert (tokens, parents) == otree.beam_from_candidates(topv, topi, [w] * 5)


def test_equal_logits_lowest_index_first_and_stable_parents():
    lg = torch.tensor([[0.0, 2.0, 2.0, -1.0], [5.0, 5.0, 0.0, 0.0]])
    for dtype in (torch.float32, torch.bfloat16):
        tokens, parents, _, _ = _run(lg.to(dtype), [2, 3], 2)
        assert (tokens, parents) == ([1, 2, 0, 1, 0], [-1, -1, 0, 0, 1])


@pytest.mark.parametrize("bad", ["nan", "neg_inf_row", "pos_inf"])
def test_non_finite_rows_raise(bad):
    lg = _logits(3, 500, torch.float32, seed=3)
    if bad == "nan":
        lg[1, 17] = float("nan")
    elif bad == "neg_inf_row":
        lg[2] = float("-inf")
    else:
        lg[0, 3] = float("inf")
    with pytest.raises(_lib.PEError, match="NaN in a logit row"):
        ptree.propose_tree_from_logits(lg.to(DEV), 3, 2, 6)
    # -inf entries alone are ordinary (probability zero)
    ok = _logits(3, 500, torch.float32, seed=3)
    ok[:, :250] = float("-inf")
    assert ptree.propose_tree_from_logits(ok.to(DEV), 3, 2, 6) == otree.reference_constant_width(ok, 3, 2, 6)


@pytest.mark.parametrize("widths,top_k,v", [((65,), 3, 100), ((3,) * 17, 3, 100), ((3,), 3, 2), ((0,), 3, 100)])
def test_rejected_shapes(widths, top_k, v):
    lg = torch.zeros(len(widths), v, device=DEV)
    with pytest.raises(_lib.PEError):
        ops.propose_tree(lg, widths, top_k)
