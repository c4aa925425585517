"""Pin the oracle's integer/byte functions (CPU): known answers from the
reference's tests, brute force on small inputs, closed forms and invariants."""

import itertools
import random

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import nf4 as onf4
from oracle import tree as otree
from oracle import verify as ov
from parallel_eagle_amd import synth
from parallel_eagle_amd.config import width_schedule


# ------------------------------------------------------------------ masks
def test_tree_mask_known_answer_from_reference_tests():
    # tests/test_masks.py:55-73 of the reference, re-expressed
    parents = [-1, 0, -1]
    assert om.tree_depths(parents) == [0, 1, 0]
    allow = om.tree_allow_mask(parents, prefix_len=2)
    assert allow.shape == (5, 5)
    assert allow[0, 0] and not allow[0, 1]
    assert allow[1, 0] and allow[1, 1]
    assert allow[2:, :2].all()
    assert allow[3, 2] and allow[3, 3] and not allow[3, 4]
    assert allow[2, 2] and not allow[2, 3] and not allow[2, 4]
    assert om.tree_position_ids(parents, prefix_len=2) == [0, 1, 2, 3, 2]


def _all_trees(t):
    """Every topologically ordered parent list of t nodes."""
    for choice in itertools.product(*[range(-1, i) for i in range(t)]):
        yield list(choice)


def _ancestors_brute(parents, node):
    # transitive closure by repeated relaxation (independent of the walk)
    anc = {node}
    changed = True
    while changed:
        changed = False
        for a in list(anc):
            p = parents[a]
            if p >= 0 and p not in anc:
                anc.add(p)
                changed = True
    return anc


@pytest.mark.parametrize("t", [1, 2, 3, 4, 5])
def test_tree_masks_brute_force(t):
    for parents in _all_trees(t):
        for P in (0, 1, 3):
            allow = om.tree_allow_mask(parents, P)
            bits = om.ancestor_bits(parents)
            n = P + t
            for i in range(n):
                for j in range(n):
                    if i < P:
                        exp = j <= i
                    elif j < P:
                        exp = True
                    else:
                        exp = (j - P) in _ancestors_brute(parents, i - P)
                    assert bool(allow[i, j]) == exp
            for i in range(t):
                assert bits[i] == sum(1 << a for a in _ancestors_brute(parents, i))
                assert om.tree_depths(parents)[i] == len(_ancestors_brute(parents, i)) - 1


def test_additive_bias_values():
    allow = om.tree_allow_mask([-1, 0, -1], 2)
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        b = om.to_additive_bias(allow, dt)
        assert b.shape == (1, 1, 5, 5)
        assert torch.equal(b[0, 0] == 0, torch.from_numpy(allow))
        assert (b[0, 0][~torch.from_numpy(allow)] == torch.finfo(dt).min).all()


# ------------------------------------------------------------------ acceptance
def _walk_brute(root, nodes, tokens, parents):
    """Acceptance by enumerating every root-to-node path: the accepted path is
    the longest chain whose every token equals the argmax of its predecessor
    row and which at each depth takes the lowest-index matching child."""
    am = [int(np.argmax(root))] + [int(np.argmax(r)) for r in nodes]
    path, cur, row = [], -1, 0
    while True:
        kids = sorted(t for t in range(len(parents)) if parents[t] == cur)
        match = [t for t in kids if tokens[t] == am[row]]
        if not match:
            return path, am[row]
        path.append(match[0])
        cur, row = match[0], 1 + match[0]


@pytest.mark.parametrize("seed", range(40))
def test_accept_tree_cached_brute_force(seed):
    rng = random.Random(seed)
    t, v = rng.randint(1, 7), rng.randint(2, 5)
    parents = [rng.randint(-1, i - 1) for i in range(t)]
    tokens = [rng.randrange(v) for _ in range(t)]
    logits = np.array([[rng.randint(0, 2) for _ in range(v)] for _ in range(t + 1)], dtype=np.float32)
    ref = _walk_brute(logits[0], logits[1:], tokens, parents)
    assert ov.accept_tree_cached(torch.from_numpy(logits[0]), torch.from_numpy(logits[1:]), tokens, parents) == ref
    # recompute variant: root row is P - 1, node t is row P + t
    P = 3
    full = np.concatenate([np.zeros((P - 1, v), np.float32), logits], 0)
    assert ov.accept_tree_greedy(torch.from_numpy(full), P, tokens, parents) == ref


def test_first_argmax_ties_and_nan():
    assert ov.first_argmax(torch.tensor([1.0, 3.0, 3.0])) == 1
    assert ov.first_argmax(torch.tensor([1.0, float("nan"), 3.0, float("nan")])) == 1
    assert ov.first_argmax(torch.tensor([2.0, 2.0], dtype=torch.bfloat16)) == 0


def test_compact_rows_keeps_prefix_and_path():
    rows = np.arange(2 * 10 * 3, dtype=np.float32).reshape(2, 10, 3)
    out = ov.compact_rows(rows, 4, [1, 3])
    assert np.array_equal(out[:, :4], rows[:, :4])
    assert np.array_equal(out[:, 4], rows[:, 5]) and np.array_equal(out[:, 5], rows[:, 7])


# ------------------------------------------------------------------ NF4
def test_nf4_table_properties():
    t = onf4.NF4_TABLE
    assert t.dtype == np.float32 and len(t) == 16
    assert t[7] == 0.0 and t[0] == -1.0 and t[15] == 1.0
    assert np.all(np.diff(t) > 0)


def test_nf4_table_closed_form_reconstruction():
    """QLoRA's construction: quantiles of N(0,1) at evenly spaced probabilities with
    offset 0.9677083, normalised by the largest; 8 positive and 7 negative levels
    plus zero. Agreement is ~1e-7, so this only pins the table's provenance."""
    from scipy.stats import norm

    offset = 0.9677083
    v1 = norm.ppf(np.linspace(offset, 0.5, 9)[:-1]).tolist()
    v3 = (-norm.ppf(np.linspace(offset, 0.5, 8)[:-1])).tolist()
    v = np.array(sorted(v1 + [0.0] + v3))
    v = v / v.max()
    assert np.max(np.abs(v - onf4.NF4_TABLE.astype(np.float64))) < 2e-6


def test_nf4_pack_unpack_round_trip_and_nibble_order():
    codes = np.array([[1, 2, 3, 4, 15, 0, 7, 9]], dtype=np.uint8)
    p = onf4.pack(codes)
    assert p.tolist() == [[0x12, 0x34, 0xF0, 0x79]]  # element 2j in the high nibble
    rng = np.random.default_rng(0)
    c = rng.integers(0, 16, size=(6, 128), dtype=np.uint8)
    assert np.array_equal(onf4.unpack(onf4.pack(c)), c)


def test_nf4_dequant_extremes_and_idempotence():
    w = synth.normal(1, 2, 64 * 256, 0.02).reshape(64, 256)
    p, a = onf4.quantize(w)
    codes = onf4.unpack(p)
    deq = onf4.bf16_bits_to_f32(onf4.dequantize(p, a)).reshape(64, 4, 64)
    amax = a.astype(np.float32)[..., None]
    c = codes.reshape(64, 4, 64)
    assert np.all(deq[c == 7] == 0.0)
    # code 15 / 0 dequantise to +/- bf16(absmax)
    bf_amax = onf4.bf16_bits_to_f32(onf4.f32_to_bf16_bits(np.broadcast_to(amax, c.shape).copy()))
    assert np.all(deq[c == 15] == bf_amax[c == 15])
    assert np.all(deq[c == 0] == -bf_amax[c == 0])
    # every block's max |w| maps to code 0 or 15
    blk_max = np.abs(w.reshape(64, 4, 64)).argmax(-1)
    picked = np.take_along_axis(c, blk_max[..., None], -1)[..., 0]
    assert np.all((picked == 0) | (picked == 15))
    # quantising the dequantised values again gives back the same codes
    p2, _ = onf4.quantize(deq.reshape(64, 256))
    assert np.array_equal(onf4.unpack(p2), codes)


def test_nf4_dequant_torch_is_bit_identical_to_numpy():
    """The threaded torch dequant (used for the timed CPU path) equals the
    numpy definition on every code and a spread of absmax values, including
    subnormal-range fp16 scales and values that round at the bf16 tie."""
    rng = np.random.default_rng(7)
    p = rng.integers(0, 256, size=(48, 512), dtype=np.uint8)
    a = rng.uniform(0, 0.1, size=(48, 16)).astype(np.float16)
    a[0, 0] = np.float16(6e-8)
    a[1, :] = np.float16(1.0)
    a[2, 3] = np.float16(0.0)
    ref = onf4.dequantize(p, a)
    got = onf4.dequantize_torch(p, a).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_nf4_quantize_nearest_code_brute_force():
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, size=(2, 128)).astype(np.float32)
    p, a = onf4.quantize(w)
    codes = onf4.unpack(p)
    for i in range(2):
        for j in range(128):
            s = np.float32(a[i, j // 64])
            xn = np.float32(w[i, j] / s)
            best = min(range(16), key=lambda c: (abs(float(np.float32(xn - onf4.NF4_TABLE[c]))), c))
            assert codes[i, j] == best


# ------------------------------------------------------------------ tree proposal
def test_width_schedules():
    assert width_schedule(8, 4, 2) == (2, 2, 2, 2)
    assert width_schedule(26, 5, 4) == (4, 5, 5, 6, 6)
    assert width_schedule(64, 6, 8) == (8, 11, 11, 11, 11, 12)
    assert width_schedule(15, 5, 3) == (3, 3, 3, 3, 3)


def test_tree_builder_matches_oracle_beam_and_reference_rule():
    logits = torch.from_numpy(synth.normal(4, synth.STREAM_DRAFT, 5 * 300).reshape(5, 300))
    for widths, top_k in [((4, 5, 5, 6, 6), 4), ((3, 3, 3, 3, 3), 3), ((2, 2, 2, 2, 2), 2)]:
        assert synth.build_tree(logits, widths, top_k) == otree.propose_tree_beam(logits, list(widths), top_k)
    # constant widths reduce to the reference's propose_tree beam (k=5, top_k=3, max_nodes=15)
    assert synth.build_tree(logits, (3,) * 5, 3) == otree.reference_constant_width(logits, 5, 3, 15)


def test_tree_builder_hand_case():
    # depth 0 logprobs favour tokens 2 > 1; depth 1 favours 0 > 3
    lg = torch.tensor([[0.0, 1.0, 2.0, -5.0], [3.0, -1.0, -1.0, 2.0]])
    tokens, parents = otree.propose_tree_beam(lg, [2, 2], 2)
    assert parents == [-1, -1, 0, 0]
    assert tokens == [2, 1, 0, 3]
    assert om.is_topological(parents)


def test_synth_generator_known_values():
    """Closed form of the counter-based generator for a few counters."""
    z = synth._hash(7, 9, 0, 3)
    s = [(int(x) & 0xFFFF) + ((int(x) >> 16) & 0xFFFF) + ((int(x) >> 32) & 0xFFFF) + (int(x) >> 48) for x in z]
    exp = [np.float32(((si + 2.0) / 65536.0 - 2.0) * 1.7320508075688772 * 0.5) for si in s]
    assert synth.normal(7, 9, 3, 0.5).tolist() == exp
    x = synth.normal(1, 1, 200_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    assert float(np.abs(x).max()) <= 2 * 1.7320508075688772 + 1e-6


@pytest.mark.parametrize("v,widths", [(6, (3, 3, 3)), (5, (4, 2, 2, 1)), (9, (1, 1, 1)), (4, (2, 2))])
def test_beam_is_the_global_best_sequences(v, widths):
    """Every depth's log-probabilities are the same for every parent, so with
    non-increasing widths the beam at depth d holds the best widths[d] token
    sequences of length d + 1 over all v^(d+1), best first (brute force)."""
    import itertools
    k = len(widths)
    lg = torch.from_numpy(synth.normal(v * 31 + k, synth.STREAM_DRAFT, k * v, 2.0).reshape(k, v))
    lp = torch.log_softmax(lg.float(), dim=-1).numpy().astype(np.float64)
    tokens, parents = otree.propose_tree_beam(lg, list(widths), max(widths))
    assert om.is_topological(parents)
    seqs = []
    for t in range(len(tokens)):
        s, a = [], t
        while a != -1:
            s.append(tokens[a])
            a = parents[a]
        seqs.append(tuple(reversed(s)))
    base = 0
    for d, w in enumerate(widths):
        every = sorted(itertools.product(range(v), repeat=d + 1), key=lambda q: -sum(lp[e, q[e]] for e in range(d + 1)))
        assert seqs[base: base + w] == every[:w]
        base += w
    assert base == len(tokens)


def test_beam_ties_take_the_lowest_token_then_the_earlier_parent():
    # depth 0: tokens 1 and 2 tie, token 1 first; depth 1: both parents extended by
    # the same row, equal sums keep parent-major order (the reference's stable sort)
    lg = torch.tensor([[0.0, 2.0, 2.0, -1.0], [5.0, 5.0, 0.0, 0.0]])
    tokens, parents = otree.propose_tree_beam(lg, [2, 3], 2)
    assert tokens == [1, 2, 0, 1, 0]
    assert parents == [-1, -1, 0, 0, 1]


# ------------------------------------------------------------------ drafter
def _drafter_weights(shape, n_layers, nfl, dt, seed, std=0.05):
    from dataclasses import replace
    H = shape.hidden
    g = torch.Generator().manual_seed(seed)

    def r(*sz, std=std):
        return (torch.randn(*sz, generator=g) * std).to(dt)

    layers = []
    for _ in range(n_layers):
        lw = {n: r(o, i) for n, o, i in replace(shape, qkv_bias=False).linear_shapes()}
        lw["attn_norm"] = (1 + r(H, std=0.1).float()).to(dt)
        lw["mlp_norm"] = (1 + r(H, std=0.1).float()).to(dt)
        layers.append(lw)
    w = {"feat_norm": (1 + r(H, std=0.1).float()).to(dt), "feat_proj": r(H, nfl * H), "in_proj": r(H, 2 * H),
         "mask_emb": r(H, std=0.02), "h_shared": r(H, std=0.02), "layers": layers}
    shared = {"embed": r(shape.vocab, H, std=0.5), "final_norm": (1 + r(H, std=0.1).float()).to(dt),
              "lm_head": r(shape.vocab, H)}
    return w, shared


def test_drafter_layers_equal_the_target_forward_in_fp32():
    """In fp32 the drafter's RMSNorm and the target's agree, so the drafter's
    layers + the shared final norm and lm_head over rows x, causal, equal the
    target oracle (pinned against transformers) whose embedding table is x."""
    from dataclasses import replace
    from oracle import drafter as od
    from oracle.model import OracleTarget
    from parallel_eagle_amd.config import TINY_LLAMA
    shape = replace(TINY_LLAMA, num_layers=2, feature_layers=(1, 2, 2))
    w, shared = _drafter_weights(shape, 2, 3, torch.float32, 0)
    dr = od.OracleDrafter(shape, w, shared, torch.float32)
    p, k = 9, 4
    ids = torch.randint(0, shape.vocab, (p,), generator=torch.Generator().manual_seed(1))
    feats = torch.randn(p, 3 * shape.hidden, generator=torch.Generator().manual_seed(2)) * 3
    x = torch.cat([dr.real_input(ids, feats), dr.mask_input(k - 1)])
    m = p + k - 1
    assert torch.equal(od.draft_allow_mask(p, k), torch.tril(torch.ones(m, m, dtype=torch.bool)))
    assert torch.equal(od.draft_positions(p, k), torch.arange(m))
    tw = {"embed": x, "final_norm": shared["final_norm"], "lm_head": shared["lm_head"],
          "layers": [dict(lw) for lw in w["layers"]]}
    logits_t, _, _ = OracleTarget(shape, tw).forward(torch.arange(m), torch.arange(m), None, None)
    got = dr.draft_logits(ids, feats, k)
    assert got.shape == (k, shape.vocab)
    assert torch.allclose(got, logits_t[0, p - 1:], rtol=1e-4, atol=1e-4), (got - logits_t[0, p - 1:]).abs().max()


def test_drafter_inputs_closed_forms():
    from dataclasses import replace
    from oracle import drafter as od
    from parallel_eagle_amd.config import TINY_LLAMA
    shape = replace(TINY_LLAMA, num_layers=1)
    H = shape.hidden
    w, shared = _drafter_weights(shape, 1, 2, torch.float32, 3)
    w["feat_norm"] = torch.ones(H)
    dr = od.OracleDrafter(shape, w, shared, torch.float32)
    ids = torch.tensor([3, 5, 7])
    feats = torch.randn(3, 2 * H) * torch.tensor([1.0] * H + [50.0] * H)
    # every feature block leaves the norm with unit RMS
    f = od.drafter_rms_norm(feats.unflatten(-1, (2, H)), w["feat_norm"], shape.rms_eps)
    assert torch.allclose(f.pow(2).mean(-1), torch.ones(3, 2), atol=1e-4)
    # in_proj of [emb; feat] is the sum of its column blocks applied separately
    feat = f.flatten(-2) @ w["feat_proj"].t()
    want = shared["embed"][ids] @ w["in_proj"][:, :H].t() + feat @ w["in_proj"][:, H:].t()
    assert torch.allclose(dr.real_input(ids, feats), want, atol=1e-5)
    mv = w["mask_emb"] @ w["in_proj"][:, :H].t() + w["h_shared"] @ w["in_proj"][:, H:].t()
    assert torch.allclose(dr.mask_input(2), mv.expand(2, -1), atol=1e-6)
