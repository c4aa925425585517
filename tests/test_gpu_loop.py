"""The decode loop and the drafter interface over the device path.

- Losslessness (tests/test_lossless.py:56-62 of the reference): the
  speculative loop (SpeculativeDecoder: the one-forward tree loop of
  src/pe/serve.py:221-355 with its state and step on the device) emits exactly
  the tokens of greedy decoding through forward_cached: exactly on the tiny
  fp32 model (kernels launched each step, P from the host), and at the 7B width
  in bf16 (recorded steps replayed, P read on the device) up to a near tie of
  the greedy decode itself. Drafters: an untrained device drafter (the miss
  path: one token at a time) and one that is told the greedy continuation at
  some depths (accepted paths of every length, compaction across steps).
- One host read per step, and the recorded steps equal the same kernels
  launched each step.
- The drafter's cached context is dropped between two prompts.
- The shared modules a reference drafter calls (src/pe/drafter.py:81-83,120,
  123,161): get_input_embeddings / get_lm_head / get_final_norm are callable
  and agree with the oracle.
"""

import random

import pytest
import torch

from oracle import drafter as od
from oracle.model import rms_norm
from parallel_eagle_amd import ops
from parallel_eagle_amd.config import LLAMA2_7B_NF4, TINY_LLAMA
from parallel_eagle_amd.drafter import DeviceDrafter
from parallel_eagle_amd.serve import SpeculativeDecoder, greedy_decode
from parallel_eagle_amd.target import TargetModel
from tests.test_oracle_pins import _drafter_weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


class PeekingDrafter:
    """A drafter that, per depth and with probability ``p``, replaces its logits
    by a peak at the token greedy decoding puts there (``greedy`` = prompt +
    greedy continuation): depth d of a call with n confirmed tokens predicts
    greedy[n + d]. The loop must stay lossless whatever the drafter proposes."""

    def __init__(self, inner, greedy: list[int], p: float, seed: int):
        self.inner, self.greedy, self.p = inner, greedy, p
        self.rng = random.Random(seed)

    @property
    def status(self):
        return self.inner.status

    @property
    def sync_status(self):
        return self.inner.sync_status

    @sync_status.setter
    def sync_status(self, v):
        self.inner.sync_status = v

    def reset(self):
        self.inner.reset()

    def draft_logits(self, ctx, feats, k):
        lg = self.inner.draft_logits(ctx, feats, k).clone()
        n = ctx.numel()
        for d in range(k):
            if n + d < len(self.greedy) and self.rng.random() < self.p:
                lg[d] = lg[d].min()
                lg[d, self.greedy[n + d]] = 30.0
        return lg


def _tiny():
    tm = TargetModel.synthetic(TINY_LLAMA, seed=1, device=DEV, norm_noise=0.1, cache_capacity=256)
    w, _ = _drafter_weights(TINY_LLAMA, 2, len(tm.feature_layers), torch.float32, seed=5, std=0.05)
    return tm, DeviceDrafter(tm, w, max_depth=5, capacity=256)


@pytest.mark.parametrize("p", [0.0, 0.6, 0.95])
def test_speculative_loop_is_lossless_on_the_tiny_fp32_model(p):
    tm, dr = _tiny()
    prompt = [1, 2, 3, 4, 5, 6]
    n = 48
    ref = greedy_decode(tm, prompt, n)
    assert len(ref.tokens) == n
    drafter = PeekingDrafter(dr, prompt + ref.tokens, p, seed=int(p * 100)) if p else dr
    dec = SpeculativeDecoder(tm, drafter, k=5, tree_top_k=3, tree_max_nodes=15)
    assert not dec.device_prefix  # fp32: kernels launched each step
    res = dec.generate(prompt, n)
    assert res.tokens == ref.tokens
    # one read per step, plus one at the end when the last step missed
    assert res.steps <= res.host_reads <= res.steps + 1
    if p >= 0.95:
        assert res.tokens_per_step > 2.0  # most steps commit several tokens
    print(f"p={p}: steps {res.steps}, target passes {res.target_passes}, tokens per step "
          f"{res.tokens_per_step:.2f}, host reads {res.host_reads}")


def test_speculative_loop_stops_at_eos():
    tm, dr = _tiny()
    prompt = [9, 8, 7]
    ref = greedy_decode(tm, prompt, 40)
    eos = ref.tokens[17]
    want = ref.tokens[: ref.tokens.index(eos) + 1]
    assert greedy_decode(tm, prompt, 40, eos_token_id=eos).tokens == want
    dr2 = PeekingDrafter(dr, prompt + ref.tokens, 0.7, seed=4)
    got = SpeculativeDecoder(tm, dr2, k=4, tree_top_k=2, tree_max_nodes=8).generate(prompt, 40, eos_token_id=eos)
    assert got.tokens == want


def test_drafter_extend_equals_a_full_recomputation():
    """DeviceDrafter.draft_logits_extend (the previous context's K/V rows kept in
    the drafter's cache, only the new rows and the query slots run) returns the
    logits of draft_logits over the whole context, bit for bit on the fp32
    model, for contexts that grow by 1 and 3 rows and stay the same."""
    tm, dr = _tiny()
    V, F = tm.shape.vocab, dr.feat_dim
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, V, (40,), generator=g).to(DEV)
    feats = torch.randn(40, F, generator=g).to(tm.dtype).to(DEV)
    want = {n: dr.draft_logits(ids[:n], feats[:n], 4).clone() for n in (20, 21, 24)}
    dr.draft_logits(ids[:20], feats[:20], 4)
    for n in (21, 24, 24):
        got = dr.draft_logits_extend(ids[:n], feats[:n], 4)
        assert torch.equal(got, want[n]), n


class RecordingDrafter:
    """Passes draft_logits_extend through to ``inner`` and checks every call
    against a second drafter with the same weights that recomputes the whole
    context (draft_logits)."""

    def __init__(self, inner, fresh):
        self.inner, self.fresh, self.calls = inner, fresh, 0

    def reset(self):
        self.inner.reset()

    def draft_logits(self, ctx, feats, k):
        return self.inner.draft_logits(ctx, feats, k)

    def draft_logits_extend(self, ctx, feats, k):
        got = self.inner.draft_logits_extend(ctx, feats, k)
        want = self.fresh.draft_logits(ctx, feats, k)
        assert torch.equal(got, want), f"call {self.calls}: the drafter reused another context's rows"
        self.calls += 1
        return got


def test_a_second_prompt_does_not_reuse_the_first_prompts_drafter_rows():
    """Two generate() calls on one DeviceDrafter with different prompts: every
    draft of the second call equals a full recomputation of its context (the
    loop resets the drafter's cached rows at the start of a call)."""
    tm, dr = _tiny()
    w, _ = _drafter_weights(TINY_LLAMA, 2, len(tm.feature_layers), torch.float32, seed=5, std=0.05)
    fresh = DeviceDrafter(tm, w, max_depth=5, capacity=256)
    rec = RecordingDrafter(dr, fresh)
    dec = SpeculativeDecoder(tm, rec, k=4, tree_top_k=2, tree_max_nodes=8)
    a = dec.generate([3, 1, 4, 1, 5, 9, 2, 6, 5, 3], 12)
    b = dec.generate([2, 7, 1, 8], 12)
    assert a.tokens == greedy_decode(tm, [3, 1, 4, 1, 5, 9, 2, 6, 5, 3], 12).tokens
    assert b.tokens == greedy_decode(tm, [2, 7, 1, 8], 12).tokens
    assert rec.calls >= 4


def _near_tie_or_equal(tm, prompt, ref_tokens, got_tokens, bound=0.0625):
    """``got`` equals greedy decoding, or first differs at a step whose greedy
    top-1 / top-2 margin is at most ``bound`` (a bf16 rounding of a different
    row block flips a near tie)."""
    if got_tokens == ref_tokens:
        return "equal"
    j = next(i for i, (a, b) in enumerate(zip(got_tokens, ref_tokens)) if a != b)
    lg = tm.forward(torch.tensor([prompt + ref_tokens[:j]])).logits[0, -1].float()
    top = lg.topk(2).values
    margin = float(top[0] - top[1])
    assert margin <= bound, f"token {j} differs with a greedy margin of {margin:.4g}"
    return f"near tie at token {j} (margin {margin:.3g})"


@pytest.mark.parametrize("tree_top_k,tree_max_nodes", [(4, 26), (20, 100)], ids=["26-nodes", "100-nodes"])
def test_speculative_loop_at_the_7b_width_bf16(tree_top_k, tree_max_nodes):
    """Two 7B-width NF4 layers in bf16, recorded steps with P read on the device.
    The tree pass and the one-token pass that greedy decoding uses compute the
    same logits in different row blocks, so a bf16 rounding can flip a near
    tie; every token must match up to the first such step, and that step's
    greedy top-1 / top-2 margin must be small. The recorded steps emit exactly
    the tokens of the same kernels launched each step with P from the host."""
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    tm = TargetModel.synthetic(shape, seed=4, device=DEV, norm_noise=0.1, cache_capacity=512)
    w, _ = _drafter_weights(shape, 1, 3, torch.bfloat16, seed=6, std=shape.init_std)
    dr = DeviceDrafter(tm, w, max_depth=5, capacity=512)
    prompt = list(range(100, 140))
    n = 64
    ref = greedy_decode(tm, prompt, n)
    graph = SpeculativeDecoder(tm, PeekingDrafter(dr, prompt + ref.tokens, 0.8, seed=3), k=5, tree_top_k=tree_top_k,
                               tree_max_nodes=tree_max_nodes)
    assert graph.device_prefix
    res = graph.generate(prompt, n)
    eager = SpeculativeDecoder(tm, PeekingDrafter(dr, prompt + ref.tokens, 0.8, seed=3), k=5, tree_top_k=tree_top_k,
                               tree_max_nodes=tree_max_nodes, use_graphs=False).generate(prompt, n)
    assert res.tokens == eager.tokens  # one key split either way at these lengths: the same roundings
    assert res.steps <= res.host_reads <= res.steps + 1
    verdict = _near_tie_or_equal(tm, prompt, ref.tokens, res.tokens)
    print(f"7B width, {tree_max_nodes} nodes: tokens per step {res.tokens_per_step:.2f}, steps {res.steps}, {verdict}")
    # an untrained drafter: every step misses and runs the one-token pass
    miss = SpeculativeDecoder(tm, dr, k=5, tree_top_k=tree_top_k, tree_max_nodes=tree_max_nodes).generate(prompt, 24)
    print("miss path:", _near_tie_or_equal(tm, prompt, ref.tokens[:24], miss.tokens))


# ------------------------------------------------------------------ the shared modules
def test_shared_modules_are_callable_and_match_the_oracle():
    shape = LLAMA2_7B_NF4.reduced(1, feature_layers=(1, 1, 1))
    tm = TargetModel.synthetic(shape, seed=2, device=DEV, keep_logical=True, norm_noise=0.1)
    hw = tm.model.host_weights()
    emb, head, norm = tm.get_input_embeddings(), tm.get_lm_head(), tm.get_final_norm()
    ids = torch.tensor([[5, 31999, 0], [7, 7, 123]])
    assert torch.equal(emb(ids.to(DEV)).cpu(), hw["embed"][ids])
    gen = torch.Generator().manual_seed(2)
    x = (torch.randn(2, 3, shape.hidden, generator=gen) * 2).to(torch.bfloat16)
    got = norm(x.to(DEV)).cpu()
    want = rms_norm(x, hw["final_norm"], shape.rms_eps)
    assert (got == want).float().mean() > 0.999
    assert torch.all((got.float() - want.float()).abs() <= 2 ** -7 * want.float().abs())
    h = want.to(DEV)
    lg = head(h).cpu().float()
    assert lg.shape == (2, 3, shape.vocab)
    ref = want.float() @ hw["lm_head"].float().t()
    assert torch.all((lg - ref).abs() <= 2e-2 + 2e-2 * ref.abs())
    with pytest.raises(Exception):
        emb(torch.tensor([shape.vocab]).to(DEV))  # outside the vocabulary


class RefShapedDrafter(torch.nn.Module):
    """A drafter built the way the reference's ParallelDrafter is (src/pe/drafter.py:
    36-83,120-160,195-236): its own layers in torch, the target's embed, lm_head
    and final norm kept in tuples and only called. Its layers follow nn.py in
    fp32 (rms norm, RoPE, softmax attention with an additive bias, SwiGLU)."""

    def __init__(self, target, w):
        super().__init__()
        self.w = w
        s = target.shape
        self.s = s
        self._embed = (target.get_input_embeddings(),)
        self._lm_head = (target.get_lm_head(),)
        self._final_norm = (target.get_final_norm(),)

    def real_input(self, ids, feats):
        H = self.s.hidden
        emb = self._embed[0](ids).float()
        f = od.drafter_rms_norm(feats.float().unflatten(-1, (-1, H)), self.w["feat_norm"], self.s.rms_eps)
        feat = f.flatten(-2) @ self.w["feat_proj"].t()
        return torch.cat([emb, feat], -1) @ self.w["in_proj"].t()

    def draft_logits(self, ids, feats, k):
        s, w = self.s, self.w
        p = ids.numel()
        m = p + k - 1
        x = torch.empty(m, s.hidden, device=ids.device)
        x[:p] = self.real_input(ids, feats)
        mask_vec = torch.cat([w["mask_emb"], w["h_shared"]]) @ w["in_proj"].t()
        x[p:] = mask_vec
        pos = od.draft_positions(p, k).to(ids.device).float()
        bias = torch.zeros(m, m, device=ids.device).masked_fill_(~od.draft_allow_mask(p, k).to(ids.device), -1e30)
        inv = 1.0 / (s.rope_theta ** (torch.arange(0, s.head_dim, 2, device=ids.device).float() / s.head_dim))
        ang = pos[:, None] * inv[None, :]
        cos, sin = torch.cat([ang, ang], -1).cos(), torch.cat([ang, ang], -1).sin()

        def rope(t):  # t: (heads, m, hd)
            half = t.shape[-1] // 2
            return t * cos + torch.cat([-t[..., half:], t[..., :half]], -1) * sin

        for lw in w["layers"]:
            h = od.drafter_rms_norm(x, lw["attn_norm"], s.rms_eps)
            q = rope((h @ lw["q"].t()).view(m, s.num_heads, s.head_dim).transpose(0, 1))
            kk = rope((h @ lw["k"].t()).view(m, s.num_kv_heads, s.head_dim).transpose(0, 1))
            vv = (h @ lw["v"].t()).view(m, s.num_kv_heads, s.head_dim).transpose(0, 1)
            g = s.num_heads // s.num_kv_heads
            kk, vv = kk.repeat_interleave(g, 0), vv.repeat_interleave(g, 0)
            att = torch.softmax(q @ kk.transpose(-1, -2) / s.head_dim ** 0.5 + bias, -1) @ vv
            x = x + att.transpose(0, 1).reshape(m, -1) @ lw["o"].t()
            h = od.drafter_rms_norm(x, lw["mlp_norm"], s.rms_eps)
            x = x + (torch.nn.functional.silu(h @ lw["gate"].t()) * (h @ lw["up"].t())) @ lw["down"].t()
        hidden = self._final_norm[0](x)
        idx = [p - 1] + list(range(p, m))
        return self._lm_head[0](hidden)[idx]


def test_a_reference_shaped_drafter_runs_on_the_shared_modules():
    """On the tiny fp32 target: the reference-shaped drafter (torch layers on the
    GPU, the target's modules called through the accessors) gives the oracle's
    draft logits, and so does the device drafter."""
    tm = TargetModel.synthetic(TINY_LLAMA, seed=3, device=DEV, keep_logical=True, norm_noise=0.1)
    hw = tm.model.host_weights()
    w, _ = _drafter_weights(TINY_LLAMA, 2, len(tm.feature_layers), torch.float32, seed=8, std=0.05)
    shared = {"embed": hw["embed"], "final_norm": hw["final_norm"], "lm_head": hw["lm_head"]}
    gen = torch.Generator().manual_seed(8)
    ids = torch.randint(0, TINY_LLAMA.vocab, (30,), generator=gen)
    feats = torch.randn(30, tm.feature_dim, generator=gen)
    want = od.OracleDrafter(TINY_LLAMA, w, shared, torch.float32).draft_logits(ids, feats, 5)
    wd = {k: (v.to(DEV) if torch.is_tensor(v) else [{a: b.to(DEV) for a, b in x.items()} for x in v])
          for k, v in w.items()}
    got = RefShapedDrafter(tm, wd).draft_logits(ids.to(DEV), feats.to(DEV), 5).cpu()
    assert torch.allclose(got, want, rtol=1e-4, atol=1e-4), float((got - want).abs().max())
    dev = DeviceDrafter(tm, w, max_depth=5, capacity=64).draft_logits(ids.to(DEV), feats.to(DEV), 5).cpu()
    assert torch.allclose(dev, want, rtol=1e-4, atol=1e-4), float((dev - want).abs().max())
    _ = ops  # the modules launch the library's kernels (pe_embed, pe_rmsnorm, pe_dense_gemm)
