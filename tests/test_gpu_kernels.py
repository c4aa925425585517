"""Kernel-level parity on the GPU: every HIP kernel against the CPU oracle.

Integer / byte / index work is compared bit for bit; floating-point kernels
within the stated tolerance (fp32 1e-4, bf16/fp16 2e-2 on values of O(1)).
"""

import numpy as np
import pytest
import torch

from oracle import masks as om
from oracle import nf4 as onf4
from oracle import verify as ov
from parallel_eagle_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _status():
    return torch.zeros(4, dtype=torch.int32, device=DEV)


# ------------------------------------------------------------------ RNG
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fill_normal_bit_exact_with_host_generator(dtype):
    n = 100_003
    out = ops.fill_normal(torch.empty(n, dtype=dtype, device=DEV), seed=11, stream_id=77, std=0.02)
    ref = torch.from_numpy(synth.normal(11, 77, n, 0.02)).to(dtype)
    assert torch.equal(out.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if dtype != torch.float32 else torch.int32))


def test_fill_uniform_int_bit_exact():
    out = ops.fill_uniform_int(torch.empty(5000, dtype=torch.int64, device=DEV), 32000, 3, 9)
    assert np.array_equal(out.cpu().numpy(), synth.uniform_int(3, 9, 5000, 32000))


# ------------------------------------------------------------------ NF4
def test_nf4_quantize_bit_exact():
    w = torch.from_numpy(synth.normal(5, 123, 96 * 256, 0.02).reshape(96, 256))
    p, a = ops.nf4_quantize(w.to(DEV))
    rp, ra = onf4.quantize(w.numpy())
    assert np.array_equal(p.cpu().numpy(), rp)
    assert np.array_equal(a.cpu().numpy().view(np.uint16), ra.view(np.uint16))


@pytest.mark.parametrize("n,k", [(32, 128), (96, 384), (4096 // 8, 1024)])
def test_nf4_repack_dequant_bit_exact(n, k):
    w = synth.normal(8, 5, n * k, 0.02).reshape(n, k)
    rp, ra = onf4.quantize(w)
    tiled, tabs = ops.nf4_repack(torch.from_numpy(rp).to(DEV), torch.from_numpy(ra).to(DEV))
    deq = ops.nf4_dequant(tiled, tabs, n, k)
    ref = onf4.dequantize(rp, ra)
    assert np.array_equal(deq.cpu().view(torch.int16).numpy().view(np.uint16), ref)


# ------------------------------------------------------------------ GEMMs
def _nf4_weight(n, k, seed):
    w = synth.normal(seed, 31, n * k, 0.02).reshape(n, k)
    p, a = onf4.quantize(w)
    tiled, tabs = ops.nf4_repack(torch.from_numpy(p).to(DEV), torch.from_numpy(a).to(DEV))
    wdq = onf4.dequantize_torch(p, a)  # bf16 [N][K]
    return (tiled, tabs), wdq


@pytest.mark.parametrize("m", [1, 26, 33, 64, 130])
@pytest.mark.parametrize("n,k", [(256, 1024), (4096, 512), (96, 4096)])
def test_nf4_linear_matches_dequant_then_linear(m, n, k):
    (tiled, tabs), wdq = _nf4_weight(n, k, seed=m + n)
    x = torch.from_numpy(synth.normal(m, 32, m * k, 1.0).reshape(m, k)).to(torch.bfloat16)
    y = ops.linear(x.to(DEV), n, nf4=(tiled, tabs)).cpu()
    ref32 = x.float() @ wdq.float().t()  # fp32 product of the exact dequantised operands
    ref = torch.nn.functional.linear(x, wdq)  # the reference's bf16 path on CPU
    assert torch.allclose(y.float(), ref32, rtol=1e-2, atol=1e-2), (y.float() - ref32).abs().max()
    assert torch.allclose(y.float(), ref.float(), rtol=2e-2, atol=2e-2)


def test_nf4_linear_deterministic_and_batch_invariant():
    n, k = 4096, 4096
    (tiled, tabs), _ = _nf4_weight(n, k, seed=3)
    x = torch.from_numpy(synth.normal(4, 33, 26 * k, 1.0).reshape(26, k)).to(torch.bfloat16).to(DEV)
    y1 = ops.linear(x, n, nf4=(tiled, tabs))
    y2 = ops.linear(x, n, nf4=(tiled, tabs))
    y_row = ops.linear(x[5:6].contiguous(), n, nf4=(tiled, tabs))
    assert torch.equal(y1, y2)
    assert torch.equal(y1[5:6], y_row)


@pytest.mark.parametrize("m", [26, 40])
@pytest.mark.parametrize("epi", ["store", "residual", "swiglu", "swiglu-tiled-out"])
def test_nf4_linear_tiled_x_equals_row_major(m, epi):
    """pe_nf4_gemm_tiled (A-tiled X, optionally A-tiled output) runs the same
    kernels on the same values as pe_nf4_gemm: results are bit-identical."""
    n, k = 1024, 2048
    (tiled, tabs), _ = _nf4_weight(n, k, seed=7 + m)
    x = torch.from_numpy(synth.normal(m, 34, m * k, 1.0).reshape(m, k)).to(torch.bfloat16).to(DEV)
    code = {"store": _lib.PE_EPI_STORE, "residual": _lib.PE_EPI_RESIDUAL}.get(epi, _lib.PE_EPI_SWIGLU)
    n_out = n // 2 if code == _lib.PE_EPI_SWIGLU else n
    resid = (torch.from_numpy(synth.normal(m, 35, m * n_out, 1.0).reshape(m, n_out)).to(torch.bfloat16).to(DEV)
             if code == _lib.PE_EPI_RESIDUAL else None)
    ref = ops.linear(x, n, nf4=(tiled, tabs), epilogue=code, resid=resid)
    xt = ops.to_xtile(x)
    if epi == "swiglu-tiled-out":
        got = ops.from_xtile(ops.linear_tiled(xt, m, k, n, (tiled, tabs), epilogue=code, out_tiled=True), m, n_out)
    else:
        got = ops.linear_tiled(xt, m, k, n, (tiled, tabs), epilogue=code, resid=resid)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("m", [1, 26, 32, 48, 64])
@pytest.mark.parametrize("n,k", [(12288, 4096), (8192, 1024), (16384, 512), (22016, 4096), (20480, 1024),
                                 (24576, 2560)])
def test_nf4_tiled_unsplit_wide_workgroups(m, n, k):
    """Unsplit launches with 128..256 column groups run eight waves per
    workgroup (two table regions); with 256..512 groups one whole group per CU
    plus the rest in two K splits joined by the last workgroup (K = 2560: ten
    units per split, uneven over the four waves). Either way the
    stored bf16 product equals the fp32 product of the exact dequantised
    operands up to bf16 rounding of the output and fp32 accumulation order."""
    (tiled, tabs), wdq = _nf4_weight(n, k, seed=m + n + k + 1)
    x = torch.from_numpy(synth.normal(m, 37, m * k, 1.0).reshape(m, k)).to(torch.bfloat16)
    got = ops.linear_tiled(ops.to_xtile(x.to(DEV)), m, k, n, (tiled, tabs)).cpu().float()
    ref32 = x.float() @ wdq.float().t()
    err = (got - ref32).abs()
    assert torch.all(err <= 2.0 ** -8 * ref32.abs() + 1e-4 * (1 + ref32.abs()) * (k / 1024)), err.max()


@pytest.mark.parametrize("m", [1, 26, 33, 64])
@pytest.mark.parametrize("n,k,tiled", [(4096, 4096, True), (22016, 4096, True), (4096, 11008, True),
                                       (256, 1024, False)])
def test_nf4_partials_sum_to_the_product(m, n, k, tiled):
    """pe_nf4_gemm_partials: the split partials, summed in split order in fp32,
    equal the fp32 product of the exact dequantised operands up to fp32
    accumulation order (every split sums the same bf16 products)."""
    (tiled_w, tabs), wdq = _nf4_weight(n, k, seed=m + n + k)
    x = torch.from_numpy(synth.normal(m, 36, m * k, 1.0).reshape(m, k)).to(torch.bfloat16)
    xd = ops.to_xtile(x.to(DEV)) if tiled else x.to(DEV)
    parts, s = ops.nf4_linear_partials(xd, m, k, n, (tiled_w, tabs), x_tiled=tiled)
    assert 1 <= s <= 16 and parts.shape == (s, m, n)
    tot = parts[0].clone()
    for i in range(1, s):
        tot += parts[i]
    ref32 = x.float() @ wdq.float().t()
    err = (tot.cpu() - ref32).abs()
    assert torch.all(err <= 1e-4 * (1 + ref32.abs()) * (k / 1024)), err.max()


@pytest.mark.parametrize("m,n,k", [(208, 27648, 5120), (97, 22016, 4096), (130, 5120, 4096), (65, 22016, 4096),
                                   (161, 22016, 4096), (150, 22016, 4096), (256, 22016, 4096)])
def test_many_row_swiglu_equals_the_swiglu_of_the_split_partials(m, n, k):
    """pe_nf4_gemm_tiled with 64 < M <= 256 rows and the SwiGLU epilogue (the
    batched pass's gate/up linear) against the SwiGLU of the same kernel's fp32
    split partials, summed in split order on the host with the rounding points
    of HF LlamaMLP (modeling_llama.py:174-176 in the dtype: gate and up rounded,
    act(gate) rounded, the product rounded). The first two shapes plan one K
    split, so the kernel stores the A-tiled activation itself; the third splits
    K and takes the partials + SwiGLU kernel. Every element is equal or one
    bf16 step apart (the device's expf and torch's exp may differ in the last
    fp32 bit), at most 0.1% of them one step apart: a wrong row, column or
    gate/up pairing would miss by far more."""
    (tiled_w, tabs), _ = _nf4_weight(n, k, seed=m + n + k + 5)
    x = torch.from_numpy(synth.normal(m, 38, m * k, 1.0).reshape(m, k)).to(torch.bfloat16)
    xt = ops.to_xtile(x.to(DEV))
    act = ops.from_xtile(ops.linear_tiled(xt, m, k, n, (tiled_w, tabs), epilogue=_lib.PE_EPI_SWIGLU,
                                          out_tiled=True), m, n // 2).cpu()
    parts, s = ops.nf4_linear_partials(xt, m, k, n, (tiled_w, tabs), x_tiled=True)
    tot = parts[0].clone()
    for i in range(1, s):
        tot += parts[i]
    gu = tot.cpu().view(m, n // 64, 2, 32)  # each 64-column group: 32 gate, then 32 up columns
    g = gu[:, :, 0, :].reshape(m, n // 2).to(torch.bfloat16).float()
    u = gu[:, :, 1, :].reshape(m, n // 2).to(torch.bfloat16).float()
    act_g = (g / (1.0 + torch.exp(-g))).to(torch.bfloat16).float()
    ref = (act_g * u).to(torch.bfloat16)
    steps = (act.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(steps.max()) <= 1, int(steps.max())
    assert int((steps == 1).sum()) <= m * (n // 2) // 1000, int((steps == 1).sum())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("epi", ["store", "bias", "residual", "swiglu"])
def test_dense_linear_epilogues(dtype, epi):
    m, n, k = 26, 512, 1024
    w = torch.from_numpy(synth.normal(1, 40, n * k, 0.02).reshape(n, k)).to(dtype)
    x = torch.from_numpy(synth.normal(2, 41, m * k, 1.0).reshape(m, k)).to(dtype)
    wt = ops.dense_repack(w.to(DEV))
    bias = torch.from_numpy(synth.normal(3, 42, n, 0.1)).to(dtype)
    resid = torch.from_numpy(synth.normal(4, 43, m * n, 1.0).reshape(m, n)).to(dtype)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    lin = torch.nn.functional.linear
    if epi == "store":
        y = ops.linear(x.to(DEV), n, dense=wt).cpu()
        ref = lin(x, w)
    elif epi == "bias":
        y = ops.linear(x.to(DEV), n, dense=wt, bias=bias.to(DEV)).cpu()
        ref = lin(x, w, bias)
    elif epi == "residual":
        y = ops.linear(x.to(DEV), n, dense=wt, epilogue=_lib.PE_EPI_RESIDUAL, resid=resid.to(DEV)).cpu()
        ref = resid + lin(x, w)
    else:
        # gate/up interleaved by 32 rows
        g, u = w[: n // 2], w[n // 2:]
        inter = torch.stack([g.view(-1, 32, k), u.view(-1, 32, k)], 1).reshape(n, k).contiguous()
        y = ops.linear(x.to(DEV), n, dense=ops.dense_repack(inter.to(DEV)), epilogue=_lib.PE_EPI_SWIGLU).cpu()
        ref = torch.nn.functional.silu(lin(x, g)) * lin(x, u)
    assert torch.allclose(y.float(), ref.float(), rtol=tol, atol=tol), (y.float() - ref.float()).abs().max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k,n", [(300, 1024, 512), (513, 1152, 768), (2047, 4096, 4096),
                                   (2048, 1024, 16384), (1025, 512, 26624)])
def test_dense_linear_over_many_rows(dtype, m, k, n):
    """pe_dense_gemm over more than 256 rows (prefill and drafter-context
    linears: 128-column workgroups, or, from 512 tiles on, 256 x 256 tiles with
    both operands through an LDS ring; last row blocks partly filled) against
    the fp32 product rounded once: outputs of
    at least 1e-3 of the largest within one step of the dtype, at most 0.5% of
    them one step away (another fp32 summation order alone moves 0.15% of fp16
    outputs by a step); every output within 1e-5 of the largest (near zero a
    step of fp16 is far below the summation-order noise of fp32)."""
    w = torch.from_numpy(synth.normal(5, 44, n * k, 0.02).reshape(n, k)).to(dtype)
    x = torch.from_numpy(synth.normal(6, 45, m * k, 1.0).reshape(m, k)).to(dtype)
    y = ops.linear(x.to(DEV), n, dense=ops.dense_repack(w.to(DEV))).cpu()
    r32 = x.float() @ w.float().t()
    ref = r32.to(dtype)
    top = float(r32.abs().max())
    big = r32.abs() >= 1e-3 * top
    steps = (y.view(torch.int16).int() - ref.view(torch.int16).int()).abs()[big]
    assert int(steps.max()) <= 1, int(steps.max())
    assert int((steps == 1).sum()) <= m * n // 200, int((steps == 1).sum())
    assert float((y.float() - r32).abs().max()) <= 1e-5 * top + float((ref.float() - r32).abs().max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [26, 40])
def test_dense_swiglu_at_the_14b_shape(dtype, m):
    """The dense gate/up at the Qwen2.5-14B shape (K = 5120, 2 x 13824 columns:
    432 column groups, between one and two per CU, one unsplit launch).
    Every column against the fp32 product with HF LlamaMLP's rounding points
    (modeling_llama.py:174-176: gate and up rounded, silu rounded, the product
    rounded) within a few 16-bit ulps, and equal for almost every column."""
    n, k = 2 * 13824, 5120
    w = torch.from_numpy(synth.normal(5, 44, n * k, 0.02).reshape(n, k)).to(dtype)
    x = torch.from_numpy(synth.normal(6, 45, m * k, 1.0).reshape(m, k)).to(dtype)
    g, u = w[: n // 2], w[n // 2:]
    inter = torch.stack([g.view(-1, 32, k), u.view(-1, 32, k)], 1).reshape(n, k).contiguous()
    y = ops.linear(x.to(DEV), n, dense=ops.dense_repack(inter.to(DEV)), epilogue=_lib.PE_EPI_SWIGLU).cpu().float()
    gf = (x.float() @ g.float().t()).to(dtype)
    uf = (x.float() @ u.float().t()).to(dtype)
    ref = (torch.nn.functional.silu(gf.float()).to(dtype).float() * uf.float()).to(dtype).float()
    err = (y - ref).abs()
    # the fp32 accumulation order may move a rounding of gate or up by one
    # 16-bit ulp, which moves the output by a few ulps of itself at most
    assert torch.all(err <= 4 * torch.finfo(dtype).eps * ref.abs() + 1e-3), err.max()
    assert float((err > 0).float().mean()) < 0.02


# ------------------------------------------------------------------ masks
TREES = [
    [-1, 0, -1],
    [-1, -1, 0, 0, 1, 2, 2, 5],
    [-1] + list(range(0, 63)),  # chain of 64
    [-1, -1, -1, -1] + [i % 4 for i in range(22)],
]


@pytest.mark.parametrize("parents", TREES)
@pytest.mark.parametrize("P", [0, 2, 37])
def test_tree_masks_match_oracle(parents, P):
    t = len(parents)
    words = (t + 63) // 64
    st = _status()
    bits, pos, dep = ops.tree_masks(torch.tensor(parents, dtype=torch.int32, device=DEV), P, words, st)
    assert int(st[0]) == 0
    ref_bits = om.ancestor_bits(parents)
    got = bits.cpu().numpy().view(np.uint64)
    for i in range(t):
        val = sum(int(got[i, w]) << (64 * w) for w in range(words))
        assert val == ref_bits[i]
    assert pos.cpu().tolist() == om.tree_position_ids(parents, P)[P:]
    assert dep.cpu().tolist() == om.tree_depths(parents)
    allow = ops.tree_allow_dense(bits, P).cpu().numpy()
    assert np.array_equal(allow, om.tree_allow_mask(parents, P))


def test_tree_masks_reject_non_topological():
    st = _status()
    ops.tree_masks(torch.tensor([-1, 2, 0], dtype=torch.int32, device=DEV), 4, 1, st)
    assert int(st[0]) & _lib.PE_ERR_TREE


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_bias_to_bits_round_trip(dtype):
    parents, P = TREES[1], 5
    allow = om.tree_allow_mask(parents, P)[P:, :]
    bias = om.to_additive_bias(allow, dtype)[0, 0].to(DEV).contiguous()
    st = _status()
    bits = ops.bias_to_bits(bias, P, 1, st)
    assert int(st[0]) == 0
    assert bits.cpu().numpy().view(np.uint64)[:, 0].tolist() == om.ancestor_bits(parents)
    bad = bias.clone()
    bad[2, 1] = torch.finfo(dtype).min  # masks a prefix column: not a tree mask
    ops.bias_to_bits(bad, P, 1, st)
    assert int(st[0]) & _lib.PE_ERR_MASK


# ------------------------------------------------------------------ attention
def _attn_ref(q, k, v, P, parents, causal, scale, dtype):
    """q [T][nh][hd], k/v [nkv][S][hd] -> [T][nh*hd] via the oracle's SDPA path."""
    T, nh, hd = q.shape
    nkv, S, _ = k.shape
    if causal:
        allow = torch.arange(T)[:, None] + P >= torch.arange(S)[None, :]
    else:
        allow = torch.from_numpy(om.tree_allow_mask(parents, P)[P:, :])
    bias = om.to_additive_bias(allow.numpy(), dtype)
    from oracle.model import repeat_kv

    qq = q.permute(1, 0, 2).unsqueeze(0)
    kk = repeat_kv(k.unsqueeze(0), nh // nkv)
    vv = repeat_kv(v.unsqueeze(0), nh // nkv)
    o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=bias, scale=scale)
    return o[0].permute(1, 0, 2).reshape(T, nh * hd)


@pytest.mark.parametrize("dtype,hd", [(torch.bfloat16, 128), (torch.float16, 128), (torch.float32, 64)])
@pytest.mark.parametrize("nh,nkv", [(4, 4), (10, 2)])
@pytest.mark.parametrize("P,parents,causal", [
    (0, [-1, -1, 0, 0, 1, 2, 2, 5], False),
    (77, TREES[3], False),
    (300, [-1, 0, 1, 2, 3], False),
    (50, None, True),
])
def test_tree_attention_matches_sdpa(dtype, hd, nh, nkv, P, parents, causal):
    T = 6 if causal else len(parents)
    S = P + T
    cap = S + 3
    q = torch.from_numpy(synth.normal(1, 50, T * nh * hd).reshape(T, nh, hd)).to(dtype)
    k = torch.from_numpy(synth.normal(2, 51, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    v = torch.from_numpy(synth.normal(3, 52, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    kc = torch.zeros((nkv, cap, hd), dtype=dtype)
    vc = torch.zeros((nkv, cap, hd), dtype=dtype)
    kc[:, :S], vc[:, :S] = k, v
    scale = hd ** -0.5
    if causal:
        bits, mode = None, _lib.PE_MASK_CAUSAL
    else:
        st = _status()
        bits, _, _ = ops.tree_masks(torch.tensor(parents, dtype=torch.int32, device=DEV), P, (T + 63) // 64, st)
        mode = _lib.PE_MASK_TREE
    out = ops.tree_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), P, mode, bits, scale).cpu()
    ref = _attn_ref(q, k, v, P, parents, causal, scale, dtype)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert torch.allclose(out.float(), ref.float(), rtol=tol, atol=tol), (out.float() - ref.float()).abs().max()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("nh,nkv,T,P", [
    (4, 4, 64, 2000),   # two row tiles, key splits; the last split holds node keys only
    (10, 2, 26, 1000),  # five row tiles per KV head, the last with two rows
    (2, 1, 26, 5000),   # two row tiles in 16 key splits
    (8, 8, 40, 0),      # node keys only, one split, the second tile 8 rows
    (32, 32, 26, 2047),  # the 7B shape: eight key splits per head, a multiple of eight KV heads
    (16, 8, 40, 3000),  # eight KV heads, two row tiles of grouped rows in key splits
])
def test_multi_tile_attention_with_key_splits_matches_sdpa(dtype, nh, nkv, T, P):
    """Tree attention over more than 32 query rows per KV head (several row
    tiles, split keys combined by the last workgroup to arrive): against SDPA
    with the reference's additive tree bias; a call repeated on the same
    workspace after a causal call (the same arrival counters) is equal."""
    hd = 128
    rng = np.random.default_rng(1000 * T + P)
    parents = [-1] + [int(rng.integers(-1, t)) for t in range(1, T)]
    S = P + T
    cap = S + 5
    q = torch.from_numpy(synth.normal(4, 60, T * nh * hd).reshape(T, nh, hd)).to(dtype)
    k = torch.from_numpy(synth.normal(5, 61, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    v = torch.from_numpy(synth.normal(6, 62, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    kc = torch.zeros((nkv, cap, hd), dtype=dtype)
    vc = torch.zeros((nkv, cap, hd), dtype=dtype)
    kc[:, :S], vc[:, :S] = k, v
    qd, kd, vd = q.to(DEV), kc.to(DEV), vc.to(DEV)
    scale = hd ** -0.5
    st = _status()
    bits, _, _ = ops.tree_masks(torch.tensor(parents, dtype=torch.int32, device=DEV), P, (T + 63) // 64, st)
    need = int(ops.lib().pe_attention_workspace_bytes(T, nh, nkv, hd, S, ops.dcode(dtype)))
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = ops.tree_attention(qd, kd, vd, P, _lib.PE_MASK_TREE, bits, scale, workspace=ws).cpu()
    causal = ops.tree_attention(qd, kd, vd, P, _lib.PE_MASK_CAUSAL, None, scale, workspace=ws).cpu()
    again = ops.tree_attention(qd, kd, vd, P, _lib.PE_MASK_TREE, bits, scale, workspace=ws).cpu()
    assert torch.equal(out, again)
    ref = _attn_ref(q, k, v, P, parents, False, scale, dtype)
    assert torch.allclose(out.float(), ref.float(), rtol=2e-2, atol=2e-2), (out.float() - ref.float()).abs().max()
    r32 = _attn_ref(q.float(), k.float(), v.float(), P, parents, False, scale, torch.float32)
    for h in range(nh):  # per query head: as close to fp32 as torch's own reduced-precision SDPA
        cols = slice(h * hd, (h + 1) * hd)
        n32 = r32[:, cols].norm()
        e_dev = float((out[:, cols].float() - r32[:, cols]).norm() / n32)
        e_ref = float((ref[:, cols].float() - r32[:, cols]).norm() / n32)
        assert e_dev <= 2 * e_ref + 1e-3, (h, e_dev, e_ref)
    ref_c = _attn_ref(q, k, v, P, None, True, scale, dtype)
    assert torch.allclose(causal.float(), ref_c.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype,nh,nkv,T,P", [
    (torch.bfloat16, 4, 4, 2048, 0),    # a prefill from an empty cache: 16 row blocks, 8 balanced pairs
    (torch.float16, 10, 2, 300, 77),    # GQA rows (node, query head), 12 row blocks, after a prefix
    (torch.bfloat16, 2, 2, 320, 5),     # 3 row blocks: the middle block is a pair of its own
    (torch.bfloat16, 4, 1, 257, 1000),  # four query heads per KV head, a long prefix, a ragged last tile
])
def test_causal_attention_over_many_rows_matches_sdpa(dtype, nh, nkv, T, P):
    """Causal passes of 256 nodes or more (prompt prefills) run attn_rows_kernel:
    against SDPA with the reference's causal additive bias, every element within
    2e-2; cache rows past P + T hold NaN, which no output may see."""
    hd = 128
    S = P + T
    cap = S + 70  # the last 64-key step reaches past the fill
    q = torch.from_numpy(synth.normal(7, 63, T * nh * hd).reshape(T, nh, hd)).to(dtype)
    k = torch.from_numpy(synth.normal(8, 64, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    v = torch.from_numpy(synth.normal(9, 65, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
    kc = torch.full((nkv, cap, hd), float("nan"), dtype=dtype)
    vc = torch.full((nkv, cap, hd), float("nan"), dtype=dtype)
    kc[:, :S], vc[:, :S] = k, v
    scale = hd ** -0.5
    out = ops.tree_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), P, _lib.PE_MASK_CAUSAL, None, scale).cpu()
    assert torch.isfinite(out.float()).all()
    ref = _attn_ref(q, k, v, P, None, True, scale, dtype)
    err = (out.float() - ref.float()).abs()
    assert torch.allclose(out.float(), ref.float(), rtol=2e-2, atol=2e-2), err.max()


BATCHED_ATTENTION_CASES = [
    # five query heads per KV head, 26-node trees: one wave per 32-row tile, 1-8 key splits per sequence
    (torch.bfloat16, 40, 8, [26] * 8, [812, 3000, 512, 4096, 1500, 700, 2222, 64]),
    (torch.float16, 40, 8, [26] * 3, [100, 513, 1024]),
    # ragged trees: 130, 35 and 200 rows per KV head (seven tiles, the short tree fills two), no prefix
    (torch.bfloat16, 40, 8, [26, 7, 40], [0, 900, 2500]),
    # one query head per KV head: two row tiles
    (torch.bfloat16, 4, 4, [26, 64], [100, 2048]),
]


def check_batched_attention(dtype, nh, nkv, trees, prefixes):
    """pe_tree_attention_batch against SDPA per sequence (its own prefix, tree
    bias and cache): for every (sequence, query head) the relative L2 distance
    from an fp32 evaluation is at most twice that of torch's own reduced-precision
    SDPA, plus 1e-3; every element within 2e-2. Cache rows past each sequence's
    fill hold NaN, which no output may see."""
    hd = 128
    B = len(trees)
    rng = np.random.default_rng(sum(prefixes) + len(trees))
    parents = [[-1] + [int(rng.integers(-1, t)) for t in range(1, T)] for T in trees]
    cap = max(p + t for p, t in zip(prefixes, trees)) + 70
    kc = torch.full((B, nkv, cap, hd), float("nan"), dtype=dtype)
    vc = torch.full((B, nkv, cap, hd), float("nan"), dtype=dtype)
    qs, ks, vs = [], [], []
    for b, (T, P) in enumerate(zip(trees, prefixes)):
        S = P + T
        q = torch.from_numpy(synth.normal(20 + b, 70, T * nh * hd).reshape(T, nh, hd)).to(dtype)
        k = torch.from_numpy(synth.normal(40 + b, 71, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
        v = torch.from_numpy(synth.normal(60 + b, 72, nkv * S * hd).reshape(nkv, S, hd)).to(dtype)
        kc[b, :, :S], vc[b, :, :S] = k, v
        qs.append(q)
        ks.append(k)
        vs.append(v)
    row0 = np.concatenate([[0], np.cumsum(trees)]).astype(np.int32)
    words = (max(trees) + 63) // 64
    bits = np.zeros((int(row0[-1]), words), dtype=np.uint64)
    for b, par in enumerate(parents):
        for t, a in enumerate(om.ancestor_bits(par)):
            for w in range(words):
                bits[row0[b] + t, w] = np.uint64((a >> (64 * w)) & ((1 << 64) - 1))
    scale = hd ** -0.5
    out = ops.tree_attention_batch(torch.cat(qs).to(DEV), kc.to(DEV), vc.to(DEV),
                                   torch.from_numpy(row0).to(DEV), torch.tensor(prefixes, dtype=torch.int64).to(DEV),
                                   torch.from_numpy(bits.view(np.int64)).to(DEV), scale, max(trees),
                                   max(prefixes)).cpu()
    assert torch.isfinite(out.float()).all()
    worst = []
    for b, (T, P) in enumerate(zip(trees, prefixes)):
        got = out[row0[b]: row0[b + 1]].float()
        ref = _attn_ref(qs[b], ks[b], vs[b], P, parents[b], False, scale, dtype).float()
        r32 = _attn_ref(qs[b].float(), ks[b].float(), vs[b].float(), P, parents[b], False, scale, torch.float32)
        assert torch.allclose(got, ref, rtol=2e-2, atol=2e-2), (b, (got - ref).abs().max())
        for h in range(nh):
            cols = slice(h * hd, (h + 1) * hd)
            n32 = r32[:, cols].norm()
            e_dev = float((got[:, cols] - r32[:, cols]).norm() / n32)
            e_ref = float((ref[:, cols] - r32[:, cols]).norm() / n32)
            worst.append((e_dev - 2 * e_ref, b, h, e_dev, e_ref))
    worst.sort(reverse=True)
    assert worst[0][0] <= 1e-3, f"(excess, sequence, head, device relL2, torch relL2): {worst[:4]}"


@pytest.mark.parametrize("dtype,nh,nkv,trees,prefixes", BATCHED_ATTENTION_CASES)
def test_batched_tree_attention_matches_sdpa_per_sequence(dtype, nh, nkv, trees, prefixes):
    """The default batched kernels (check_batched_attention)."""
    check_batched_attention(dtype, nh, nkv, trees, prefixes)


def test_batched_tree_attention_on_the_opt_in_rows_kernel():
    """The same cases with PE_ATTN_BATCH_ROWS=1 (attn_batch_rows_kernel and its
    split combine for four to eight row tiles per sequence and KV head). The
    switch is read once per process, so the cases run in one child process."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path[:0] = [{r!r}, {t!r}]\n"
            "import test_gpu_kernels as t\n"
            "for c in t.BATCHED_ATTENTION_CASES: t.check_batched_attention(*c)\n"
            "print('rows kernel cases passed')\n").format(r=root, t=os.path.join(root, "tests"))
    env = dict(os.environ, PE_ATTN_BATCH_ROWS="1")
    res = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
    assert "rows kernel cases passed" in res.stdout


# ------------------------------------------------------------------ acceptance and compaction
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("seed", range(6))
def test_accept_tree_matches_oracle(dtype, seed):
    rng = np.random.default_rng(seed)
    V, T = 50, 12
    parents = [-1]
    for t in range(1, T):
        parents.append(int(rng.integers(-1, t)))
    # coarse values so ties are common; plant matches along a random chain
    logits = torch.from_numpy(rng.integers(0, 4, size=(T + 1, V)).astype(np.float32)).to(dtype)
    tokens = [int(x) for x in rng.integers(0, V, size=T)]
    amax = [ov.first_argmax(logits[r]) for r in range(T + 1)]
    cur, row = -1, 0
    for _ in range(3):
        kids = [t for t in range(T) if parents[t] == cur]
        if not kids:
            break
        c = kids[int(rng.integers(0, len(kids)))]
        tokens[c] = amax[row]
        cur, row = c, 1 + c
    ref = ov.accept_tree_cached(logits[0], logits[1:], tokens, parents)
    out = ops.accept_tree(logits[0].to(DEV), logits[1:].to(DEV), torch.tensor(tokens, device=DEV),
                          torch.tensor(parents, dtype=torch.int32, device=DEV)).cpu().tolist()
    assert (out[2: 2 + out[0]], out[1]) == ref


@pytest.mark.parametrize("T", [0, 1, 70, 200])
def test_accept_tree_shared_scratch_and_wide_trees(T):
    """One scratch buffer across consecutive calls (its arrival counter must
    return to zero) on trees wider than one wave, so the walk's child search
    spans several ballots; each call matches the oracle walk."""
    rng = np.random.default_rng(T + 5)
    V = 40
    scratch = torch.zeros(T + 2, dtype=torch.int32, device=DEV)
    for call in range(3):
        parents = ([-1] + [int(rng.integers(-1, t)) for t in range(1, T)])[:T]
        logits = torch.from_numpy(rng.integers(0, 3, size=(T + 1, V)).astype(np.float32)).to(torch.bfloat16)
        tokens = [int(x) for x in rng.integers(0, V, size=T)]
        amax = [ov.first_argmax(logits[r]) for r in range(T + 1)]
        cur, row = -1, 0
        for _ in range(6):  # plant a chain, preferring late children (found by a later ballot)
            kids = [t for t in range(T) if parents[t] == cur]
            if not kids:
                break
            c = kids[-1]
            tokens[c] = amax[row]
            cur, row = c, 1 + c
        ref = ov.accept_tree_cached(logits[0], logits[1:], tokens, parents)
        nl = logits[1:].to(DEV) if T > 0 else logits[:1].to(DEV)
        out = ops.accept_tree(logits[0].to(DEV), nl, torch.tensor(tokens, dtype=torch.int64, device=DEV),
                              torch.tensor(parents, dtype=torch.int32, device=DEV), scratch=scratch).cpu().tolist()
        assert (out[2: 2 + out[0]], out[1]) == ref, (call, out[:8], ref)
        assert scratch[0].item() == 0  # the arrival counter (index 0) is back at zero


def test_argmax_rows_first_index_and_nan():
    x = torch.zeros((3, 1000), dtype=torch.float32)
    x[0, 7] = 5.0
    x[0, 900] = 5.0
    x[1, 300] = float("nan")
    x[1, 10] = float("nan")
    x[2, :] = -1.0
    got = ops.argmax_rows(x.to(DEV)).cpu().tolist()
    assert got == [7, 10, 0]


def _argmax_gemm(x, w_tiled, n, dtype):
    L = _lib.load()
    m, k = x.shape
    groups = int(L.pe_dense_gemm_argmax_groups(m, n, k))
    out = torch.empty((m, n), dtype=dtype, device=DEV)
    keys = torch.zeros((m, groups), dtype=torch.int64, device=DEV)
    wsb = int(L.pe_gemm_workspace_bytes(m, n, k, _lib.PE_WFMT_DENSE, ops.dcode(dtype), _lib.PE_EPI_STORE))
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    _lib.check(L.pe_dense_gemm_argmax(x.data_ptr(), k, m, k, w_tiled.data_ptr(), ops.dcode(dtype), n, out.data_ptr(),
                                      n, keys.data_ptr(), ws.data_ptr(), wsb, ops.stream_ptr()), "pe_dense_gemm_argmax")
    return out, keys, groups


def _tied_lm_head(n, k, dtype, m, seed):
    """Weights whose rows 5, 900 and n - 1 are identical and carry a feature X
    has at 10 in every row: those three columns tie exactly at (nearly always)
    the row's maximum."""
    g = torch.Generator().manual_seed(seed)
    w = 0.02 * torch.randn(n, k, generator=g)
    w[:, 0] = 0.0
    w[5, 0] = 1.0
    w[900] = w[5]
    w[n - 1] = w[5]
    x = torch.randn(m, k, generator=g)
    x[:, 0] = 10.0
    return x.to(dtype), w.to(dtype)


@pytest.mark.parametrize("dtype,m", [(torch.bfloat16, 26), (torch.float16, 26), (torch.bfloat16, 100)])
def test_lm_head_argmax_keys_name_each_rows_first_maximum(dtype, m):
    """pe_dense_gemm_argmax at the 7B lm_head's shape (K = 4096, N = 32000; 100
    rows run as two launches): the logits equal pe_dense_gemm's bit for bit, and
    each row's largest key names the first maximum of that row's stored logits
    (np.argmax), here mostly a three-way exact tie."""
    n, k = 32000, 4096
    x, w = _tied_lm_head(n, k, dtype, m, seed=m)
    wt = ops.dense_repack(w.to(DEV))
    out, keys, groups = _argmax_gemm(x.to(DEV), wt, n, dtype)
    assert groups == n // 64
    ref = ops.linear(x.to(DEV), n, dense=wt)
    assert torch.equal(out, ref)
    logits = out.float().cpu().numpy()
    kk = keys.cpu().numpy().view(np.uint64)
    best = kk.max(axis=1)
    got = (np.uint64(0xFFFFFFFF) - (best & np.uint64(0xFFFFFFFF))).astype(np.int64)
    want = logits.argmax(axis=1)
    assert np.array_equal(got, want)
    assert np.mean(want == 5) > 0.9  # the planted tie decides most rows


def test_accept_tree_from_argmax_keys_equals_the_logit_walk():
    """pe_accept_tree_keys (node argmaxes from the lm_head's keys) returns what
    pe_accept_tree returns on the same logits, with a chain of node tokens
    planted on the rows' argmaxes so the walk goes deep."""
    n, k, dtype = 32000, 4096, torch.bfloat16
    parents = [-1, 0, 0, 1, 1, 2, 3, 3, 4, 6, 6, 9]
    T = len(parents)
    x, w = _tied_lm_head(n, k, dtype, T, seed=11)
    x[1:, 0] = 0.0  # most rows without the tie feature: their own argmaxes
    logits, keys, groups = _argmax_gemm(x.to(DEV), ops.dense_repack(w.to(DEV)), n, dtype)
    root = torch.randn(n, generator=torch.Generator().manual_seed(4)).to(dtype).to(DEV)
    amax = [int(root.float().argmax())] + [int(r) for r in logits.float().argmax(dim=1).cpu()]
    tokens = [0] * T
    for node in (0, 1, 3, 6, 9):  # a chain through the tree
        tokens[node] = amax[0] if parents[node] < 0 else amax[1 + parents[node]]
    tok = torch.tensor(tokens, dtype=torch.int64, device=DEV)
    par = torch.tensor(parents, dtype=torch.int32, device=DEV)
    want = ops.accept_tree(root, logits, tok, par).cpu().tolist()
    L = _lib.load()
    out = torch.zeros(T + 2, dtype=torch.int32, device=DEV)
    scratch = torch.zeros(T + 2, dtype=torch.int32, device=DEV)
    _lib.check(L.pe_accept_tree_keys(root.data_ptr(), n, ops.dcode(dtype), keys.data_ptr(), groups, T, tok.data_ptr(),
                                     par.data_ptr(), out.data_ptr(), scratch.data_ptr(), ops.stream_ptr()),
               "pe_accept_tree_keys")
    got = out.cpu().tolist()
    assert got[: 2 + got[0]] == want[: 2 + want[0]]
    assert got[0] >= 5
    assert scratch[0].item() == 0


@pytest.mark.parametrize("path", [[], [0], [1, 3, 7], [0, 1, 2, 3, 4]])
def test_kv_compact_matches_gather_semantics(path):
    L, nkv, cap, hd, P, T = 3, 2, 64, 128, 20, 9
    k = torch.from_numpy(synth.normal(1, 60, L * nkv * cap * hd).reshape(L, nkv, cap, hd)).to(torch.bfloat16)
    v = torch.from_numpy(synth.normal(2, 61, L * nkv * cap * hd).reshape(L, nkv, cap, hd)).to(torch.bfloat16)
    res = torch.tensor([len(path), 0] + path + [0] * (T - len(path)), dtype=torch.int32)
    kd, vd = k.to(DEV), v.to(DEV)
    ops.kv_compact(kd, vd, P, res.to(DEV))
    n = P + len(path)
    ref_k = ov.compact_rows(k[:, :, : P + T].float().numpy(), P, path)
    ref_v = ov.compact_rows(v[:, :, : P + T].float().numpy(), P, path)
    assert np.array_equal(kd[:, :, :n].cpu().float().numpy(), ref_k)
    assert np.array_equal(vd[:, :, :n].cpu().float().numpy(), ref_v)


def test_kv_gather_general_keep_and_rejects_unsorted():
    L, nkv, cap, hd = 2, 2, 40, 64
    k = torch.from_numpy(synth.normal(3, 62, L * nkv * cap * hd).reshape(L, nkv, cap, hd))
    v = torch.from_numpy(synth.normal(4, 63, L * nkv * cap * hd).reshape(L, nkv, cap, hd))
    keep = [0, 1, 2, 5, 6, 9, 20, 21, 33]
    kd, vd = k.to(DEV), v.to(DEV)
    st = _status()
    ops.kv_gather(kd, vd, torch.tensor(keep, device=DEV), st)
    assert int(st[0]) == 0
    assert torch.equal(kd[:, :, : len(keep)].cpu(), k[:, :, keep])
    assert torch.equal(vd[:, :, : len(keep)].cpu(), v[:, :, keep])
    ops.kv_gather(kd, vd, torch.tensor([0, 3, 2], device=DEV), st)
    assert int(st[0]) & _lib.PE_ERR_INDEX
