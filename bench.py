#!/usr/bin/env python3
"""Tree-verification pass benchmark on one MI355X.

One step is one verification pass of a drafted tree against the KV cache,
entirely on the device and captured in a HIP graph: ancestor bitmasks and
positions from the parent list, the masked forward over the cache (embeddings,
every decoder layer with the in-place K/V append, final norm, lm_head over all
tree rows, fused features), the greedy acceptance walk and the in-place
compaction of the accepted rows. The default workload is the Llama-2-7B shape
with NF4 linears (block 64, fp16 absmax, bf16 compute), a 26-node depth-5 tree
over a 2048-token bf16 KV prefix, batch 1. Weights and the KV prefix are
synthetic (counter-based N(0, 0.02) weights, N(0, 1) K/V), resident in HBM
before timing starts.

Printed (one JSON line): ``value`` = algorithmic HBM bytes of one pass divided
by the measured pass time (GB/s), ``ms_per_step`` = pass latency, plus

- ``roofline``: the NF4 dequant-GEMM (every q/k/v, o, gate/up and down launch
  of one pass, in pass order, replayed from a HIP graph with HIP events on its
  stream), algorithmic bytes per launch over the mean launch time, against the
  8 TB/s HBM peak;
- ``cpu_baseline``: the CPU restatement of the reference path (per-call NF4
  dequantise, bf16 matmuls, masked SDPA, acceptance walk, index_select commit)
  timed on the host cores on a 4-layer slice of the same shape and scaled to
  the full layer count;
- ``roofline.traffic``: HBM bytes per NF4 GEMM launch as rocprofv3's
  FETCH_SIZE + WRITE_SIZE counters read them (calibrated on a plain copy, see
  ``--calibrate-copy``), taken from the committed profile summary of this
  workload.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--workload NAME] [--no-cpu-baseline]
       python bench.py --loop    (decode-loop tokens/s)
       python bench.py --calibrate-copy
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16 / fp16
DTYPE_NAMES = {"bfloat16": "bf16", "float16": "f16", "float32": "f32"}
METRIC = "tree-verify pass latency + HBM GB/s (% peak), 7B-int4 T=26 KV=2048 bs=1"
DEFAULT_WORKLOAD = "llama2-7b-nf4-T26-P2048"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default=DEFAULT_WORKLOAD)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--gemm-reps", type=int, default=10, help="replays of the per-pass NF4 GEMM sequence")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-layers", type=int, default=4, help="layers of the CPU-path sample")
    p.add_argument("--cpu-runs", type=int, default=12)
    p.add_argument("--prefill", action="store_true",
                   help="instead of the verification pass: time a causal prefill of the workload's prefix length "
                        "from an empty cache and a one-token continuation (eager forward_cached calls)")
    p.add_argument("--loop", action="store_true",
                   help="tokens/s of the decode loop (greedy and the device-resident speculative loop)")
    p.add_argument("--draft", action="store_true",
                   help="instead of the verification pass: time the drafting step before it (a 2-layer drafter's "
                        "draft_logits over the workload's prefix plus k - 1 mask slots, then the beam tree proposal)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run a 256 MiB device copy three times (the known-size kernel the HBM counters "
                        "FETCH_SIZE / WRITE_SIZE are calibrated on)")
    return p.parse_args(argv)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "nf4_gemm_traffic_llama2-7b-nf4-T26-P2048.md")


def profiled_traffic(workload: str):
    """HBM bytes per NF4 GEMM launch measured with rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, calibrated on a plain copy) for this workload, from the committed
    profile summary; None if there is none."""
    if workload != DEFAULT_WORKLOAD or not os.path.exists(TRAFFIC_PROFILE):
        return None
    for line in open(TRAFFIC_PROFILE):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- device pass
def build_step(wl, seed):
    import torch

    from parallel_eagle_amd import ops, synth
    from parallel_eagle_amd.target import TargetModel

    shape, P, T = wl.model, wl.prefix_len, wl.tree_nodes
    t0 = time.perf_counter()
    tm = TargetModel.synthetic(shape, seed=seed, device="cuda:0", cache_capacity=P + T)
    torch.cuda.synchronize()
    log(f"model {shape.name}: {tm.model.weight_bytes() / 1e9:.2f} GB of repacked layer weights "
        f"in {time.perf_counter() - t0:.1f} s")
    cache = tm.make_cache(P + T)
    ops.fill_normal(cache.k, seed, synth.STREAM_KV, 1.0)
    ops.fill_normal(cache.v, seed, synth.STREAM_KV_V, 1.0)
    # the root logit: a 1-token continuation that writes prefix row P - 1
    cache.seq_len = P - 1
    last = int(synth.uniform_int(seed, synth.STREAM_PROMPT, 1, shape.vocab)[0])
    root, _, cache = tm.forward_cached(torch.tensor([[last]]), cache, torch.tensor([[P - 1]]))
    root = root[0, -1].clone()
    tokens, parents = synth.tree_for_seed(seed, shape.vocab, wl.depth, wl.widths, wl.top_k)
    step = tm.verify_step(cache, T)
    # plant the device's own greedy chain along the deepest first branch, so the
    # timed pass accepts a full-depth path and compacts it
    chain = synth.chain_nodes(parents, synth.deepest_first_leaf(parents))
    row = root
    for node in chain:
        synth.set_token(tokens, parents, node, int(row.float().argmax()), shape.vocab)
        step.load_tree(tokens, parents, root)
        step.run()
        row = step.logits[node].clone()
    step.load_tree(tokens, parents, root)
    step.run()
    path, bonus = step.result()
    log(f"tree T={T} depth={wl.depth} widths={list(wl.widths)}: accepted {len(path)} nodes {path}, bonus {bonus}")
    return tm, cache, step, (tokens, parents, path, bonus)


def time_pass(step, steps: int, warmup: int):
    import torch

    step.capture()
    for _ in range(warmup):
        step.run()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(steps):
        step.run()
        evs[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(steps)]
    total_ms = evs[0].elapsed_time(evs[-1])
    return total_ms / steps, statistics.median(per), wall


def mfma_flops_per_pass(shape, T: int, P: int) -> int:
    """MFMA FLOPs one single-sequence pass issues, counted on the launch shapes
    (the v_mfma_f32_32x32x16 tiles: rows padded to 32; attention over the
    key blocks of 32 and the row tiles of the T x heads-per-KV-head query
    rows). The rocprofv3 counter SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 of the
    GEMM launches equals the GEMM part exactly."""
    mp = -(-T // 32) * 32
    lin = sum(n * k for _, n, k in shape.linear_shapes())
    gemm = 2 * mp * lin * shape.num_layers + 2 * mp * shape.vocab * shape.hidden
    g = shape.num_heads // shape.num_kv_heads
    rows = -(-T * g // 32) * 32
    keys = -(-(P + T) // 32) * 32
    attn = 4 * rows * keys * shape.head_dim * shape.num_kv_heads * shape.num_layers
    return gemm + attn


def nf4_gemm_roofline(tm, wl, reps: int):
    """Mean duration and algorithmic bytes per launch of the NF4 dequant-GEMM
    kernel as the pass runs it: the 4 * L launches of one pass on A-tiled
    activations, same weights, shapes and launch plans (q/k/v unsplit with
    eight waves per workgroup, here with the plain store epilogue in place of
    RoPE + KV append; o and down as fp32 split partials; gate/up unsplit with
    the SwiGLU epilogue into the A-tiled activation), replayed from a HIP graph
    and timed with HIP events on the stream the launches use."""
    import ctypes as C

    import torch

    from parallel_eagle_amd import _lib, ops

    L = _lib.load()
    m, s = tm.model, tm.shape
    M, H, ip = wl.tree_nodes * wl.batch, s.hidden, m.ipad
    qd, kvd = s.q_dim, s.kv_dim
    nqkv = qd + 2 * kvd
    dev = tm.device
    bf = torch.bfloat16
    xn_t = ops.to_xtile(torch.randn((M, H), device=dev).to(bf))
    attn_t = ops.to_xtile(torch.randn((M, qd), device=dev).to(bf))
    act_t = ops.to_xtile((0.1 * torch.randn((M, ip), device=dev)).to(bf))
    part_bytes = max(int(L.pe_nf4_gemm_partials_bytes(M, n, k)) for n, k in
                     [(nqkv, H), (H, qd), (2 * ip, H), (H, ip)])
    part = torch.empty(part_bytes // 4, dtype=torch.float32, device=dev)
    splits = C.c_int(0)
    st = ops.stream_ptr
    qkv_out = torch.empty((M, nqkv), dtype=bf, device=dev)
    act_out = torch.zeros_like(act_t)
    ws_bytes = max(int(L.pe_gemm_workspace_bytes(M, n, H, _lib.PE_WFMT_NF4, _lib.PE_DTYPE_BF16, epi))
                   for n, epi in ((nqkv, _lib.PE_EPI_STORE), (2 * ip, _lib.PE_EPI_SWIGLU)))
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)

    def unsplit(x, K, w, a, N, epi, out, ld_out, out_units):
        _lib.check(L.pe_nf4_gemm_tiled(x.data_ptr(), M, K, w.data_ptr(), a.data_ptr(), N, epi, None, None, 0,
                                       out.data_ptr(), ld_out, out_units, ws.data_ptr(), ws_bytes, st()),
                   "pe_nf4_gemm_tiled")

    def partials(x, K, w, a, N):
        _lib.check(L.pe_nf4_gemm_partials(x.data_ptr(), K, 1, M, K, w.data_ptr(), a.data_ptr(), N,
                                          part.data_ptr(), part_bytes, C.byref(splits), st()),
                   "pe_nf4_gemm_partials")

    def seq():
        for ly in m.layers:
            unsplit(xn_t, H, ly["w_qkv"], ly["a_qkv"], nqkv, _lib.PE_EPI_STORE, qkv_out, nqkv, 0)
            partials(attn_t, qd, ly["w_o"], ly["a_o"], H)
            unsplit(xn_t, H, ly["w_gu"], ly["a_gu"], 2 * ip, _lib.PE_EPI_SWIGLU, act_out, 0, ip // 128)
            partials(act_t, ip, ly["w_down"], ly["a_down"], H)

    seq()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        seq()
    g.replay()
    torch.cuda.synchronize()
    # events on the current stream, which is the stream the replay runs on
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    launches = 4 * s.num_layers
    mean_us = e0.elapsed_time(e1) * 1e3 / (reps * launches)
    # algorithmic bytes: NF4 codes (0.5 B) + fp16 absmax (2 B / 64) + bf16 X once + the
    # linear's bf16 output once
    def nf4_bytes(n, k):
        return n * k // 2 + (n * k // 64) * 2

    I = s.intermediate
    per_layer = sum(nf4_bytes(n, k) + 2 * M * k + 2 * M * n for n, k in ((nqkv, H), (H, qd), (2 * I, H), (H, I)))
    bytes_per_launch = per_layer * s.num_layers / launches
    gbs = bytes_per_launch / (mean_us * 1e-6) / 1e9
    return {"kernel": "nf4_gemm_kernel (A-tiled X; q/k/v unsplit, gate/up as whole column groups plus halves, "
                      "o and down fp32 split partials in one round of workgroups: the 4 x L launches of one pass)",
            "mean_launch_us": round(mean_us, 3), "bytes_per_launch": int(bytes_per_launch),
            "achieved": round(gbs, 1)}


# ---------------------------------------------------------------- CPU path
def cpu_baseline(wl, seed, n_layers: int, runs: int):
    """The reference path on the host cores (the oracle restatement, timed):
    tree mask + additive bias, forward with per-call NF4 dequantise, matmuls
    and masked SDPA, the acceptance walk, and the index_select commit over
    every layer's cache, on an ``n_layers`` slice of the shape at full width,
    P and T (the whole model when it has no more layers). Stages are timed
    separately (median of ``runs`` warm runs): mask, dequant, matmul (the
    lm_head apart), sdpa, the rest of the forward (norms, RoPE, SwiGLU, KV
    concatenation), walk and commit; per-layer stages are scaled to the full
    layer count. A second timing with every linear dequantised once beforehand
    is the lower bound of the same path without per-call dequantisation."""
    import torch

    from oracle import masks as om
    from oracle import verify as ov
    from oracle.model import OracleTarget
    from parallel_eagle_amd import synth
    from parallel_eagle_amd.config import algorithmic_bytes
    from parallel_eagle_amd.model import DeviceModel

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    full = wl.model
    n_layers = min(n_layers, full.num_layers)
    scale = full.num_layers / n_layers
    if n_layers < full.num_layers:
        fl = tuple(min(f, n_layers) for f in (1, n_layers, n_layers))
        shape = full.reduced(n_layers, feature_layers=fl)
    else:
        shape = full
    dm = DeviceModel.synthetic(shape, seed, "cuda:0", keep_logical=True)
    hw = dm.host_weights()
    del dm
    torch.cuda.empty_cache()
    orc = OracleTarget(shape, hw)
    orc.timer.enabled = True
    P, T = wl.prefix_len, wl.tree_nodes
    dt = orc.dtype
    g = torch.Generator().manual_seed(seed)
    kv = [(torch.randn((1, full.num_kv_heads, P, full.head_dim), generator=g).to(dt),
           torch.randn((1, full.num_kv_heads, P, full.head_dim), generator=g).to(dt)) for _ in range(n_layers)]
    root = torch.randn(full.vocab, generator=g).to(dt)
    tokens, parents = synth.tree_for_seed(seed, full.vocab, wl.depth, wl.widths, wl.top_k)

    def one():
        orc.timer.seconds.clear()
        t0 = time.perf_counter()
        allow = om.tree_allow_mask(parents, P)
        bias = om.to_additive_bias(allow[P:, :], dt)
        pos = om.tree_position_ids(parents, P)[P:]
        t1 = time.perf_counter()
        lg, _, cache = orc.forward(tokens, pos, kv, bias)
        t2 = time.perf_counter()
        path, _ = ov.accept_tree_cached(root, lg[0], tokens, parents)
        t3 = time.perf_counter()
        keep = torch.tensor(list(range(P)) + [P + t for t in path])
        for k_, v_ in cache:
            k_.index_select(2, keep).contiguous()
            v_.index_select(2, keep).contiguous()
        t4 = time.perf_counter()
        st = dict(orc.timer.seconds)
        return {"mask": t1 - t0, "forward": t2 - t1, "walk": t3 - t2, "commit": t4 - t3,
                "dequant": st.get("dequant", 0.0), "matmul": st.get("matmul", 0.0), "sdpa": st.get("sdpa", 0.0)}

    def median_of(samples, key):
        return statistics.median(smp[key] for smp in samples)

    one()  # warm-up
    samples = [one() for _ in range(runs)]
    # the lm_head product alone: the per-pass (unscaled) part of "matmul"
    x = torch.randn((1, T, full.hidden)).to(dt)
    lm = hw["lm_head"]
    heads = []
    for _ in range(runs + 1):
        t0 = time.perf_counter()
        torch.nn.functional.linear(x, lm)
        heads.append(time.perf_counter() - t0)
    t_head = statistics.median(heads[1:])

    def full_pass(smp):
        st = {k: median_of(smp, k) for k in ("mask", "forward", "walk", "commit", "dequant", "matmul", "sdpa")}
        mm_layers = max(0.0, st["matmul"] - t_head)
        other = max(0.0, st["forward"] - st["dequant"] - st["matmul"] - st["sdpa"])
        stages = {"mask": st["mask"], "dequant": st["dequant"] * scale, "matmul": mm_layers * scale + t_head,
                  "sdpa": st["sdpa"] * scale, "other_forward": other * scale, "walk": st["walk"],
                  "commit": st["commit"] * scale}
        return stages, sum(stages.values())

    stages, t_pass = full_pass(samples)
    # lower bound: the same forward with every linear dequantised once beforehand
    orc.cache_dequant = True
    one()
    pre = [one() for _ in range(runs)]
    _, t_pre = full_pass(pre)
    pass_bytes = algorithmic_bytes(full, [P] * wl.batch, T)
    nf4 = full.weight_format == "nf4"
    return {"value": round(pass_bytes / t_pass / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "ms_per_pass": round(t_pass * 1e3, 1),
            "stages_ms": {k: round(v * 1e3, 2) for k, v in stages.items()},
            "ms_per_pass_predequantised": round(t_pre * 1e3, 1) if nf4 else None,
            "sample": (f"oracle forward of {'a ' + str(n_layers) + '-layer slice' if scale > 1 else 'the whole model'}"
                       f" at full width (H={full.hidden}, I={full.intermediate}, V={full.vocab}, P={P}, T={T}"
                       f"{'; per-call NF4 dequantise in torch' if nf4 else ''}), median of {runs} runs after "
                       f"1 warm-up{', per-layer stages scaled x' + format(scale, 'g') if scale > 1 else ''}; "
                       f"torch threads = {cores}")}


# ---------------------------------------------------------------- main
def prefill_line(wl, seed: int, reps: int = 3) -> dict:
    """Latency of the causal prefill of the workload's prefix (P tokens from an empty
    cache, the prompt step before the first verification) and of a one-token
    continuation (the miss path), eager forward_cached calls after a warm-up call
    each. Past 256 tokens the prefill runs every linear once over all rows on the
    library's many-row MFMA kernels; ``mfma`` is the pass's matrix-core FLOP (the
    linears and the lm_head, 2 M N K each, plus causal attention) over its time."""
    import torch

    from parallel_eagle_amd import synth
    from parallel_eagle_amd.target import TargetModel

    shape, P = wl.model, wl.prefix_len
    tm = TargetModel.synthetic(shape, seed=seed, device="cuda:0", cache_capacity=P + 64)
    ids = torch.tensor([synth.uniform_int(seed, synth.STREAM_PROMPT, P, shape.vocab).tolist()])
    pos = torch.arange(P).unsqueeze(0)
    pre, one = [], []
    for r in range(reps + 1):
        cache = tm.make_cache(P + 64)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tm.forward_cached(ids, cache, pos)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        tm.forward_cached(torch.tensor([[5]]), cache, torch.tensor([[P]]))
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if r:
            pre.append(t1 - t0)
            one.append(t2 - t1)
    ms = statistics.median(pre) * 1e3
    lin = sum(n * k for _, n, k in shape.linear_shapes()) * shape.num_layers + shape.vocab * shape.hidden
    attn = 2 * 2 * shape.num_heads * shape.head_dim * P * (P + 1) / 2 * shape.num_layers  # causal QK^T and PV
    flop = 2 * P * lin + attn
    return {"metric": "prefill latency (causal, from an empty cache) and one-token continuation latency",
            "value": round(P / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": reps,
            "ms_prefill": round(ms, 3), "ms_one_token": round(statistics.median(one) * 1e3, 3),
            "mfma": {"flop": flop, "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                     "util": round(flop / (ms * 1e-3) / (MFMA_BF16_PEAK_TFLOPS * 1e12), 4)},
            "higher_is_better": True, "dtype": DTYPE_NAMES[shape.dtype], "data": "synthetic",
            "config": {"workload": wl.name, "prefill_tokens": P, "layers": shape.num_layers,
                       "weights": shape.weight_format, "eager": True}}


def loop_line(wl, seed: int, new_tokens: int = 96) -> dict:
    """Tokens/s of the whole decode loop on the workload's model (synthetic
    weights, all layers) over a P-token random prompt: greedy decoding through
    forward_cached (greedy_decode, one one-token pass per token) and the
    device-resident speculative loop (SpeculativeDecoder: drafter, device beam,
    then one recorded step replayed: masks, verification pass, walk,
    compaction, commit; one host read per step)
    with (a) a random 2-layer device drafter (nothing is accepted: every step
    is the miss path) and (b) the same drafter told the greedy continuation
    (every depth the greedy decode chose). Each run reports whether it emitted
    exactly the greedy tokens. On random weights the logits are flat (about 30%
    of greedy steps have a top-1 / top-2 margin under 0.1, a few bf16 ulps),
    and a tree pass over 20 rows rounds differently from a one-token pass, so
    the hint is rejected at such near ties and the output can part from greedy
    decoding there; the loop's exactness is tested on the fp32 model."""
    import torch

    from parallel_eagle_amd import synth
    from parallel_eagle_amd.drafter import DeviceDrafter
    from parallel_eagle_amd.serve import SpeculativeDecoder, greedy_decode
    from parallel_eagle_amd.target import TargetModel
    from parallel_eagle_amd.tree import beam_width

    shape, P, k = wl.model, wl.prefix_len, wl.depth
    top_k, max_nodes = wl.top_k, wl.tree_nodes
    T = beam_width(k, top_k, max_nodes) * k
    cap = P + new_tokens + T + 64
    tm = TargetModel.synthetic(shape, seed=seed, device="cuda:0", cache_capacity=cap)
    H, nfl = shape.hidden, len(shape.resolved_feature_layers())
    g = torch.Generator(device="cuda:0").manual_seed(seed)

    def r(*sz, std=shape.init_std):
        return (torch.randn(*sz, generator=g, device="cuda:0") * std).to(tm.dtype)

    from dataclasses import replace
    layers = []
    for _ in range(2):
        lw = {n: r(o, i) for n, o, i in replace(shape, qkv_bias=False).linear_shapes()}
        lw["attn_norm"] = torch.ones(H, dtype=tm.dtype, device="cuda:0")
        lw["mlp_norm"] = torch.ones(H, dtype=tm.dtype, device="cuda:0")
        layers.append(lw)
    w = {"feat_norm": torch.ones(H, dtype=tm.dtype, device="cuda:0"), "feat_proj": r(H, nfl * H),
         "in_proj": r(H, 2 * H), "mask_emb": r(H), "h_shared": r(H), "layers": layers}
    drafter = DeviceDrafter(tm, w, max_depth=k, capacity=cap)
    prompt = synth.uniform_int(seed, synth.STREAM_PROMPT, P, shape.vocab).tolist()

    class GreedyHint:
        """The drafter, its logits replaced by a peak at the greedy token of each depth."""

        def __init__(self, inner, greedy):
            self.inner, self.greedy = inner, greedy
            self.status = inner.status

        @property
        def sync_status(self):
            return self.inner.sync_status

        @sync_status.setter
        def sync_status(self, v):
            self.inner.sync_status = v

        def reset(self):
            self.inner.reset()

        def draft_logits(self, ctx, feats, kk):
            return self._hint(self.inner.draft_logits(ctx, feats, kk), ctx, kk)

        def draft_logits_extend(self, ctx, feats, kk):
            return self._hint(self.inner.draft_logits_extend(ctx, feats, kk), ctx, kk)

        def _hint(self, lg, ctx, kk):
            lg = lg.clone()
            n = ctx.numel()
            for d in range(kk):
                if n + d < len(self.greedy):
                    lg[d] = lg[d].min()
                    lg[d, self.greedy[n + d]] = 30.0
            return lg

    greedy_decode(tm, prompt, 4)  # warm-up (kernel loads, caches)
    torch.cuda.synchronize()
    greedy = greedy_decode(tm, prompt, new_tokens)
    full = prompt + greedy.tokens
    runs = {}
    for name, dr in (("random_drafter", drafter), ("greedy_hint_drafter", GreedyHint(drafter, full))):
        dec = SpeculativeDecoder(tm, dr, k=k, tree_top_k=top_k, tree_max_nodes=max_nodes)
        dec.generate(prompt, 8)  # warm-up
        res = dec.generate(prompt, new_tokens)
        same = res.tokens == greedy.tokens
        first = next((i for i, (x, y) in enumerate(zip(res.tokens, greedy.tokens)) if x != y), None)
        runs[name] = {"tokens_per_s": round(res.tokens_per_second, 1), "steps": res.steps,
                      "ms_per_step": round(res.seconds * 1e3 / max(1, res.steps), 3),
                      "tokens_per_step": round(res.tokens_per_step, 3), "target_passes": res.target_passes,
                      "host_reads": res.host_reads, "recorded_steps": dec.device_prefix,
                      "equal_to_greedy": same, "first_difference": first}
        log(f"loop ({name}): {res.tokens_per_second:.1f} tokens/s, {res.tokens_per_step:.2f} tokens per step, "
            f"{runs[name]['ms_per_step']} ms per step, {res.host_reads} host reads in {res.steps} steps, "
            f"equal to greedy decoding: {same}" + ("" if same else f" (first difference at token {first})"))
    log(f"greedy decoding through the same API: {greedy.tokens_per_second:.1f} tokens/s")
    best = runs["greedy_hint_drafter"]
    return {
        "metric": "decode loop tokens/s (device-resident speculative loop, synthetic weights)",
        "value": best["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": DTYPE_NAMES[shape.dtype], "data": "synthetic",
        "config": {"workload": wl.name, "layers": shape.num_layers, "prompt_len": P, "new_tokens": new_tokens,
                   "depth": k, "tree_nodes": T, "drafter_layers": 2},
        "greedy_tokens_per_s": round(greedy.tokens_per_second, 1), "speculative": runs,
    }


def draft_line(wl, seed: int, reps: int = 10) -> dict:
    """Latency of one drafting step at the workload's shape: DeviceDrafter.draft_logits
    (2 dense decoder layers, the reference's default depth, over the P context rows
    plus k - 1 mask slots, sharing the target's embed / final norm / lm_head) and the
    device beam over its k logit rows with the workload's per-depth widths. Random
    drafter weights at the target's init scale; eager calls after a warm-up call."""
    import torch

    from parallel_eagle_amd import synth
    from parallel_eagle_amd.drafter import DeviceDrafter
    from parallel_eagle_amd.target import TargetModel
    from parallel_eagle_amd.tree import propose_tree_device

    shape, P, k = wl.model, wl.prefix_len, wl.depth
    # the drafter reads only the target's embed, final norm and lm_head
    tm = TargetModel.synthetic(shape.reduced(1), seed=seed, device="cuda:0", cache_capacity=64)
    H, nfl = shape.hidden, len(shape.resolved_feature_layers())
    g = torch.Generator(device="cuda:0").manual_seed(seed)

    def r(*sz, std=shape.init_std):
        return (torch.randn(*sz, generator=g, device="cuda:0") * std).to(torch.bfloat16)

    from dataclasses import replace
    layers = []
    for _ in range(2):
        lw = {n: r(o, i) for n, o, i in replace(shape, qkv_bias=False).linear_shapes()}
        lw["attn_norm"] = torch.ones(H, dtype=torch.bfloat16, device="cuda:0")
        lw["mlp_norm"] = torch.ones(H, dtype=torch.bfloat16, device="cuda:0")
        layers.append(lw)
    w = {"feat_norm": torch.ones(H, dtype=torch.bfloat16, device="cuda:0"), "feat_proj": r(H, nfl * H),
         "in_proj": r(H, 2 * H), "mask_emb": r(H), "h_shared": r(H), "layers": layers}
    dr = DeviceDrafter(tm, w, max_depth=k, capacity=P + k)
    ids = torch.tensor(synth.uniform_int(seed, synth.STREAM_PROMPT, P, shape.vocab).tolist(), device="cuda:0")
    feats = r(P, nfl * H, std=1.0)
    full, logit_only = [], []
    for i in range(reps + 1):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        lg = dr.draft_logits(ids, feats, k)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        tok, par, st = propose_tree_device(lg, wl.widths, wl.top_k)
        n = int(st.item()) + tok.numel()  # waits for the beam
        t2 = time.perf_counter()
        if i:
            logit_only.append(t1 - t0)
            full.append(t2 - t0)
    assert n == sum(wl.widths)
    ms = statistics.median(full) * 1e3
    return {"metric": "drafting step latency (draft_logits over the context + beam tree proposal)",
            "value": round(ms, 3), "unit": "ms", "n_gpus": 1, "steps": reps,
            "ms_draft_logits": round(statistics.median(logit_only) * 1e3, 3),
            "ms_tree_proposal": round(ms - statistics.median(logit_only) * 1e3, 3),
            "higher_is_better": False, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": wl.name, "context_tokens": P, "depths": k, "tree_nodes": sum(wl.widths),
                       "drafter_layers": 2, "eager": True}}




def batch_line(wl, seed: int, steps: int, warmup: int, gemm_reps: int) -> dict:
    """The batched workload: wl.batch sequences, each a wl.tree_nodes-node tree
    over its own prefix (seeded lengths in [prefix_min, prefix_len]), one
    BatchVerifyStep (masks -> batched pass -> per-sequence walks -> ragged
    compaction) replayed from a HIP graph. Roofline: the NF4 GEMM launches of
    one pass at M = batch * tree_nodes rows (one many-row launch per linear),
    replayed from a graph; FLOPs 2 * rows * N * K per launch against the dense
    bf16 MFMA peak."""
    import ctypes as C

    import torch

    from parallel_eagle_amd import _lib, ops, synth
    from parallel_eagle_amd import batch as pb
    from parallel_eagle_amd.config import algorithmic_bytes
    from parallel_eagle_amd.target import TargetModel

    shape, T, B = wl.model, wl.tree_nodes, wl.batch
    prefixes = (synth.uniform_int(seed, 8, B, wl.prefix_len - wl.prefix_min + 1) + wl.prefix_min).tolist()
    cap = max(prefixes) + T + 32
    t0 = time.perf_counter()
    tm = TargetModel.synthetic(shape, seed=seed, device="cuda:0", cache_capacity=cap)
    torch.cuda.synchronize()
    log(f"model {shape.name}: {tm.model.weight_bytes() / 1e9:.2f} GB of repacked layer weights "
        f"in {time.perf_counter() - t0:.1f} s; prefixes {prefixes}")
    cache = pb.BatchKVCache(tm, B, cap)
    ops.fill_normal(cache.k, seed, synth.STREAM_KV, 1.0)
    ops.fill_normal(cache.v, seed, synth.STREAM_KV_V, 1.0)
    for b, P in enumerate(prefixes):
        cache.seq(b).seq_len = P
    trees = [synth.tree_for_seed(16 * seed + b, shape.vocab, wl.depth, wl.widths, wl.top_k) for b in range(B)]
    tokens = [t for t, _ in trees]
    parents = [p for _, p in trees]
    roots = ops.fill_normal(torch.empty((B, shape.vocab), dtype=tm.dtype, device="cuda:0"), seed, 9, 1.0)
    # plant each sequence's greedy chain (root argmax, then the pass's own node
    # argmaxes) along its deepest first branch: every timed pass accepts full depth
    chains = [synth.chain_nodes(p, synth.deepest_first_leaf(p)) for p in parents]
    rows = [roots[b] for b in range(B)]
    for d in range(wl.depth):
        for b in range(B):
            synth.set_token(tokens[b], parents[b], chains[b][d], int(rows[b].float().argmax()), shape.vocab)
        step = pb.BatchVerifyStep(tm, cache, tokens, parents)
        step.root.copy_(roots)
        step.run()
        torch.cuda.synchronize()
        for b in range(B):
            cache.seq(b).seq_len = prefixes[b]
        rows = [step.logits[step.trees.row0[b] + chains[b][d]].clone() for b in range(B)]
    step = pb.BatchVerifyStep(tm, cache, tokens, parents)
    step.root.copy_(roots)
    step.run()
    res = step.results()
    log(f"accepted per sequence: {[len(p) for p, _ in res]}")
    ms, med_ms, _ = time_pass(step, steps, warmup)
    if step.results() != res:
        log("WARNING: graph replay accepted other paths than the eager pass")
    pass_bytes = algorithmic_bytes(shape, prefixes, T)
    M = B * T
    lin = sum(n * k for _, n, k in shape.linear_shapes()) * shape.num_layers + shape.vocab * shape.hidden
    kv_flops = sum(4 * shape.num_heads * shape.head_dim * T * (P + T) for P in prefixes) * shape.num_layers
    pass_flops = 2 * M * lin + kv_flops
    # the NF4 GEMM launches of one pass (the many-row kernel on A-tiled
    # activations, fp32 split partials), replayed from a graph
    L = _lib.load()
    m = tm.model
    H, ip, qd = shape.hidden, m.ipad, shape.q_dim
    nqkv = qd + 2 * shape.kv_dim
    bf = torch.bfloat16
    xs = {k: ops.to_xtile((0.5 * torch.randn((M, k), device="cuda:0")).to(bf)) for k in (H, qd, ip)}
    dims = ((nqkv, H), (H, qd), (2 * ip, H), (H, ip))
    pb_bytes = max(int(L.pe_nf4_gemm_partials_bytes(M, n, k)) for n, k in dims)
    if pb_bytes <= 0:
        raise RuntimeError(f"no many-row NF4 plan for {M} rows")
    part = torch.empty(pb_bytes // 4, dtype=torch.float32, device="cuda:0")
    splits = C.c_int(0)

    def gemm(x, K, w, a, N):
        _lib.check(L.pe_nf4_gemm_partials(x.data_ptr(), K, 1, M, K, w.data_ptr(), a.data_ptr(), N, part.data_ptr(),
                                          pb_bytes, C.byref(splits), ops.stream_ptr()), "pe_nf4_gemm_partials")

    def seq():
        for ly in m.layers:
            gemm(xs[H], H, ly["w_qkv"], ly["a_qkv"], nqkv)
            gemm(xs[qd], qd, ly["w_o"], ly["a_o"], H)
            gemm(xs[H], H, ly["w_gu"], ly["a_gu"], 2 * ip)
            gemm(xs[ip], ip, ly["w_down"], ly["a_down"], H)

    seq()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        seq()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(gemm_reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    launches = 4 * shape.num_layers
    gemm_s = e0.elapsed_time(e1) * 1e-3 / gemm_reps
    gemm_flops = 2 * M * sum(n * k for _, n, k in shape.linear_shapes()) * shape.num_layers
    tflops = gemm_flops / gemm_s / 1e12
    log(f"batched pass {ms:.3f} ms; NF4 GEMMs {gemm_s * 1e3:.3f} ms per pass ({launches} launches), "
        f"{tflops:.1f} TFLOP/s")
    return {
        "metric": "batched tree-verify pass latency + MFMA TFLOP/s (% of dense bf16 peak), "
                  "Qwen2.5-14B-int4 B=8 T=26 KV~U[512,4096]",
        "value": round(pass_flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": wl.name, "layers": shape.num_layers, "hidden": shape.hidden,
                   "heads": f"{shape.num_heads}/{shape.num_kv_heads}", "intermediate": shape.intermediate,
                   "vocab": shape.vocab, "weights": shape.weight_format, "batch": B, "tree_nodes": T,
                   "rows": M, "prefix_lens": prefixes, "pass_bytes": pass_bytes, "pass_flops": pass_flops,
                   "hip_graph": True},
        "latency_ms_median": round(med_ms, 4),
        "pass_gbs": round(pass_bytes / (ms * 1e-3) / 1e9, 1),
        "accepted": [len(p) for p, _ in res],
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": f"nf4_gemm_bigws_kernel (A-tiled X, all {M} rows in one launch per linear, each "
                               f"weight dequantised once by producer waves for the consumer waves' MFMAs; fp32 "
                               f"split partials: the {launches} launches of one pass)",
                     "mean_launch_us": round(gemm_s * 1e6 / launches, 3)},
        "cpu_baseline": None,
    }


def main(argv=None) -> int:
    a = parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: the verification pass runs on a single device and no multi-GPU "
              f"path is built (asked for --gpus {a.gpus})", file=sys.stderr)
        return 2
    import torch

    from parallel_eagle_amd.config import WORKLOADS, algorithmic_bytes

    if a.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copied 256 MiB three times")
        return 0
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    wl = WORKLOADS[a.workload]
    if a.prefill:
        print(json.dumps(prefill_line(wl, a.seed)))
        return 0
    if a.draft:
        print(json.dumps(draft_line(wl, a.seed)))
        return 0
    if a.loop:
        print(json.dumps(loop_line(wl, a.seed)))
        return 0
    if wl.batch != 1:
        print(json.dumps(batch_line(wl, a.seed, a.steps, a.warmup, a.gemm_reps)), flush=True)
        return 0
    tm, cache, step, (tokens, parents, path, bonus) = build_step(wl, a.seed)
    pass_bytes = algorithmic_bytes(wl.model, [wl.prefix_len], wl.tree_nodes)
    ms, med_ms, wall = time_pass(step, a.steps, a.warmup)
    path2, bonus2 = step.result()
    if (path2, bonus2) != (path, bonus):
        log(f"WARNING: graph replay accepted {path2}/{bonus2}, eager pass {path}/{bonus}")
    gbs = pass_bytes / (ms * 1e-3) / 1e9
    log(f"pass: {ms:.4f} ms mean, {med_ms:.4f} ms median over {a.steps} steps "
        f"({pass_bytes / 1e9:.3f} GB algorithmic -> {gbs:.0f} GB/s, {gbs / HBM_PEAK_GBS:.1%} of peak)")
    roof = None
    if wl.model.weight_format == "nf4":
        r = nf4_gemm_roofline(tm, wl, a.gemm_reps)
        log(f"NF4 GEMM: {r['mean_launch_us']} us per launch, {r['bytes_per_launch'] / 1e6:.2f} MB -> "
            f"{r['achieved']} GB/s")
        roof = {"bound": "hbm", "achieved": r["achieved"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(r["achieved"] / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(wl.name),
                "kernel": r["kernel"], "mean_launch_us": r["mean_launch_us"],
                "bytes_per_launch": r["bytes_per_launch"]}
    mfma = None
    if wl.model.dtype != "float32":  # the fp32 path runs on the VALU
        fl = mfma_flops_per_pass(wl.model, wl.tree_nodes, wl.prefix_len)
        tf = fl / (ms * 1e-3) / 1e12
        mfma = {"flops_per_pass": fl, "tflops": round(tf, 1), "util": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                "peak_tflops": MFMA_BF16_PEAK_TFLOPS}
    cpu = None
    if not a.no_cpu_baseline:
        del step
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        cpu = cpu_baseline(wl, a.seed, a.cpu_layers, a.cpu_runs)
        log(f"CPU path: {cpu['ms_per_pass']} ms per pass on {cpu['cores']} threads "
            f"({time.perf_counter() - t0:.1f} s of sampling)")
    out = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": DTYPE_NAMES[wl.model.dtype], "data": "synthetic",
        "config": {"workload": wl.name, "layers": wl.model.num_layers, "hidden": wl.model.hidden,
                   "heads": f"{wl.model.num_heads}/{wl.model.num_kv_heads}", "intermediate": wl.model.intermediate,
                   "vocab": wl.model.vocab, "weights": wl.model.weight_format, "tree_nodes": wl.tree_nodes,
                   "tree_depth": wl.depth, "prefix_len": wl.prefix_len, "batch": wl.batch,
                   "pass_bytes": pass_bytes, "hip_graph": True},
        "latency_ms_median": round(med_ms, 4),
        "pass_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
        "accepted": len(path),
        "mfma": mfma,
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
