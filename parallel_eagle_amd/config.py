"""Model shapes and verification-pass workloads.

A ``ModelShape`` carries what the reference reads from the HF config of its
frozen target (``src/pe/target.py:100-166``): layer count, hidden size, head
layout, intermediate size, vocabulary, RMSNorm epsilon, RoPE theta, whether
q/k/v carry a bias (Qwen2, HF ``models/qwen2/modeling_qwen2.py:189-192``), the
storage format of the linear weights, and the three feature layers whose hidden
states are fused (``src/pe/target.py:103-128,161-162``).

``PassWorkload`` adds the per-pass sizes: KV prefix length ``P``, tree size ``T``
and depth, the per-depth beam widths, and the batch of independent sequences.
The five named workloads are the shapes the verification pass is tested and
measured on.
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace


@dataclass(frozen=True)
class ModelShape:
    name: str
    num_layers: int
    hidden: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0
    qkv_bias: bool = False
    # "nf4": linears are NF4 (block 64 along K, fp16 absmax) computed in bf16;
    # "dense": linears are stored in ``dtype``.
    weight_format: str = "dense"
    # compute dtype: "float32" | "bfloat16" | "float16"
    dtype: str = "bfloat16"
    feature_layers: tuple[int, ...] | None = None
    max_positions: int = 16384
    init_std: float = 0.02

    @property
    def q_dim(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def group(self) -> int:
        return self.num_heads // self.num_kv_heads

    def resolved_feature_layers(self) -> tuple[int, ...]:
        return resolve_feature_layers(self.feature_layers, self.num_layers)

    def linear_shapes(self) -> list[tuple[str, int, int]]:
        """(name, N_out, K_in) for every per-layer linear, in forward order."""
        return [
            ("q", self.q_dim, self.hidden),
            ("k", self.kv_dim, self.hidden),
            ("v", self.kv_dim, self.hidden),
            ("o", self.hidden, self.q_dim),
            ("gate", self.intermediate, self.hidden),
            ("up", self.intermediate, self.hidden),
            ("down", self.hidden, self.intermediate),
        ]

    def reduced(self, num_layers: int, **kw) -> "ModelShape":
        """Same shape with fewer layers (parity at full width, bounded CPU time)."""
        return replace(self, name=f"{self.name}-L{num_layers}", num_layers=num_layers, **kw)


def resolve_feature_layers(layers, num_layers: int) -> tuple[int, ...]:
    """Map requested feature-layer indices onto valid hidden-state slots.

    Mirrors ``TargetModel._resolve_feature_layers`` (``src/pe/target.py:103-128``):
    ``None`` picks round(n * f) for f in (0.25, 0.55, 0.95); indices are clamped
    to [1, n]; duplicates are replaced by the distinct depth-relative set padded
    with its last entry.
    """
    n = num_layers
    if layers is None:
        layers = tuple(round(n * f) for f in (0.25, 0.55, 0.95))
    out = []
    for layer in layers:
        idx = layer if layer >= 0 else n + 1 + layer
        out.append(max(1, min(idx, n)))
    if len(set(out)) < len(out):
        out = sorted({max(1, min(round(n * frac), n)) for frac in (0.25, 0.55, 0.95)})
        while len(out) < len(layers):
            out.append(out[-1])
    return tuple(out)


@dataclass(frozen=True)
class PassWorkload:
    name: str
    model: ModelShape
    prefix_len: int  # P (batch 1) or the upper bound of the ragged range
    tree_nodes: int  # T per sequence
    depth: int  # k, number of tree depths
    top_k: int
    widths: tuple[int, ...]  # nodes kept per depth (sums to tree_nodes)
    batch: int = 1
    prefix_min: int | None = None  # ragged batches: P_b ~ U[prefix_min, prefix_len]
    seeds: tuple[int, ...] = field(default=tuple(range(10)))


def width_schedule(tree_nodes: int, depth: int, top_k: int) -> tuple[int, ...]:
    """Per-depth beam widths for a tree of ``tree_nodes`` nodes over ``depth`` depths.

    The reference's ``propose_tree`` (``src/pe/decode/tree.py:36-55``) keeps a
    constant width ``min(top_k, max_nodes // k)``. Tree sizes that are not a
    multiple of ``k`` need per-depth widths: depth 0 keeps ``min(top_k, T // k)``
    and the remaining nodes are spread evenly over depths 1..k-1 with the extras
    on the deepest depths. Where ``T == k * w`` this is the constant schedule.
    """
    w0 = max(1, min(top_k, tree_nodes // depth))
    if depth == 1:
        return (min(w0, tree_nodes),)
    rest = tree_nodes - w0
    base, extra = divmod(rest, depth - 1)
    widths = [w0] + [base + (1 if d >= (depth - 1) - extra else 0) for d in range(depth - 1)]
    return tuple(widths)


TINY_LLAMA = ModelShape(
    name="tiny-llama-fp32", num_layers=2, hidden=256, num_heads=4, num_kv_heads=2, head_dim=64,
    intermediate=688, vocab=1024, rms_eps=1e-5, rope_theta=1e4, weight_format="dense",
    dtype="float32", feature_layers=(1, 2, 2),
)
LLAMA2_7B_NF4 = ModelShape(
    name="llama2-7b-nf4", num_layers=32, hidden=4096, num_heads=32, num_kv_heads=32, head_dim=128,
    intermediate=11008, vocab=32000, rms_eps=1e-5, rope_theta=1e4, weight_format="nf4",
    dtype="bfloat16", feature_layers=(8, 18, 30),
)
QWEN25_14B_FP16 = ModelShape(
    name="qwen2.5-14b-fp16", num_layers=48, hidden=5120, num_heads=40, num_kv_heads=8, head_dim=128,
    intermediate=13824, vocab=152064, rms_eps=1e-6, rope_theta=1e6, qkv_bias=True,
    weight_format="dense", dtype="float16", feature_layers=(12, 26, 46),
)
QWEN25_14B_NF4 = replace(QWEN25_14B_FP16, name="qwen2.5-14b-nf4", weight_format="nf4", dtype="bfloat16")

WORKLOADS: dict[str, PassWorkload] = {
    "tiny-fp32-T8-P64": PassWorkload(
        "tiny-fp32-T8-P64", TINY_LLAMA, prefix_len=64, tree_nodes=8, depth=4, top_k=2,
        widths=width_schedule(8, 4, 2)),
    "llama2-7b-nf4-T26-P2048": PassWorkload(
        "llama2-7b-nf4-T26-P2048", LLAMA2_7B_NF4, prefix_len=2048, tree_nodes=26, depth=5, top_k=4,
        widths=width_schedule(26, 5, 4)),
    "qwen2.5-14b-fp16-T26-P4096": PassWorkload(
        "qwen2.5-14b-fp16-T26-P4096", QWEN25_14B_FP16, prefix_len=4096, tree_nodes=26, depth=5,
        top_k=4, widths=width_schedule(26, 5, 4)),
    "llama2-7b-nf4-T64-P8192": PassWorkload(
        "llama2-7b-nf4-T64-P8192", LLAMA2_7B_NF4, prefix_len=8192, tree_nodes=64, depth=6, top_k=8,
        widths=width_schedule(64, 6, 8)),
    "qwen2.5-14b-nf4-B8-T26": PassWorkload(
        "qwen2.5-14b-nf4-B8-T26", QWEN25_14B_NF4, prefix_len=4096, prefix_min=512, tree_nodes=26,
        depth=5, top_k=4, widths=width_schedule(26, 5, 4), batch=8),
}


def algorithmic_bytes(shape: ModelShape, prefix_lens: list[int], tree_nodes: int) -> int:
    """HBM bytes one verification pass must move at minimum.

    Every weight, KV row and output is counted once with no temporaries: NF4
    linears at 0.5 B/param plus 2 B per 64-element absmax block, dense linears
    at the storage width, bf16/fp16/fp32 embeddings rows and lm_head at the
    compute width, the cached prefix read once, the T new K/V rows written once,
    and the logits, fused features and embedding rows of the T nodes.
    """
    esz = {"float32": 4, "bfloat16": 2, "float16": 2}[shape.dtype]
    L, H = shape.num_layers, shape.hidden
    nk = sum(n * k for _, n, k in shape.linear_shapes())
    if shape.weight_format == "nf4":
        lin = nk // 2 + (nk // 64) * 2
    else:
        lin = nk * esz
    lin *= L
    bias = L * (shape.q_dim + 2 * shape.kv_dim) * esz if shape.qkv_bias else 0
    norms = (2 * L + 1) * H * esz
    lm_head = shape.vocab * H * esz
    kv_row = L * 2 * shape.kv_dim * esz
    t_tot = tree_nodes * len(prefix_lens)
    kv_read = sum(prefix_lens) * kv_row
    kv_write = t_tot * kv_row
    outs = t_tot * (shape.vocab + 3 * H + H) * esz
    return lin + bias + norms + lm_head + kv_read + kv_write + outs
