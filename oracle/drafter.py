"""ParallelDrafter.draft_logits restated on the CPU (oracle; test
infrastructure only).

Follows src/pe/drafter.py:126-133 (real_input), :135-138 (mask_input),
:149-160 (forward) and :195-236 (draft_logits), with the layers of
src/pe/nn.py:16-124: the drafter's RMSNorm multiplies by the weight in fp32
and rounds once (nn.py:22-26); RoPE casts cos/sin to the activation dtype
(nn.py:45-49); attention adds the additive bias to QK^T / sqrt(hd) and takes
the softmax in fp32 (nn.py:84-87). The final norm and the lm_head are the
target's (an HF LlamaRMSNorm: the normalised row is rounded before the weight
multiply).

Pinned by tests/test_oracle_pins.py: in fp32 (where the two RMSNorm forms
agree) the layer stack equals the target oracle's forward, itself pinned
against transformers, run on the same rows; the draft mask equals the causal
mask over the p + k - 1 rows, position for position; in_proj of the
concatenation equals the sum of its two column blocks applied separately;
every feature block leaves feat_norm with unit RMS (times the weight).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .model import inv_freq, repeat_kv, rms_norm, rotate_half


def drafter_rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """src/pe/nn.py:22-26: fp32 normalise, fp32 weight multiply, one rounding."""
    dt = x.dtype
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * w.float()).to(dt)


def draft_allow_mask(p: int, k: int) -> torch.Tensor:
    """src/pe/drafter.py:218-224: real rows causal, mask slots see every real row
    and the slots up to their own."""
    m = p + k - 1
    allow = torch.zeros(m, m, dtype=torch.bool)
    allow[:p, :p] = torch.tril(torch.ones(p, p, dtype=torch.bool))
    if k > 1:
        allow[p:, :p] = True
        allow[p:, p:] = torch.tril(torch.ones(k - 1, k - 1, dtype=torch.bool))
    return allow


def draft_positions(p: int, k: int) -> torch.Tensor:
    """src/pe/drafter.py:214-216: 0..p-1, then (p - 1) + d for d = 1..k-1."""
    pos = torch.arange(p + k - 1)
    pos[p:] = (p - 1) + torch.arange(1, k)
    return pos


class OracleDrafter:
    """``shape``: the target's ModelShape (hidden, heads, eps, theta, dtype).
    ``weights``: {"feat_norm" [H], "feat_proj" [H][F], "in_proj" [H][2H],
    "mask_emb" [H], "h_shared" [H], "layers": [{"attn_norm", "mlp_norm", "q", "k",
    "v", "o", "gate", "up", "down"}]} in the compute dtype; ``shared``: the
    target's {"embed", "final_norm", "lm_head"}."""

    def __init__(self, shape, weights: dict, shared: dict, dtype: torch.dtype):
        self.s = shape
        self.w = weights
        self.shared = shared
        self.dtype = dtype
        self.inv = inv_freq(shape.head_dim, shape.rope_theta)

    def real_input(self, ids: torch.Tensor, feats: torch.Tensor) -> torch.Tensor:
        H = self.s.hidden
        emb = self.shared["embed"][ids].to(self.dtype)
        f = feats.to(self.dtype).unflatten(-1, (-1, H))
        f = drafter_rms_norm(f, self.w["feat_norm"], self.s.rms_eps)
        feat = F.linear(f.flatten(-2), self.w["feat_proj"])
        return F.linear(torch.cat([emb, feat], dim=-1), self.w["in_proj"])

    def mask_input(self, n: int) -> torch.Tensor:
        vec = F.linear(torch.cat([self.w["mask_emb"], self.w["h_shared"]], dim=-1), self.w["in_proj"])
        return vec.unsqueeze(0).expand(n, -1)

    def layers_forward(self, x: torch.Tensor, pos: torch.Tensor, allow: torch.Tensor) -> torch.Tensor:
        """src/pe/drafter.py:149-160 without the final norm. x: (m, H)."""
        s, dt = self.s, self.dtype
        m = x.shape[0]
        ang = pos.float()[:, None] * self.inv[None, :]
        emb = torch.cat([ang, ang], dim=-1)
        cos, sin = emb.cos().to(dt), emb.sin().to(dt)
        bias = torch.zeros(m, m, dtype=dt).masked_fill(~allow, torch.finfo(dt).min)
        hd = s.head_dim
        for lw in self.w["layers"]:
            h = drafter_rms_norm(x, lw["attn_norm"], s.rms_eps)
            q = F.linear(h, lw["q"]).view(m, -1, hd).transpose(0, 1)
            k = F.linear(h, lw["k"]).view(m, -1, hd).transpose(0, 1)
            v = F.linear(h, lw["v"]).view(m, -1, hd).transpose(0, 1)
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
            g = s.num_heads // s.num_kv_heads
            k = repeat_kv(k.unsqueeze(0), g)[0]
            v = repeat_kv(v.unsqueeze(0), g)[0]
            sc = torch.matmul(q, k.transpose(-1, -2).contiguous()) / (hd ** 0.5) + bias
            a = torch.softmax(sc.float(), dim=-1).to(dt)
            o = torch.matmul(a, v).transpose(0, 1).reshape(m, -1)
            x = x + F.linear(o, lw["o"])
            h = drafter_rms_norm(x, lw["mlp_norm"], s.rms_eps)
            x = x + F.linear(F.silu(F.linear(h, lw["gate"])) * F.linear(h, lw["up"]), lw["down"])
        return x

    @torch.no_grad()
    def draft_logits(self, ids: torch.Tensor, feats: torch.Tensor, k: int) -> torch.Tensor:
        p = ids.shape[0]
        x = self.real_input(ids, feats)
        if k > 1:
            x = torch.cat([x, self.mask_input(k - 1)], dim=0)
        hidden = self.layers_forward(x, draft_positions(p, k), draft_allow_mask(p, k))
        # the final norm and lm_head act row by row: only the k rows read are computed
        hidden = rms_norm(hidden[p - 1:], self.shared["final_norm"], self.s.rms_eps)
        return F.linear(hidden, self.shared["lm_head"])
