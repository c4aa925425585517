"""Device-resident target weights in the layouts the HIP kernels stream.

The reference's frozen target is an HF causal LM whose linears are bf16/fp16
``nn.Linear`` or bitsandbytes NF4 ``Linear4bit`` (src/pe/target.py:32-38,80-101).
Here the same weights live on the device, repacked once at load time:

- q, k, v concatenated along N (one GEMM, one RoPE/KV-append pass),
- gate and up interleaved in 32-row tiles so one workgroup owns the gate and up
  columns of the same outputs and applies SwiGLU in its epilogue,
- the intermediate size padded with zero rows/columns to the GEMM's K granule,
- 16-bit and NF4 matrices repacked to the MFMA-tiled layouts of pe_format.hip
  (fp32 matrices stay row-major for the VALU path),
- a RoPE cos/sin table for every position, computed with HF's fp32 formula
  (modeling_llama.py:93-127) and rounded to the compute dtype.

Weights come either from the counter-based generator on the device
(``synthetic``) or from a dict of host tensors (``from_weights``).
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _lib, ops, synth
from .config import ModelShape

TORCH_DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
NF4_ZERO_BYTE = 0x77  # two code-7 (0.0) nibbles


def rope_table(head_dim: int, theta: float, max_pos: int, dtype: torch.dtype) -> torch.Tensor:
    """[2][max_pos][head_dim] cos, sin for positions 0..max_pos-1.

    Same ops as HF LlamaRotaryEmbedding.forward in fp32, evaluated in chunks of
    128 positions so each cos/sin call runs one vectorised chunk like HF's
    per-forward call does.
    """
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    out = torch.empty((2, max_pos, head_dim), dtype=dtype)
    step = 128
    for p0 in range(0, max_pos, step):
        pos = torch.arange(p0, min(max_pos, p0 + step)).reshape(1, -1)
        inv_e = inv[None, :, None].float().expand(1, -1, 1)
        freqs = (inv_e.float() @ pos[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        out[0, p0:p0 + pos.shape[1]] = (emb.cos() * 1.0).to(dtype)[0]
        out[1, p0:p0 + pos.shape[1]] = (emb.sin() * 1.0).to(dtype)[0]
    return out


def padded_intermediate(shape: ModelShape) -> int:
    g = 128 if (shape.weight_format == "nf4" or shape.dtype != "float32") else 32
    return (shape.intermediate + g - 1) // g * g


class DeviceModel:
    """Repacked weights + the pe_model_desc descriptor pointing at them."""

    def __init__(self, shape: ModelShape, device: torch.device | str = "cuda"):
        self.shape = shape
        self.device = torch.device(device)
        self.dtype = TORCH_DTYPES[shape.dtype]
        self.nf4 = shape.weight_format == "nf4"
        self.absmax_dtype = None  # fp16 (the quantiser's) or fp32 (bitsandbytes checkpoints); set by the first layer
        if self.nf4 and self.dtype != torch.bfloat16:
            raise ValueError("NF4 linears compute in bfloat16")
        self.ipad = padded_intermediate(shape)
        # 16-bit models with 128-dim heads run the fused pass, whose q/k/v GEMM
        # applies RoPE in its epilogue: rows of w_qkv in RoPE-paired tile order.
        self.qkv_paired = self.dtype != torch.float32 and shape.head_dim == 128
        self.layers: list[dict] = []
        self.logical: list[dict] | None = None  # per-layer host-exportable logical weights
        self.embed = None
        self.final_norm = None
        self.lm_head = None  # tiled (16-bit) / row-major (fp32)
        self.lm_head_logical = None
        self.cos_sin = None
        # rounding of the per-layer RMSNorms (PE_NORM_*): HF's for a target; the
        # drafter's layer stack rounds once (src/pe/nn.py:22-26)
        self.norm_mode = _lib.PE_NORM_HF
        # attention arithmetic (PE_ATTN_*): torch SDPA's for a target, the
        # drafter's explicit softmax (src/pe/nn.py:84-87) for its layer stack
        self.attn_mode = _lib.PE_ATTN_SDPA
        self._desc = None
        self._keep = []

    # ------------------------------------------------------------ construction
    @classmethod
    def synthetic(cls, shape: ModelShape, seed: int, device="cuda", keep_logical: bool = False,
                  norm_noise: float = 0.0) -> "DeviceModel":
        """Weights ~ the counter-based N(0, init_std) on the device; NF4 linears are
        quantised from fp32 draws. Norm weights are 1 (+ optional noise)."""
        self = cls(shape, device)
        s, dev, dt = shape, self.device, self.dtype
        self.embed = ops.fill_normal(torch.empty((s.vocab, s.hidden), dtype=dt, device=dev), seed,
                                     synth.STREAM_EMBED, s.init_std)
        self.final_norm = self._norm(seed, 0, 2, norm_noise)
        lm = ops.fill_normal(torch.empty((s.vocab, s.hidden), dtype=dt, device=dev), seed, synth.STREAM_LM_HEAD,
                             s.init_std)
        self._set_lm_head(lm, keep_logical)
        self.logical = [] if keep_logical else None
        for li in range(s.num_layers):
            lin = {}
            for name, n, k in s.linear_shapes():
                sid = synth.layer_stream(li, name)
                if self.nf4:
                    w = ops.fill_normal(torch.empty((n, k), dtype=torch.float32, device=dev), seed, sid, s.init_std)
                    lin[name] = ops.nf4_quantize(w)
                    del w
                else:
                    lin[name] = ops.fill_normal(torch.empty((n, k), dtype=dt, device=dev), seed, sid, s.init_std)
            if s.qkv_bias:
                for name, n in (("q_bias", s.q_dim), ("k_bias", s.kv_dim), ("v_bias", s.kv_dim)):
                    lin[name] = ops.fill_normal(torch.empty(n, dtype=dt, device=dev), seed,
                                                synth.layer_stream(li, name), s.init_std)
            lin["attn_norm"] = self._norm(seed, li, 0, norm_noise)
            lin["mlp_norm"] = self._norm(seed, li, 1, norm_noise)
            self._add_layer(lin, keep_logical)
        self._finish()
        return self

    @classmethod
    def from_weights(cls, shape: ModelShape, weights: dict, device="cuda", keep_logical: bool = False):
        """weights: the oracle's dict layout (host tensors; NF4 linears as
        ("nf4", packed uint8 [N][K/2], absmax fp16 or fp32 [N][K/64]))."""
        self = cls(shape, device)
        dev, dt = self.device, self.dtype

        def up(x):
            if isinstance(x, tuple) and x[0] == "nf4":
                return (torch.as_tensor(x[1]).to(dev).contiguous(), torch.as_tensor(x[2]).to(dev).contiguous())
            return torch.as_tensor(x).to(device=dev, dtype=dt).contiguous()

        self.embed = up(weights["embed"])
        self.final_norm = up(weights["final_norm"])
        self._set_lm_head(up(weights["lm_head"]), keep_logical)
        self.logical = [] if keep_logical else None
        for lw in weights["layers"]:
            self._add_layer({k: up(v) for k, v in lw.items()}, keep_logical)
        self._finish()
        return self

    def _norm(self, seed, layer, which, noise):
        n = torch.ones(self.shape.hidden, dtype=torch.float32, device=self.device)
        if noise:
            n += ops.fill_normal(torch.empty_like(n), seed, 900000 + 4 * layer + which, noise)
        return n.to(self.dtype)

    def _set_lm_head(self, lm: torch.Tensor, keep_logical: bool):
        self.lm_head_logical = lm
        self.lm_head = ops.dense_repack(lm) if self.dtype != torch.float32 else lm.contiguous()

    def _qkv_row_order(self, device) -> torch.Tensor | None:
        """Row gather for PE_QKV_ROPE_PAIRED: within each head, 32-row tiles in the
        order [0,32) [hd/2, hd/2+32) [32,64) [hd/2+32, hd/2+64) ...; None if plain."""
        if not self.qkv_paired:
            return None
        s = self.shape
        hd, units = s.head_dim, s.num_heads + 2 * s.num_kv_heads
        within = torch.cat([torch.cat([torch.arange(32 * j, 32 * j + 32),
                                       torch.arange(hd // 2 + 32 * j, hd // 2 + 32 * j + 32)])
                            for j in range(hd // 64)])
        order = (torch.arange(units)[:, None] * hd + within[None, :]).reshape(-1)
        return order.to(device)

    def _add_layer(self, lin: dict, keep_logical: bool):
        s = self.shape
        out = {"attn_norm": lin["attn_norm"], "mlp_norm": lin["mlp_norm"]}
        if self.nf4:
            adt = lin["q"][1].dtype
            if self.absmax_dtype is None:
                self.absmax_dtype = adt
            if any(lin[nm][1].dtype != self.absmax_dtype for nm in ("q", "k", "v", "o", "gate", "up", "down")):
                raise ValueError("every NF4 linear of a model needs the same absmax dtype (fp16 or fp32)")
            qkv_p = torch.cat([lin["q"][0], lin["k"][0], lin["v"][0]], 0).contiguous()
            qkv_a = torch.cat([lin["q"][1], lin["k"][1], lin["v"][1]], 0).contiguous()
            order = self._qkv_row_order(qkv_p.device)
            if order is not None:
                qkv_p, qkv_a = qkv_p[order].contiguous(), qkv_a[order].contiguous()
            out["w_qkv"], out["a_qkv"] = ops.nf4_repack(qkv_p, qkv_a)
            out["w_o"], out["a_o"] = ops.nf4_repack(lin["o"][0], lin["o"][1])
            gp, ga = self._interleave_nf4(lin["gate"], lin["up"])
            out["w_gu"], out["a_gu"] = ops.nf4_repack(gp, ga)
            dp, da = self._pad_k_nf4(lin["down"])
            out["w_down"], out["a_down"] = ops.nf4_repack(dp, da)
        else:
            qkv = torch.cat([lin["q"], lin["k"], lin["v"]], 0).contiguous()
            order = self._qkv_row_order(qkv.device)
            if order is not None:
                qkv = qkv[order].contiguous()
            out["w_qkv"] = self._tile(qkv)
            out["w_o"] = self._tile(lin["o"])
            out["w_gu"] = self._tile(self._interleave_dense(lin["gate"], lin["up"]))
            out["w_down"] = self._tile(self._pad_k_dense(lin["down"]))
        if s.qkv_bias:
            out["b_qkv"] = torch.cat([lin["q_bias"], lin["k_bias"], lin["v_bias"]]).contiguous()
        self.layers.append(out)
        if keep_logical:
            self.logical.append(lin)

    def _tile(self, w: torch.Tensor) -> torch.Tensor:
        return ops.dense_repack(w) if self.dtype != torch.float32 else w.contiguous()

    def _interleave_dense(self, g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
        ip, k = self.ipad, g.shape[1]
        gp = torch.zeros((ip, k), dtype=g.dtype, device=g.device)
        upd = torch.zeros((ip, k), dtype=u.dtype, device=u.device)
        gp[: g.shape[0]] = g
        upd[: u.shape[0]] = u
        return torch.stack([gp.view(ip // 32, 32, k), upd.view(ip // 32, 32, k)], 1).reshape(2 * ip, k).contiguous()

    def _interleave_nf4(self, g: tuple, u: tuple):
        ip = self.ipad
        kh, ka = g[0].shape[1], g[1].shape[1]
        gp = torch.full((ip, kh), NF4_ZERO_BYTE, dtype=torch.uint8, device=g[0].device)
        upk = torch.full((ip, kh), NF4_ZERO_BYTE, dtype=torch.uint8, device=g[0].device)
        ga = torch.zeros((ip, ka), dtype=g[1].dtype, device=g[0].device)
        ua = torch.zeros((ip, ka), dtype=u[1].dtype, device=g[0].device)
        gp[: g[0].shape[0]] = g[0]
        upk[: u[0].shape[0]] = u[0]
        ga[: g[1].shape[0]] = g[1]
        ua[: u[1].shape[0]] = u[1]
        p = torch.stack([gp.view(ip // 32, 32, kh), upk.view(ip // 32, 32, kh)], 1).reshape(2 * ip, kh)
        a = torch.stack([ga.view(ip // 32, 32, ka), ua.view(ip // 32, 32, ka)], 1).reshape(2 * ip, ka)
        return p.contiguous(), a.contiguous()

    def _pad_k_dense(self, d: torch.Tensor) -> torch.Tensor:
        if d.shape[1] == self.ipad:
            return d.contiguous()
        out = torch.zeros((d.shape[0], self.ipad), dtype=d.dtype, device=d.device)
        out[:, : d.shape[1]] = d
        return out

    def _pad_k_nf4(self, d: tuple):
        if d[0].shape[1] * 2 == self.ipad:
            return d[0].contiguous(), d[1].contiguous()
        p = torch.full((d[0].shape[0], self.ipad // 2), NF4_ZERO_BYTE, dtype=torch.uint8, device=d[0].device)
        a = torch.zeros((d[0].shape[0], self.ipad // 64), dtype=d[1].dtype, device=d[0].device)
        p[:, : d[0].shape[1]] = d[0]
        a[:, : d[1].shape[1]] = d[1]
        return p, a

    def _finish(self):
        s = self.shape
        self.cos_sin = rope_table(s.head_dim, s.rope_theta, s.max_positions, self.dtype).to(self.device)
        torch.cuda.synchronize(self.device)
        self._desc = None

    # ------------------------------------------------------------ descriptor
    def desc(self) -> _lib.ModelDesc:
        if self._desc is not None:
            return self._desc
        s = self.shape
        L = s.num_layers
        arr = C.c_void_p * L

        def parr(key):
            a = arr(*[(ly[key].data_ptr() if ly.get(key) is not None else None) for ly in self.layers])
            self._keep.append(a)
            return C.cast(a, C.POINTER(C.c_void_p))

        d = _lib.ModelDesc()
        d.num_layers, d.hidden, d.num_heads, d.num_kv_heads = L, s.hidden, s.num_heads, s.num_kv_heads
        d.head_dim, d.intermediate, d.vocab, d.intermediate_padded = s.head_dim, s.intermediate, s.vocab, self.ipad
        d.dtype = ops.dcode(self.dtype)
        if not self.nf4:
            d.weight_format = _lib.PE_WFMT_DENSE
        elif self.absmax_dtype == torch.float32:
            d.weight_format = _lib.PE_WFMT_NF4_F32ABS
        else:
            d.weight_format = _lib.PE_WFMT_NF4
        d.qkv_layout = _lib.PE_QKV_ROPE_PAIRED if self.qkv_paired else _lib.PE_QKV_PLAIN
        d.rms_eps = s.rms_eps
        d.norm_mode = self.norm_mode
        d.embed_rows = self.embed.shape[0]
        d.attn_mode = self.attn_mode
        d.max_positions = s.max_positions
        d.embed, d.final_norm = self.embed.data_ptr(), self.final_norm.data_ptr()
        d.lm_head, d.rope_cos_sin = self.lm_head.data_ptr(), self.cos_sin.data_ptr()
        d.attn_norm, d.mlp_norm = parr("attn_norm"), parr("mlp_norm")
        d.w_qkv, d.a_qkv, d.b_qkv = parr("w_qkv"), parr("a_qkv"), parr("b_qkv")
        d.w_o, d.a_o = parr("w_o"), parr("a_o")
        d.w_gu, d.a_gu = parr("w_gu"), parr("a_gu")
        d.w_down, d.a_down = parr("w_down"), parr("a_down")
        self._desc = d
        return d

    def workspace_bytes(self, m: int, kv_len: int) -> int:
        return int(_lib.load().pe_forward_workspace_bytes(C.byref(self.desc()), m, kv_len))

    # ------------------------------------------------------------ export for the checker
    def host_weights(self) -> dict:
        """Host copy in the oracle's dict layout (requires keep_logical=True)."""
        if self.logical is None:
            raise RuntimeError("model was built without keep_logical=True")

        def down(x):
            if isinstance(x, tuple):
                return ("nf4", x[0].cpu().numpy(), x[1].cpu().numpy())
            return x.cpu()

        layers = [{k: down(v) for k, v in lin.items()} for lin in self.logical]
        return {"embed": self.embed.cpu(), "final_norm": self.final_norm.cpu(),
                "lm_head": self.lm_head_logical.cpu(), "layers": layers}

    def weight_bytes(self) -> int:
        tot = 0
        for ly in self.layers:
            for v in ly.values():
                if isinstance(v, torch.Tensor):
                    tot += v.numel() * v.element_size()
        return tot
