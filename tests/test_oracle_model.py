"""Pin the CPU oracle's forward against transformers' own models (CPU, no GPU).

The reference's verification forward is transformers' LlamaForCausalLM /
Qwen2ForCausalLM called exactly as TargetModel.forward_cached does
(src/pe/target.py:216-224): a DynamicCache, explicit position ids, a 4-D
additive tree bias and output_hidden_states=True, fused by _fuse
(src/pe/target.py:161-162). Those models are installed third-party code (not
the reference), built here locally with no hub access. The oracle must agree
with them bit for bit: logits, fused features and the cache rows.
"""

import pytest
import torch

from oracle import masks as omasks
from oracle.model import OracleTarget, weights_from_hf
from parallel_eagle_amd.config import ModelShape


def _hf_model(kind: str, shape: ModelShape, seed: int):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    common = dict(
        hidden_size=shape.hidden, num_hidden_layers=shape.num_layers, num_attention_heads=shape.num_heads,
        num_key_value_heads=shape.num_kv_heads, intermediate_size=shape.intermediate, vocab_size=shape.vocab,
        max_position_embeddings=4096, rms_norm_eps=shape.rms_eps, rope_theta=shape.rope_theta,
        tie_word_embeddings=False,
    )
    if kind == "llama":
        model = LlamaForCausalLM(LlamaConfig(**common, head_dim=shape.head_dim))
    else:
        model = Qwen2ForCausalLM(Qwen2Config(**common))
    # non-trivial norm weights and biases so their rounding points are exercised
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
            if name.endswith("bias"):
                p.copy_(0.02 * torch.randn_like(p))
    dt = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}[shape.dtype]
    # from_pretrained(dtype=...) (src/pe/target.py:38) keeps the RoPE inv_freq buffer
    # in fp32; a plain .to(dtype) would round it, so restore it after the cast.
    rot = model.model.rotary_emb
    inv = rot.inv_freq.clone()
    model = model.to(dt).eval()
    rot.inv_freq = inv
    rot.original_inv_freq = inv.clone()
    return model, dt


def _hf_tree_pass(model, prompt, node_tokens, parents, dtype, feature_layers):
    from transformers import DynamicCache

    cache = DynamicCache()
    P = len(prompt)
    with torch.no_grad():
        out = model(input_ids=torch.tensor([prompt]), past_key_values=cache,
                    position_ids=torch.arange(P).unsqueeze(0), use_cache=True, output_hidden_states=True)
        pre_logits = out.logits
        allow = torch.from_numpy(omasks.tree_allow_mask(parents, P))[P:, :]
        bias = omasks.to_additive_bias(allow.numpy(), dtype)
        pos = torch.tensor([omasks.tree_position_ids(parents, P)[P:]])
        out2 = model(input_ids=torch.tensor([node_tokens]), past_key_values=cache, position_ids=pos,
                     attention_mask=bias, use_cache=True, output_hidden_states=True)
    fused = torch.cat([out2.hidden_states[i] for i in feature_layers], dim=-1)
    return pre_logits, out2.logits, fused, cache, bias, pos


CASES = [
    ("llama", ModelShape("t-llama-f32", 2, 128, 4, 2, 32, 176, 512, rms_eps=1e-5, rope_theta=1e4,
                         dtype="float32", feature_layers=(1, 2, 2))),
    ("llama", ModelShape("t-llama-bf16", 3, 128, 4, 4, 32, 192, 512, rms_eps=1e-5, rope_theta=1e4,
                         dtype="bfloat16", feature_layers=(1, 2, 3))),
    ("qwen2", ModelShape("t-qwen-f16", 2, 160, 5, 1, 32, 224, 640, rms_eps=1e-6, rope_theta=1e6,
                         qkv_bias=True, dtype="float16", feature_layers=(0, 1, 2))),
]


# Llama-2-7B's real width (H=4096, 32 heads of 128, I=11008, V=32000) at two
# layers: the GEMM reduction lengths, head count and vocabulary the GPU path
# runs at, in fp32 and in bf16.
WIDE = [
    ("llama", ModelShape("llama7b-width-2l-f32", 2, 4096, 32, 32, 128, 11008, 32000, rms_eps=1e-5, rope_theta=1e4,
                         dtype="float32", feature_layers=(0, 1, 2))),
    ("llama", ModelShape("llama7b-width-2l-bf16", 2, 4096, 32, 32, 128, 11008, 32000, rms_eps=1e-5,
                         rope_theta=1e4, dtype="bfloat16", feature_layers=(0, 1, 2))),
]


@pytest.mark.parametrize("kind,shape", CASES + WIDE, ids=[c[1].name for c in CASES + WIDE])
def test_oracle_matches_transformers(kind, shape):
    model, dt = _hf_model(kind, shape, seed=7)
    prompt = [3, 17, 250, 9, 44, 101, 7, 300, 12, 5, 77]
    parents = [-1, -1, 0, 0, 1, 2, 2, 5]
    node_tokens = [11, 12, 13, 14, 15, 16, 17, 18]
    fl = shape.resolved_feature_layers()
    pre_logits, logits, fused, cache, bias, pos = _hf_tree_pass(model, prompt, node_tokens, parents, dt, fl)

    orc = OracleTarget(shape, weights_from_hf(model, dt))
    P = len(prompt)
    o_pre, _, o_cache = orc.forward(prompt, list(range(P)), None, None)
    o_logits, o_fused, o_cache2 = orc.forward(node_tokens, pos[0].tolist(), o_cache, bias)

    assert torch.equal(o_pre, pre_logits)
    assert torch.equal(o_logits, logits)
    assert torch.equal(o_fused, fused)
    for li, layer in enumerate(cache.layers):
        assert torch.equal(o_cache2[li][0], layer.keys)
        assert torch.equal(o_cache2[li][1], layer.values)


def test_oracle_one_token_continuation_matches_transformers():
    shape = CASES[1][1]
    model, dt = _hf_model("llama", shape, seed=3)
    from transformers import DynamicCache

    prompt = [5, 6, 7, 8, 9]
    cache = DynamicCache()
    with torch.no_grad():
        model(input_ids=torch.tensor([prompt]), past_key_values=cache,
              position_ids=torch.arange(len(prompt)).unsqueeze(0), use_cache=True)
        out = model(input_ids=torch.tensor([[42]]), past_key_values=cache,
                    position_ids=torch.tensor([[len(prompt)]]), use_cache=True)
    orc = OracleTarget(shape, weights_from_hf(model, dt))
    _, _, oc = orc.forward(prompt, list(range(len(prompt))), None, None)
    o_logits, _, _ = orc.forward([42], [len(prompt)], oc, None)
    assert torch.equal(o_logits, out.logits)
