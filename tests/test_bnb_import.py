"""bitsandbytes NF4 checkpoint import: host-side parsing, its errors, and the
oracle's double-quantised absmax (no GPU)."""
import json

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from parallel_eagle_amd import bnb
from tests import bnb_checkpoint as bc


def _linear(n=64, k=256, seed=0, nested=False):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.02
    packed, absmax16 = onf4.quantize(w)
    a32 = bc.fp32_absmax(absmax16, rng)
    sd, eff = bc.linear_entries("blk.lin.", packed, a32, nested)
    return sd, packed, a32, eff


@pytest.mark.parametrize("nested", [False, True])
def test_read_linear4bit_round_trips_the_serialized_state(nested):
    sd, packed, a32, eff = _linear(nested=nested)
    lin = bnb.read_linear4bit(sd, "blk.lin.")
    assert (lin.n, lin.k) == (64, 256)
    assert np.array_equal(lin.packed.numpy(), packed)
    assert lin.nested == nested
    if nested:
        assert lin.absmax.dtype == torch.uint8 and lin.nested_blocksize == bc.NESTED_BLOCK
        got = onf4.absmax_from_double_quant(lin.absmax.numpy(), lin.nested_code.numpy(), lin.nested_absmax.numpy(),
                                            lin.nested_blocksize, lin.nested_offset)
        assert np.array_equal(got.view(np.uint32), eff.reshape(-1).view(np.uint32))
        # the double quantisation is close to the fp32 absmax it stands for
        assert np.max(np.abs(got - a32) / np.abs(a32)) < 0.05
    else:
        assert np.array_equal(lin.absmax.numpy().view(np.uint32), a32.view(np.uint32))


def _mutate_state(sd, **changes):
    key = "blk.lin.weight.quant_state.bitsandbytes__nf4"
    qs = json.loads(bytes(sd[key].tolist()).decode())
    qs.update(changes)
    out = dict(sd)
    out[key] = torch.tensor(list(json.dumps(qs).encode()), dtype=torch.uint8)
    return out


@pytest.mark.parametrize("case", ["fp4", "block128", "shape", "quant_map", "missing", "absmax_dtype", "garbled",
                                  "nested_short", "fp16_compute", "no_compute_dtype"])
def test_read_linear4bit_rejects_what_the_kernels_cannot_run(case):
    sd, *_ = _linear(nested=case == "nested_short")
    if case == "fp4":
        sd = _mutate_state(sd, quant_type="fp4")
    elif case == "block128":
        sd = _mutate_state(sd, blocksize=128)
    elif case == "shape":
        sd = _mutate_state(sd, shape=[64, 512])
    elif case == "quant_map":
        qm = sd["blk.lin.weight.quant_map"].clone()
        qm[3] = qm[3] + 1e-7
        sd["blk.lin.weight.quant_map"] = qm
    elif case == "missing":
        del sd["blk.lin.weight.absmax"]
    elif case == "absmax_dtype":
        sd["blk.lin.weight.absmax"] = sd["blk.lin.weight.absmax"].to(torch.float16)
    elif case == "garbled":
        sd["blk.lin.weight.quant_state.bitsandbytes__nf4"] = torch.tensor([0xff, 0xfe, 0x00], dtype=torch.uint8)
    elif case == "nested_short":
        sd["blk.lin.weight.nested_absmax"] = sd["blk.lin.weight.nested_absmax"][:0]
    elif case == "fp16_compute":
        # quantised for an fp16 model: running it in bf16 would change its logits
        sd = _mutate_state(sd, dtype="float16")
    elif case == "no_compute_dtype":
        sd = _mutate_state(sd, dtype="")
    with pytest.raises(bnb.CheckpointError):
        bnb.read_linear4bit(sd, "blk.lin.")


def test_torch_prefixed_compute_dtype_is_accepted():
    sd, *_ = _linear()
    lin = bnb.read_linear4bit(_mutate_state(sd, dtype="torch.bfloat16"), "blk.lin.")
    assert (lin.n, lin.k) == (64, 256)


def test_fp16_dense_tensors_of_an_nf4_checkpoint_are_refused():
    """The embedding, norms and lm_head of an fp16 checkpoint name an fp16 model
    (the reference computes in the embedding's dtype, src/pe/target.py:89)."""
    from parallel_eagle_amd.config import ModelShape
    shape = ModelShape(name="t", num_layers=1, hidden=256, num_heads=2, num_kv_heads=2, head_dim=128,
                       intermediate=256, vocab=64, weight_format="nf4")
    sd = {"model.embed_tokens.weight": torch.zeros(64, 256, dtype=torch.float16)}
    with pytest.raises(bnb.CheckpointError, match="bfloat16"):
        bnb.weights_from_state_dict(shape, sd, device="cpu")


def test_nf4_code_book_of_the_importer_is_the_oracles():
    assert np.array_equal(bnb.NF4_CODE.view(np.uint32), onf4.NF4_TABLE.astype(np.float32).view(np.uint32))


def test_double_quant_absmax_exact_where_fp32_is_exact():
    # code values and scales that are small dyadic rationals: every product and
    # sum is representable, so the result is the exact value
    code = (np.arange(256, dtype=np.float32) - 128) / np.float32(64)
    q = np.arange(512, dtype=np.int64) % 256
    nested = np.array([0.5, 4.0], dtype=np.float32)
    got = onf4.absmax_from_double_quant(q.astype(np.uint8), code, nested, 256, 0.25)
    want = code[q].astype(np.float64) * nested[np.arange(512) // 256].astype(np.float64) + 0.25
    assert np.array_equal(got.astype(np.float64), want)


def test_double_quant_absmax_is_two_roundings_not_a_fused_multiply_add():
    rng = np.random.default_rng(3)
    code = np.sort(rng.uniform(-1, 1, 256).astype(np.float32))
    n = 1 << 16
    q = rng.integers(0, 256, n).astype(np.uint8)
    nested = rng.uniform(0.5, 2, n // 256).astype(np.float32)
    offset = np.float32(0.3)
    got = onf4.absmax_from_double_quant(q, code, nested, 256, float(offset))
    prod64 = code[q].astype(np.float64) * nested[np.arange(n) // 256].astype(np.float64)  # exact (24 + 24 bits)
    two_step = (prod64.astype(np.float32).astype(np.float64) + np.float64(offset)).astype(np.float32)
    fused = (prod64 + np.float64(offset)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), two_step.view(np.uint32))
    # the sample holds inputs where a fused multiply-add would round differently
    assert np.count_nonzero(two_step != fused) > 0
    # and the error is that of two roundings: half an ulp of the product plus
    # half an ulp of the result
    exact = prod64 + np.float64(offset)
    bound = 0.5 * np.spacing(np.abs(prod64.astype(np.float32))).astype(np.float64) + \
        0.5 * np.spacing(np.abs(got)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
