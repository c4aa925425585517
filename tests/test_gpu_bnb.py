"""bitsandbytes NF4 checkpoints on the GPU: the double-quantised absmax, the
fp32-absmax repack / dequant / GEMM, and a 7B-width model loaded from a
serialized state dict, each against the oracle."""
import json

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4
from parallel_eagle_amd import _lib, ops, synth
from parallel_eagle_amd.config import LLAMA2_7B_NF4, WORKLOADS
from parallel_eagle_amd.target import TargetModel
from tests import bnb_checkpoint as bc
from tests.test_gpu_target import _run_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("n,nbs", [(1, 256), (1000, 256), (65536, 256), (4099, 64)])
def test_absmax_dequant_bit_exact(n, nbs):
    rng = np.random.default_rng(n)
    code = np.sort(rng.uniform(-1, 1, 256).astype(np.float32))
    q = rng.integers(0, 256, n).astype(np.uint8)
    nested = rng.uniform(1e-3, 2, -(-n // nbs)).astype(np.float32)
    offset = float(np.float32(rng.uniform(-0.5, 0.5)))
    ref = onf4.absmax_from_double_quant(q, code, nested, nbs, offset)
    got = ops.nf4_absmax_dequant(torch.from_numpy(q).to(DEV), torch.from_numpy(code).to(DEV),
                                 torch.from_numpy(nested).to(DEV), nbs, offset).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _f32_weight(n, k, seed):
    w = synth.normal(seed, 41, n * k, 0.02).reshape(n, k)
    p, a16 = onf4.quantize(w)
    a32 = bc.fp32_absmax(a16, np.random.default_rng(seed)).reshape(a16.shape)
    assert not np.array_equal(a32.astype(np.float16).astype(np.float32), a32)  # really fp32
    tiled, tabs = ops.nf4_repack(torch.from_numpy(p).to(DEV), torch.from_numpy(a32).to(DEV))
    assert tabs.dtype == torch.float32
    return p, a32, (tiled, tabs)


@pytest.mark.parametrize("n,k", [(64, 128), (256, 1024), (4096, 4096)])
def test_f32abs_repack_dequant_bit_exact(n, k):
    p, a32, (tiled, tabs) = _f32_weight(n, k, seed=n + k)
    got = ops.nf4_dequant(tiled, tabs, n, k).cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, onf4.dequantize(p, a32))


@pytest.mark.parametrize("m", [1, 26, 64, 130])
@pytest.mark.parametrize("n,k", [(256, 1024), (4096, 512), (12288, 4096)])
def test_f32abs_gemm_matches_dequant_then_linear(m, n, k):
    p, a32, w = _f32_weight(n, k, seed=m + n + k)
    wdq = onf4.dequantize_torch(p, a32)
    x = torch.from_numpy(synth.normal(m, 42, m * k, 1.0).reshape(m, k)).to(torch.bfloat16)
    y = ops.linear(x.to(DEV), n, nf4=w).cpu().float()
    ref32 = x.float() @ wdq.float().t()
    err = (y - ref32).abs()
    assert torch.all(err <= 2.0 ** -8 * ref32.abs() + 1e-4 * (1 + ref32.abs()) * (k / 1024)), err.max()


@pytest.mark.parametrize("nested,P", [(False, 48), (True, 48), (True, 300)])
def test_llama7b_width_from_bnb_state_dict(nested, P):
    """A 2-layer 7B-width model saved as bitsandbytes Params4bit (fp32 absmax, or
    uint8 absmax with a nested state) runs the fp32-absmax kernels and matches the
    oracle on the weights the importer decodes."""
    wl = WORKLOADS["llama2-7b-nf4-T26-P2048"]
    shape = LLAMA2_7B_NF4.reduced(2, feature_layers=(1, 2, 2))
    seed = 4
    src = TargetModel.synthetic(shape, seed=seed, device=DEV, keep_logical=True, norm_noise=0.1)
    sd = bc.model_state_dict(shape, src.model.host_weights(), nested, seed)
    del src
    torch.cuda.empty_cache()
    tm = TargetModel.from_bnb_state_dict(shape, sd, DEV, keep_logical=True, cache_capacity=P + 128)
    assert tm.model.desc().weight_format == _lib.PE_WFMT_NF4_F32ABS
    # the importer's absmax is the fp32 decode of what was saved
    lw = tm.model.host_weights()["layers"][0]
    prefix = "model.layers.0.self_attn.q_proj.weight."
    if nested:
        qs = json.loads(bytes(sd[prefix + "quant_state.bitsandbytes__nf4"].tolist()).decode())
        want = onf4.absmax_from_double_quant(sd[prefix + "absmax"].numpy(), sd[prefix + "nested_quant_map"].numpy(),
                                             sd[prefix + "nested_absmax"].numpy(), qs["nested_blocksize"],
                                             qs["nested_offset"])
    else:
        want = sd[prefix + "absmax"].numpy()
    assert np.array_equal(np.asarray(lw["q"][2]).reshape(-1).view(np.uint32), want.reshape(-1).view(np.uint32))
    v, n, err = _run_case(shape, seed, P, wl.depth, wl.widths, wl.top_k, plant=lambda s: 1 + s % wl.depth,
                          tol=2e-2, tm=tm)
    print(f"nested={nested}: {v}, accepted {n}, max |dlogit| {err:.3g}")
