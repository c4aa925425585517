"""The 14B fp16 workload at full depth against the oracle.

The dense fp16 Qwen2.5-14B-shaped model (48 layers, hidden 5120, GQA 40/8
heads with q/k/v bias, intermediate 13824, vocabulary 152064) scores a
26-node tree over a random 4095-row prefix plus each seed's root token
(P = 4096), through forward_cached -> accept_tree_cached -> gather_cache, on
the device and through the oracle restatement of target.py:203-224 and
verify.py:104-125 (the HF Qwen2 forward in fp16 on the CPU, and an fp32
evaluation of the same weights as the yardstick of both fp16 evaluations).
Logits, fused features and every layer's appended K/V rows are held to the
parity rule of test_gpu_target._close, the committed path to the oracle's or
a bounded near tie, the compaction bit for bit.

Host memory: the fp16 weights (about 30 GB) and their fp32 copy (about 59 GB)
for the module's lifetime; it is a module of its own so that no other
module's full-size model is held at the same time.
"""

import pytest

from parallel_eagle_amd.config import QWEN25_14B_FP16, WORKLOADS
from tests.test_gpu_target import Prepared, _report, _run_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def full_14b():
    return Prepared(QWEN25_14B_FP16, 0, P=4095, kv_seed=4096, cache_capacity=4096 + 64)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("seed", WORKLOADS["qwen2.5-14b-fp16-T26-P4096"].seeds)
def test_qwen14b_fp16_full_depth_against_the_oracle(full_14b, seed):
    wl = WORKLOADS["qwen2.5-14b-fp16-T26-P4096"]
    det = {}
    v, n, err = _run_case(QWEN25_14B_FP16, seed, None, wl.depth, wl.widths, wl.top_k,
                          plant=lambda s: 1 + s % wl.depth, tol=2e-2, prep=full_14b, details=det)
    _report("14b-fp16-48layer-P4096", det)
    assert v == "exact" or v.startswith("near-tie")
