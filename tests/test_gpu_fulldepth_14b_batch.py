"""The batched workload at full depth against batch-1 oracle runs.

Eight sequences, each a 26-node depth-5 tree over its own random prefix drawn
from [512, 4096], through the Qwen2.5-14B-shaped NF4 model at full depth (48
layers, GQA 40/8 with q/k/v bias, vocabulary 152064) in one batched pass
(208 rows), one batched walk and one ragged commit. Each sequence is checked
against the oracle's batch-1 restatement of the reference step
(src/pe/target.py:203-224, src/pe/decode/verify.py:104-125,
src/pe/target.py:194-201): logits, fused features and every layer's appended
K/V rows within the parity rule of test_gpu_target._close, acceptance exact
or a near tie of the deciding row, the ragged commit bit for bit.

Host memory: the oracle's dequantised bf16 weights (about 30 GB), their fp32
copy (about 59 GB) and the prefixes' K/V; a module of its own, so that no
other module's full-size model is held at the same time.
"""

import pytest

from parallel_eagle_amd import synth
from parallel_eagle_amd.config import QWEN25_14B_NF4, WORKLOADS
from tests.test_gpu_batch import STREAM_BATCH_PREFIX, _batch_case, _check_sequences

pytestmark = pytest.mark.gpu


@pytest.mark.timeout(900)
def test_batched_workload_at_full_depth_against_the_oracle():
    wl = WORKLOADS["qwen2.5-14b-nf4-B8-T26"]
    prefixes = (synth.uniform_int(5, STREAM_BATCH_PREFIX, wl.batch, wl.prefix_len - wl.prefix_min + 1)
                + wl.prefix_min).tolist()
    spec = [(wl.depth, wl.widths, wl.top_k)] * wl.batch
    c = _batch_case(QWEN25_14B_NF4, 5, prefixes, spec, plant=lambda b: 1 + b % 4)
    assert c["trees"].M == 208
    verdicts = _check_sequences(QWEN25_14B_NF4, c)
    print("prefixes", prefixes, "verdicts", verdicts, "accepted", [len(r[0]) for r in c["res"]])
    for v in verdicts:
        assert v == "exact" or v.startswith("near-tie")
