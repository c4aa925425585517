"""API compatibility with the reference's verification path, by signature.

tests/golden/ref_signatures.json holds the reference's signatures, read from
its source with ``ast`` (tests/golden/ref_signatures.py). Each of this
package's counterparts must accept every call the reference's callers make:
the same parameters in the same order (``self`` aside; a staticmethod of the
reference is called on the instance by src/pe/serve.py), the same defaults,
and any extra parameter optional and after the reference's own.
"""

import inspect
import json
from pathlib import Path

import pytest

from parallel_eagle_amd import masks, tree, verify
from parallel_eagle_amd.target import TargetModel

REF = json.loads((Path(__file__).resolve().parent / "golden" / "ref_signatures.json").read_text())

# Deliberate differences: the mask helpers default to the HIP device, where
# they build the masks (the reference defaults to "cpu"; its loop always passes
# device=, src/pe/serve.py:291,293; a CPU device is refused, not emulated).
DEFAULT_DIFFERS = {("tree_allow_mask", "device"), ("tree_position_ids", "device")}

OURS = {
    "TargetModel.forward_cached": TargetModel.forward_cached,
    "TargetModel.forward": TargetModel.forward,
    "TargetModel.make_cache": TargetModel.make_cache,
    "TargetModel.gather_cache": TargetModel.gather_cache,
    "TargetModel.get_input_embeddings": TargetModel.get_input_embeddings,
    "TargetModel.get_lm_head": TargetModel.get_lm_head,
    "TargetModel.get_final_norm": TargetModel.get_final_norm,
    "to_additive_bias": masks.to_additive_bias,
    "tree_depths": masks.tree_depths,
    "tree_allow_mask": masks.tree_allow_mask,
    "tree_position_ids": masks.tree_position_ids,
    "accept_tree_cached": verify.accept_tree_cached,
    "accept_tree_greedy": verify.accept_tree_greedy,
    "propose_tree": tree.propose_tree,
}


def test_every_reference_signature_has_a_counterpart():
    assert set(REF) == set(OURS)


@pytest.mark.parametrize("name", sorted(REF))
def test_signature_accepts_the_reference_calls(name):
    ref = REF[name]
    sig = inspect.signature(OURS[name])
    params = list(sig.parameters.values())
    if "." in name and params and params[0].name == "self":
        params = params[1:]
    ref_params = [p for p in ref["params"] if p != "self"]
    ours_pos = [p for p in params if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
    # the reference's positional parameters, by name and in order
    assert [p.name for p in ours_pos[: len(ref_params)]] == ref_params, (name, [p.name for p in params])
    for p in ours_pos[: len(ref_params)]:
        if p.name in ref["defaults"]:
            assert p.default is not inspect.Parameter.empty, (name, p.name)
            want = ref["defaults"][p.name]
            if (name, p.name) not in DEFAULT_DIFFERS and (want is None or isinstance(want, (int, float, str, bool))):
                assert p.default == want, (name, p.name, p.default, want)
        else:
            assert p.default is inspect.Parameter.empty or p.name == "device", (name, p.name)
    # the reference's keyword-only parameters exist here too
    for k in ref["kwonly"]:
        assert k in sig.parameters, (name, k)
    # anything else is optional
    for p in params[len(ref_params):]:
        if p.name in ref["kwonly"] or p.kind in (p.VAR_POSITIONAL, p.VAR_KEYWORD):
            continue
        assert p.default is not inspect.Parameter.empty, (name, p.name, "extra parameters must be optional")
