"""CPU oracle for the tree-verification pass — TEST INFRASTRUCTURE ONLY.

This package restates the reference's algorithm on the CPU so the HIP path can
be checked against it. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import it, and only as the checker (or the
timed CPU baseline); the product package ``parallel_eagle_amd`` never imports,
calls or falls back to anything here.

Modules and what pins each one (details in each module's docstring):

- ``masks``   tree_depths / tree_allow_mask / tree_position_ids / to_additive_bias
              (src/pe/masks.py:29-33,118-156); pinned by the reference's known
              answer (tests/test_masks.py:55-73) and brute-force ancestor
              enumeration.
- ``verify``  accept_tree_cached / accept_tree_greedy (src/pe/decode/verify.py:35-57,
              104-125); pinned by brute force over small trees and logits.
- ``tree``    the beam of propose_tree (src/pe/decode/tree.py:34-55) with per-depth
              widths; pinned by hand-checked cases and its constant-width reduction.
- ``nf4``     NF4 code book, logical packing, quantise and dequantise (the
              bitsandbytes format read at src/pe/target.py:55-62); pinned by the
              published table's invariants and a closed-form reconstruction.
- ``model``   the Llama/Qwen2 forward of TargetModel.forward_cached
              (src/pe/target.py:203-224 -> HF modeling_llama.py / modeling_qwen2.py);
              pinned bit-for-bit against transformers' own LlamaForCausalLM /
              Qwen2ForCausalLM run on the same weights.
"""
