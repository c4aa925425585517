"""MI355X-native target tree-verification pass for parallel_eagle.

The reference API is mirrored by:
- ``parallel_eagle_amd.target``: ``TargetModel`` (forward_cached, make_cache,
  gather_cache, forward) and ``TreeKVCache``
- ``parallel_eagle_amd.verify``: ``accept_tree_cached``, ``accept_tree_greedy``
- ``parallel_eagle_amd.masks``: ``tree_depths``, ``tree_allow_mask``,
  ``tree_position_ids``, ``to_additive_bias`` (+ ``tree_ancestor_bits``)

All device work runs in libpe_hip.so (HIP kernels for gfx950, C ABI in
include/pe_hip.h); loading fails loudly if the library has not been built.
"""

__version__ = "0.1.0"
