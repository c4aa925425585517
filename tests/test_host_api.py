"""Host-side behaviour of the reference-shaped API that needs no GPU: the cache's
DynamicCache semantics, the guard that stops a captured step from running on
a reallocated cache, and the shared target modules' nn.Module surface."""

import pytest
import torch

from parallel_eagle_amd.config import TINY_LLAMA
from parallel_eagle_amd.target import DeviceLMHead, DeviceRMSNorm, TreeKVCache, VerifyStep


def _cache(cap=16):
    c = TreeKVCache(TINY_LLAMA, torch.float32, "cpu", cap)
    c.seq_len = 10
    return c


def test_crop_keeps_absolute_length_and_negative_trims_from_the_end():
    """HF DynamicCache.crop (cache_utils.py:165-188), as serve.py:186,319 call it."""
    c = _cache()
    c.crop(12)
    assert c.get_seq_length() == 10  # longer than the cache: unchanged
    c.crop(7)
    assert c.get_seq_length() == 7
    c.crop(-2)
    assert c.get_seq_length() == 5
    assert c.layers[1].keys.shape == (1, TINY_LLAMA.num_kv_heads, 5, TINY_LLAMA.head_dim)


def test_growing_the_cache_keeps_rows_and_changes_the_buffers():
    c = _cache()
    c.k[:, :, :10] = torch.randn_like(c.k[:, :, :10])
    before = c.k[:, :, :10].clone()
    b0 = c.buffers()
    c.ensure_capacity(12)
    assert c.buffers() == b0  # fits: nothing moves
    c.ensure_capacity(40)
    assert c.capacity >= 40 and c.buffers() != b0
    assert torch.equal(c.k[:, :, :10], before)


def test_a_step_refuses_a_cache_reallocated_after_it_was_built():
    """A VerifyStep (and its captured graph) holds the K/V pointers and capacity
    it was built with; after the cache grows it must raise, not write through
    freed memory."""
    c = _cache()
    step = VerifyStep.__new__(VerifyStep)
    step.cache = c
    step._buffers = c.buffers()
    step._check_cache()  # unchanged: fine
    c.ensure_capacity(c.capacity + 1)
    with pytest.raises(RuntimeError, match="reallocated"):
        step._check_cache()
    with pytest.raises(RuntimeError, match="reallocated"):
        step.run()


def test_shared_modules_check_to_instead_of_copying():
    w = torch.ones(8)
    norm = DeviceRMSNorm(w, 1e-5)
    assert norm.to("cpu") is norm and norm.to(torch.float32) is norm
    assert norm.weight is w and norm.variance_epsilon == 1e-5
    with pytest.raises(ValueError):
        norm.to(torch.float16)
    # registered nowhere: the reference keeps them out of the drafter's parameters
    assert list(norm.parameters()) == [] and list(norm.buffers()) == []
    head = DeviceLMHead(torch.zeros(4, 8), torch.zeros(32))
    assert head.weight.shape == (4, 8)
    with pytest.raises(ValueError, match="HIP device"):
        norm(torch.ones(2, 8))
