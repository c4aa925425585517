"""The 16-bit parity rule of the end-to-end GPU tests (test_gpu_target._close)
on constructed tensors, so that its behaviour is pinned on the CPU: what it
accepts (the bound itself; a device as close to the fp32 evaluation as the
oracle) and what it rejects (a device further from fp32 in L2 or in the
count of elements outside the band, or with its arguments swapped)."""

import torch

from tests.test_gpu_target import _close

TOL = 2e-2


def _case(n=100_000, seed=0):
    g = torch.Generator().manual_seed(seed)
    ref = torch.randn(n, generator=g) * 4.0
    noise = lambda s: torch.randn(n, generator=g) * s  # noqa: E731
    return ref, noise


def test_every_element_within_the_bound_of_the_oracle_passes():
    ref, noise = _case()
    orc = ref + noise(0.2)          # far from fp32 on many elements
    dev = orc + noise(0.002)        # but within 2e-2 of the oracle everywhere
    ok, _ = _close(dev, orc, TOL, ref)
    assert ok


def test_a_device_as_close_to_fp32_as_the_oracle_passes():
    ref, noise = _case(seed=1)
    orc = ref + noise(0.05)
    dev = ref + noise(0.05)         # an independent evaluation of the same quality
    ok, _ = _close(dev, orc, TOL, ref)
    assert ok


def test_a_device_further_from_fp32_in_l2_fails():
    ref, noise = _case(seed=2)
    orc = ref + noise(0.05)
    dev = ref + noise(0.06)         # 20% further in L2
    ok, _ = _close(dev, orc, TOL, ref)
    assert not ok


def test_a_device_with_more_elements_outside_the_band_fails_at_equal_l2():
    ref, noise = _case(seed=3)
    band = TOL + TOL * ref.abs()
    orc = ref + noise(0.05)
    err = noise(0.045)
    # push the elements in the outer half of the band just past its edge: more
    # elements outside at about the same L2 distance
    edge = (err.abs() > 0.5 * band) & (err.abs() <= band)
    err[edge] = torch.sign(err[edge]) * 1.05 * band[edge]
    dev = ref + err
    e_dev = (dev - ref).norm() / ref.norm()
    e_orc = (orc - ref).norm() / ref.norm()
    out_dev = int(((dev - ref).abs() > band).sum())
    out_orc = int(((orc - ref).abs() > band).sum())
    assert e_dev <= 1.1 * e_orc and out_dev > 1.3 * out_orc  # the count, not L2, decides
    ok, _ = _close(dev, orc, TOL, ref)
    assert not ok


def test_swapping_device_and_oracle_is_not_symmetric_when_one_is_worse():
    ref, noise = _case(seed=4)
    good = ref + noise(0.03)
    bad = ref + noise(0.045)
    assert _close(good, bad, TOL, ref)[0]
    assert not _close(bad, good, TOL, ref)[0]


def test_fp32_requires_every_element_within_the_bound():
    ref, noise = _case(seed=5)
    dev = ref + noise(1e-3)
    assert _close(dev, ref, 1e-2)[0]
    dev[7] += 1.0
    assert not _close(dev, ref, 1e-2)[0]
