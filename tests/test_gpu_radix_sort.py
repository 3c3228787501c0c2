"""The reverse index's radix sort (bf_radix_sort_keys) against numpy's stable argsort of the same bit
field, for every digit plan it picks: 9-bit digits with 2048-, 4096- and 6144-key tiles, 8-bit digits, one
partial tile, a single-bit field, all 64 bits (sign bit included) and an empty bit range. Keys mix
uniform 64-bit patterns with fields drawn from a steep power law (long runs of one digit, many equal
fields), so stability is checked on ties. Integer work: bit-exact."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _keys(n, b0, b1, seed):
    rng = np.random.default_rng(seed)
    keys = rng.integers(0, 2 ** 63, size=n, dtype=np.uint64) * np.uint64(2) + rng.integers(0, 2, size=n,
                                                                                            dtype=np.uint64)
    bits = b1 - b0
    if bits:
        # half of the keys get a skewed field: a few values hold most of them
        skew = np.floor((2.0 ** bits) * rng.random(n) ** 6).astype(np.uint64)
        skew = np.minimum(skew, np.uint64(2 ** bits - 1)) if bits < 64 else skew
        field_mask = np.uint64(((1 << bits) - 1) << b0) if bits < 64 else np.uint64(2 ** 64 - 1)
        pick = rng.random(n) < 0.5
        keys[pick] = (keys[pick] & ~field_mask) | (skew[pick] << np.uint64(b0))
    return keys


def _expected(keys, b0, b1):
    bits = b1 - b0
    if bits == 0:
        return keys
    field = keys >> np.uint64(b0)
    if bits < 64:
        field = field & np.uint64((1 << bits) - 1)
    return keys[np.argsort(field, kind="stable")]


@pytest.mark.parametrize("n,b0,b1", [
    (1, 0, 5),
    (1000, 3, 21),             # 18 bits: two 9-bit passes, one partial tile
    (823_801, 22, 40),         # the c2 reverse-index shape
    (5_000_000, 10, 28),       # 18 bits past 4M keys: 4096-key tiles
    (34_000_000, 5, 23),       # 18 bits past 32M keys: 6144-key tiles
    (3_000_000, 20, 42),       # 22 bits: three 8-bit passes
    (2_000_000, 0, 27),        # 27 bits: three 9-bit passes
    (300_000, 0, 64),          # every bit, the top one included: eight 8-bit passes
    (70_000, 40, 41),          # a single bit
    (5000, 7, 7),              # an empty range: a copy
])
def test_radix_sort_equals_stable_argsort(hip_device, n, b0, b1):
    from budgetformer_amd import hip_ops
    keys = _keys(n, b0, b1, seed=n + b0)
    got = hip_ops.radix_sort_keys(torch.from_numpy(keys.view(np.int64)).to(hip_device), b0, b1)
    assert np.array_equal(got.cpu().numpy().view(np.uint64), _expected(keys, b0, b1))


def test_radix_sort_empty_input_and_bad_arguments(hip_device):
    from budgetformer_amd import hip_ops
    empty = torch.zeros(0, dtype=torch.int64, device=hip_device)
    assert hip_ops.radix_sort_keys(empty, 0, 20).numel() == 0
    keys = torch.arange(10, dtype=torch.int64, device=hip_device)
    with pytest.raises(ValueError):
        hip_ops.radix_sort_keys(keys, 10, 5)
    with pytest.raises(ValueError):
        hip_ops.radix_sort_keys(keys, 0, 65)
