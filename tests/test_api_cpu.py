"""Host logic of the public API, runnable without a GPU: validation and its
error types/messages, meta-device shapes, the mask cache, and the absence of
any CPU fallback.

Behaviours pinned (the reference tests that hold them):
* a volume not divisible by the window raises ValueError mentioning
  "divisible", and a shift of at least the window raises ValueError
  mentioning "shift_size" (tests/test_padding.py:9-18);
* the mask cache computes once per key and returns the stored object, the
  CRUMPET_DISABLE_MASK_CACHE switch computes every time, and a mask above
  CRUMPET_MASK_CACHE_MAX_BYTES is returned without being stored
  (tests/test_cache.py:13-43);
* dtype errors (tests/test_dtype.py) and meta shapes (tests/test_fake_tensor.py).
"""

from __future__ import annotations

import pytest
import torch

import crumpet_amd
from crumpet_amd.cache import clear_mask_cache, get_or_compute_mask, make_mask_key, mask_cache_info

# (volume shape [B, D, H, W, C], window, shift, message fragment): each breaks
# exactly one rule of the partition's argument checks
_BAD_PARTITIONS = [
    ((2, 21, 14, 13, 6), (7, 7, 7), (2, 2, 2), "divisible"),   # W = 13 on a 7-window
    ((1, 12, 12, 10, 3), (4, 4, 4), (1, 1, 1), "divisible"),   # W = 10 on a 4-window
    ((1, 12, 12, 12, 3), (4, 4, 4), (0, 4, 0), "shift_size"),  # shift equal to the window
    ((3, 10, 10, 10, 2), (5, 5, 5), (1, 6, 2), "shift_size"),  # shift past the window
]


@pytest.mark.parametrize("shape,ws,ss,fragment", _BAD_PARTITIONS)
def test_partition_argument_errors(shape, ws, ss, fragment):
    x = torch.zeros(shape, dtype=torch.float16)
    with pytest.raises(ValueError, match=fragment):
        crumpet_amd.fused_shift_partition_3d(x, ws, ss)


def test_other_validation_errors():
    with pytest.raises(ValueError, match=r"\[B, D, H, W, C\]"):
        crumpet_amd.fused_shift_partition_3d(torch.zeros(14, 14, 14, 4), (7, 7, 7), (3, 3, 3))
    with pytest.raises(ValueError, match="three values"):
        crumpet_amd.fused_shift_partition_3d(torch.zeros(1, 14, 14, 14, 4), (7, 7), (3, 3, 3))
    with pytest.raises(ValueError, match="non-negative"):
        crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (-1, 3, 3), torch.float16, "meta")
    with pytest.raises(TypeError):
        crumpet_amd.fused_shift_partition_3d(torch.zeros((1, 14, 14, 14, 4), dtype=torch.float64),
                                             (7, 7, 7), (3, 3, 3))
    with pytest.raises(TypeError):
        crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.int32, "meta")
    with pytest.raises(ValueError, match="windows must have shape"):
        crumpet_amd.fused_unshift_unpartition_3d(torch.zeros((7, 343, 4)), 1, 14, 14, 14, 4,
                                                 (7, 7, 7), (3, 3, 3))


def test_validated_grid_reuse():
    """The gather wrappers keep each validated window grid: a repeated valid
    geometry returns the same grid, an invalid one raises on every call
    (after a valid call with the same window too), and list arguments, which
    cannot be kept, give an equal grid."""
    from crumpet_amd import _grid

    first = _grid(14, 14, 14, (7, 7, 7), (3, 3, 3))
    assert _grid(14, 14, 14, (7, 7, 7), (3, 3, 3)) is first
    assert _grid(14, 14, 14, [7, 7, 7], [3, 3, 3]) == first
    for _ in range(2):
        with pytest.raises(ValueError, match="divisible"):
            _grid(14, 14, 13, (7, 7, 7), (3, 3, 3))
        with pytest.raises(ValueError, match="shift_size"):
            _grid(14, 14, 14, (7, 7, 7), (3, 7, 3))
    x = torch.empty((2, 14, 14, 14, 48), device="meta", dtype=torch.float16)
    for ws, ss in (((7, 7, 7), (3, 3, 3)), ([7, 7, 7], [3, 3, 3])):
        assert crumpet_amd.fused_shift_partition_3d(x, ws, ss).shape == (16, 343, 48)


def test_meta_shape_propagation():
    x = torch.empty((2, 14, 14, 14, 48), device="meta", dtype=torch.float16)
    windows = crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3))
    assert windows.shape == (16, 343, 48)
    restored = crumpet_amd.fused_unshift_unpartition_3d(windows, 2, 14, 14, 14, 48, (7, 7, 7), (3, 3, 3))
    assert restored.shape == x.shape
    mask = crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float16, "meta")
    assert mask.shape == (8, 343, 343)


def test_no_cpu_fallback():
    """The product path never computes on the CPU: CPU tensors raise."""
    x = torch.randn((1, 14, 14, 14, 4))
    with pytest.raises(RuntimeError, match="HIP"):
        crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3))
    with pytest.raises(RuntimeError, match="HIP"):
        crumpet_amd.fused_unshift_unpartition_3d(torch.zeros((8, 343, 4)), 1, 14, 14, 14, 4,
                                                 (7, 7, 7), (3, 3, 3))
    with pytest.raises(RuntimeError, match="HIP"):
        crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float16, "cpu")


def test_missing_extension_raises(monkeypatch, tmp_path):
    """With the libraries absent the loader reports it (and tries again on
    the next call, so a build in the same process is picked up)."""
    from crumpet_amd import _native

    monkeypatch.setattr(_native, "_ops", None)
    monkeypatch.setattr(_native, "_error", None)
    monkeypatch.setattr(_native, "HIP_LIB", tmp_path / "libcrumpet_hip.so")
    with pytest.raises(RuntimeError, match="not available"):
        _native.ops()
    assert "not built" in _native.load_error()


class _CountingMask:
    """A mask factory that records its calls and returns a distinct tensor per call."""

    def __init__(self, numel=3):
        self.calls = 0
        self.numel = numel

    def __call__(self):
        self.calls += 1
        return torch.full((self.numel,), float(self.calls), dtype=torch.float16)


@pytest.fixture
def empty_cache():
    clear_mask_cache()
    yield
    clear_mask_cache()


def test_cache_computes_once_per_key(empty_cache):
    factory = _CountingMask()
    k1 = make_mask_key(28, 28, 28, (7, 7, 7), (3, 3, 3), torch.float16, "cpu")
    k2 = make_mask_key(28, 28, 28, (7, 7, 7), (0, 0, 0), torch.float16, "cpu")
    first = [get_or_compute_mask(k1, factory) for _ in range(3)]
    assert factory.calls == 1 and all(m is first[0] for m in first)
    other = get_or_compute_mask(k2, factory)  # a different shift is a different key
    assert factory.calls == 2 and other is not first[0]
    info = mask_cache_info()
    assert info["entries"] == 2 and info["bytes"] == 2 * 3 * 2


def test_cache_switch_recomputes(monkeypatch, empty_cache):
    monkeypatch.setenv("CRUMPET_DISABLE_MASK_CACHE", "1")
    factory = _CountingMask()
    key = make_mask_key(21, 14, 7, (7, 7, 7), (3, 3, 3), torch.float16, "cpu")
    values = [get_or_compute_mask(key, factory) for _ in range(2)]
    assert factory.calls == 2
    assert values[0][0].item() == 1.0 and values[1][0].item() == 2.0
    assert mask_cache_info()["entries"] == 0


def test_cache_byte_cap_and_lru(monkeypatch, empty_cache):
    # one 8-element fp16 mask is 16 bytes: above a 15-byte cap it is returned, not stored
    monkeypatch.setenv("CRUMPET_MASK_CACHE_MAX_BYTES", "15")
    big = _CountingMask(numel=8)
    key = make_mask_key(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float16, "cpu")
    assert get_or_compute_mask(key, big).numel() == 8
    assert mask_cache_info()["entries"] == 0
    get_or_compute_mask(key, big)
    assert big.calls == 2
    # two entries at most: a third key evicts the least recently used one
    monkeypatch.setenv("CRUMPET_MASK_CACHE_MAX_BYTES", "4096")
    monkeypatch.setenv("CRUMPET_MASK_CACHE_SIZE", "2")
    small = _CountingMask(numel=4)
    keys = [make_mask_key(7, 7, 7 * (i + 2), (7, 7, 7), (3, 3, 3), torch.float16, "cpu") for i in range(3)]
    get_or_compute_mask(keys[0], small)
    get_or_compute_mask(keys[1], small)
    get_or_compute_mask(keys[0], small)  # touch: keys[1] is now the oldest
    get_or_compute_mask(keys[2], small)
    assert small.calls == 3 and mask_cache_info()["entries"] == 2
    get_or_compute_mask(keys[0], small)  # still cached
    assert small.calls == 3
    get_or_compute_mask(keys[1], small)  # evicted: computed again
    assert small.calls == 4
