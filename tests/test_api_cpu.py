"""Host logic of the public API, runnable without a GPU: validation and its
error types/messages (reference tests/test_padding.py, tests/test_dtype.py),
meta-device shapes (tests/test_fake_tensor.py), the mask cache
(tests/test_cache.py), and the absence of any CPU fallback."""

from __future__ import annotations

import pytest
import torch

import crumpet_amd
from crumpet_amd.cache import clear_mask_cache, get_or_compute_mask, make_mask_key, mask_cache_info


def test_invalid_divisibility_fails_clearly():
    x = torch.randn((1, 15, 14, 14, 4))
    with pytest.raises(ValueError, match="divisible"):
        crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3))


def test_invalid_shift_fails_clearly():
    x = torch.randn((1, 14, 14, 14, 4))
    with pytest.raises(ValueError, match="shift_size"):
        crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (7, 0, 0))


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


def test_cache_hit_and_miss():
    clear_mask_cache()
    calls = {"n": 0}
    key = make_mask_key(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float32, "cpu")

    def compute():
        calls["n"] += 1
        return torch.zeros((1,), dtype=torch.float32)

    a = get_or_compute_mask(key, compute)
    b = get_or_compute_mask(key, compute)
    assert a is b
    assert calls["n"] == 1
    assert mask_cache_info()["entries"] == 1
    clear_mask_cache()


def test_cache_disabled(monkeypatch):
    clear_mask_cache()
    monkeypatch.setenv("CRUMPET_DISABLE_MASK_CACHE", "1")
    key = make_mask_key(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float32, "cpu")
    a = get_or_compute_mask(key, lambda: torch.zeros((1,)))
    b = get_or_compute_mask(key, lambda: torch.ones((1,)))
    assert not torch.equal(a, b)


def test_cache_byte_cap_and_lru(monkeypatch):
    clear_mask_cache()
    monkeypatch.setenv("CRUMPET_MASK_CACHE_MAX_BYTES", "1")
    key = make_mask_key(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float32, "cpu")
    get_or_compute_mask(key, lambda: torch.zeros((2,), dtype=torch.float32))
    assert mask_cache_info()["entries"] == 0
    monkeypatch.setenv("CRUMPET_MASK_CACHE_MAX_BYTES", "1000")
    monkeypatch.setenv("CRUMPET_MASK_CACHE_SIZE", "2")
    keys = [make_mask_key(7 * (i + 1), 7, 7, (7, 7, 7), (3, 3, 3), torch.float32, "cpu") for i in range(3)]
    for i, k in enumerate(keys):
        get_or_compute_mask(k, lambda i=i: torch.full((4,), float(i)))
    info = mask_cache_info()
    assert info["entries"] == 2 and info["bytes"] == 32
    # the first key was evicted: recomputing gives a new value
    assert get_or_compute_mask(keys[0], lambda: torch.full((4,), 9.0))[0] == 9.0
    clear_mask_cache()
