"""Bit-exact parity of the HIP shifted-window mask kernel with the CPU oracle.

Cases follow tests/test_correctness.py:20-58 of the reference plus the
BASELINE shapes (config 2 at 98^3 and the stage-0 49^3 mask).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import crumpet_amd
from helpers import raw

pytestmark = pytest.mark.gpu

CASES = [
    ((14, 14, 14), (7, 7, 7), (3, 3, 3)),
    ((14, 14, 14), (7, 7, 7), (0, 0, 0)),
    ((8, 8, 8), (4, 4, 4), (2, 2, 2)),
    ((6, 4, 2), (2, 2, 2), (1, 1, 1)),
    ((21, 14, 7), (7, 7, 7), (3, 2, 1)),
    ((12, 8, 6), (4, 4, 3), (1, 0, 2)),
    ((2, 2, 2), (1, 1, 1), (0, 0, 0)),
    ((3, 3, 3), (3, 3, 3), (1, 1, 1)),
    ((49, 49, 49), (7, 7, 7), (3, 3, 3)),
    ((28, 28, 28), (7, 7, 7), (3, 3, 3)),
    ((16, 16, 16), (8, 8, 8), (4, 4, 4)),
]

NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


@pytest.fixture(autouse=True)
def _no_cache(monkeypatch):
    monkeypatch.setenv("CRUMPET_DISABLE_MASK_CACHE", "1")


@pytest.mark.parametrize("shape,ws,ss", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_mask_bit_exact(oracle, dev, shape, ws, ss, dtype):
    print(f"mask {shape} ws={ws} ss={ss} {dtype}", flush=True)
    got = crumpet_amd.compute_attn_mask_3d(*shape, ws, ss, dtype, dev)
    ref = oracle.attn_mask_bits(*shape, ws, ss, NAMES[dtype])
    assert got.shape == ref.shape and got.dtype == dtype
    assert np.array_equal(raw(got).view(ref.dtype), ref)


def test_config2_mask_98_fp16(oracle, dev):
    """[2744, 343, 343] fp16 at D=H=W=98, ws 7, ss 3."""
    got = crumpet_amd.compute_attn_mask_3d(98, 98, 98, (7, 7, 7), (3, 3, 3), torch.float16, dev)
    ref = oracle.attn_mask_bits(98, 98, 98, (7, 7, 7), (3, 3, 3), "float16")
    assert np.array_equal(raw(got).view(np.uint16), ref)


def test_zero_shift_is_zero(dev):
    m = crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (0, 0, 0), torch.float16, dev)
    assert torch.count_nonzero(m).item() == 0


def test_mask_overwrites_stale_memory(oracle, dev):
    """Every element is written (no reliance on zeroed memory)."""
    out = torch.full((8, 343, 343), 7.0, dtype=torch.float16, device=dev)
    torch.ops.crumpet_ops.compute_attn_mask_3d(out, 14, 14, 14, 7, 7, 7, 3, 3, 3)
    ref = oracle.attn_mask_bits(14, 14, 14, (7, 7, 7), (3, 3, 3), "float16")
    assert np.array_equal(raw(out).view(np.uint16), ref)


def test_cache_hit_returns_same_tensor(dev, monkeypatch):
    monkeypatch.setenv("CRUMPET_DISABLE_MASK_CACHE", "0")
    crumpet_amd.clear_mask_cache()
    a = crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float16, dev)
    b = crumpet_amd.compute_attn_mask_3d(14, 14, 14, (7, 7, 7), (3, 3, 3), torch.float16, dev)
    assert a is b
    assert crumpet_amd.mask_cache_info()["entries"] == 1
    crumpet_amd.clear_mask_cache()


def test_large_window_volume_rejected(dev):
    with pytest.raises(RuntimeError, match="1024"):
        crumpet_amd.compute_attn_mask_3d(11, 11, 11, (11, 11, 11), (5, 5, 5), torch.float16, dev)
