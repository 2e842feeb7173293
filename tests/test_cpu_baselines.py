"""The CPU baselines bench.py times are the reference's eager constructions:
pin them to the oracle bit for bit on small shapes (CPU only)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from crumpet_amd import swin_unetr_compat as sw  # noqa: E402


@pytest.mark.parametrize("dims,ws,ss", [((14, 14, 14), (7, 7, 7), (3, 3, 3)),
                                        ((12, 8, 6), (4, 4, 3), (2, 1, 1)),
                                        ((6, 6, 6), (3, 3, 3), (0, 1, 0))])
@pytest.mark.parametrize("dtype,name", [(torch.float16, "float16"), (torch.bfloat16, "bfloat16"),
                                        (torch.float32, "float32")])
def test_torch_mask_constructions_match_oracle(oracle, dims, ws, ss, dtype, name):
    want = oracle.attn_mask_bits(*dims, ws, ss, name)
    got_where = bench.cpu_mask_where(*dims, ws, ss, dtype)
    got_slices = sw.compute_mask(dims, ws, ss, "cpu").to(dtype)
    bits = {2: torch.int16, 4: torch.int32}[got_where.element_size()]
    for got in (got_where, got_slices):
        arr = got.contiguous().view(bits).numpy().view(want.dtype)
        assert np.array_equal(arr, want)
