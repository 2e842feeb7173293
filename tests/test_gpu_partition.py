"""Bit-exact parity of the HIP shift-partition / unshift-unpartition kernels
with the CPU oracle (oracle/crumpet_oracle.c), on seeded inputs.

Cases follow the reference tests (tests/test_correctness.py:61-97,
tests/test_dtype.py:13-25, tests/test_backward.py:14-24) plus the BASELINE
shapes (config 1 at 98^3 and the stage 1-3 block shapes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import crumpet_amd
from helpers import raw, seeded

pytestmark = pytest.mark.gpu

CASES = [
    # (B, D, H, W, C, ws, ss)
    (2, 14, 14, 14, 13, (7, 7, 7), (3, 3, 3)),
    (2, 14, 14, 14, 48, (7, 7, 7), (0, 0, 0)),
    (2, 8, 8, 8, 7, (4, 4, 4), (2, 2, 2)),
    (1, 8, 8, 8, 4, (4, 4, 4), (2, 2, 2)),
    (1, 6, 4, 2, 3, (2, 2, 2), (1, 1, 1)),
    (1, 6, 8, 4, 5, (3, 4, 2), (2, 1, 1)),
    (2, 7, 7, 14, 4, (7, 7, 7), (3, 0, 5)),
    (4, 28, 28, 28, 96, (7, 7, 7), (3, 3, 3)),
    (4, 14, 14, 14, 192, (7, 7, 7), (3, 3, 3)),
    (4, 7, 7, 7, 384, (7, 7, 7), (0, 0, 0)),
    (4, 6, 6, 6, 384, (6, 6, 6), (0, 0, 0)),
    (1, 49, 49, 49, 48, (7, 7, 7), (3, 3, 3)),
    (1, 14, 14, 14, 1, (7, 7, 7), (3, 3, 3)),
]

DTS = [torch.float32, torch.float16, torch.bfloat16]


def _check_case(oracle, dev, case, dtype, seed=0):
    B, D, H, W, C, ws, ss = case
    print(f"case {case} {dtype}", flush=True)
    x = seeded((B, D, H, W, C), dtype, seed)
    xr = raw(x)
    ref = oracle.shift_partition(xr, ws, ss)
    xd = x.to(dev)
    win = crumpet_amd.fused_shift_partition_3d(xd, ws, ss)
    assert win.shape == ref.shape and win.dtype == dtype
    assert np.array_equal(raw(win), ref)
    back = crumpet_amd.fused_unshift_unpartition_3d(win, B, D, H, W, C, ws, ss)
    assert np.array_equal(raw(back), xr)
    # unpartition of an independent tensor vs the oracle's inverse
    w2 = seeded(tuple(win.shape), dtype, seed + 1)
    ref2 = oracle.unshift_unpartition(raw(w2), B, D, H, W, C, ws, ss)
    got2 = crumpet_amd.fused_unshift_unpartition_3d(w2.to(dev), B, D, H, W, C, ws, ss)
    assert np.array_equal(raw(got2), ref2)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", DTS)
def test_partition_unpartition_bit_exact(oracle, dev, case, dtype):
    _check_case(oracle, dev, case, dtype)


def test_config1_round_trip_98_fp16(oracle, dev):
    """[1, 98^3, 48] fp16, ws 7, ss 3 -> [2744, 343, 48] and back."""
    _check_case(oracle, dev, (1, 98, 98, 98, 48, (7, 7, 7), (3, 3, 3)), torch.float16, seed=7)


def test_strided_input_is_made_contiguous(oracle, dev):
    base = seeded((1, 14, 14, 14, 96), torch.float16, 3)
    x = base[..., ::2]  # non-contiguous view, C = 48
    ref = oracle.shift_partition(raw(x), (7, 7, 7), (3, 3, 3))
    got = crumpet_amd.fused_shift_partition_3d(base.to(dev)[..., ::2], (7, 7, 7), (3, 3, 3))
    assert np.array_equal(raw(got), ref)


def test_misaligned_base_pointer(oracle, dev):
    """A view starting 2 bytes into its storage forces the narrow-vector path."""
    flat = seeded((1 + 8 * 8 * 8 * 8,), torch.float16, 5)
    x = flat[1:].view(1, 8, 8, 8, 8)
    ref = oracle.shift_partition(raw(x), (4, 4, 4), (2, 2, 2))
    xd = flat.to(dev)[1:].view(1, 8, 8, 8, 8)
    assert xd.data_ptr() % 16 != 0
    got = crumpet_amd.fused_shift_partition_3d(xd, (4, 4, 4), (2, 2, 2))
    assert np.array_equal(raw(got), ref)


@pytest.mark.parametrize("ss", [(3, 3, 3), (0, 0, 0)])
def test_autograd_backward_matches_inverse(oracle, dev, ss):
    """tests/test_backward.py:14-24: grad of partition = unpartition of the grad."""
    x = seeded((1, 14, 14, 14, 5), torch.float32, 11).to(dev).requires_grad_(True)
    y = crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), ss)
    g = seeded(tuple(y.shape), torch.float32, 12)
    y.backward(g.to(dev))
    ref = oracle.unshift_unpartition(g.numpy(), 1, 14, 14, 14, 5, (7, 7, 7), ss)
    assert np.array_equal(x.grad.cpu().numpy(), ref)

    w = seeded((8, 343, 5), torch.float32, 13).to(dev).requires_grad_(True)
    z = crumpet_amd.fused_unshift_unpartition_3d(w, 1, 14, 14, 14, 5, (7, 7, 7), ss)
    gz = seeded(tuple(z.shape), torch.float32, 14)
    z.backward(gz.to(dev))
    refw = oracle.shift_partition(gz.numpy(), (7, 7, 7), ss)
    assert np.array_equal(w.grad.cpu().numpy(), refw)


def test_raw_dispatcher_ops(oracle, dev):
    """The five crumpet_ops schemas of torch-ext/torch_binding.cpp:16-31."""
    ops = torch.ops.crumpet_ops
    x = seeded((2, 8, 8, 8, 6), torch.float16, 21)
    ref = oracle.shift_partition(raw(x), (4, 4, 4), (1, 2, 3))
    out = torch.empty((16, 64, 6), dtype=torch.float16, device=dev)
    ops.fused_shift_partition_3d(out, x.to(dev), 4, 4, 4, 1, 2, 3)
    assert np.array_equal(raw(out), ref)
    back = torch.empty((2, 8, 8, 8, 6), dtype=torch.float16, device=dev)
    ops.fused_unshift_unpartition_3d(back, out, 2, 8, 8, 8, 6, 4, 4, 4, 1, 2, 3)
    assert np.array_equal(raw(back), raw(x))
    gx = torch.empty_like(back)
    ops.fused_shift_partition_3d_backward(gx, out, 2, 8, 8, 8, 6, 4, 4, 4, 1, 2, 3)
    assert np.array_equal(raw(gx), raw(x))
    gw = torch.empty_like(out)
    ops.fused_unshift_unpartition_3d_backward(gw, back, 4, 4, 4, 1, 2, 3)
    assert np.array_equal(raw(gw), ref)


def test_empty_and_invalid(dev):
    x = torch.empty((0, 14, 14, 14, 4), device=dev, dtype=torch.float16)
    assert crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3)).shape == (0, 343, 4)
    with pytest.raises(ValueError, match="divisible"):
        crumpet_amd.fused_shift_partition_3d(torch.zeros((1, 15, 14, 14, 4), device=dev), (7, 7, 7), (3, 3, 3))
    with pytest.raises(ValueError, match="shift_size"):
        crumpet_amd.fused_shift_partition_3d(torch.zeros((1, 14, 14, 14, 4), device=dev), (7, 7, 7), (7, 0, 0))
    with pytest.raises(RuntimeError):
        out = torch.empty((7, 343, 4), device=dev)
        torch.ops.crumpet_ops.fused_shift_partition_3d(out, torch.zeros((1, 14, 14, 14, 4), device=dev), 7, 7, 7, 3, 3, 3)
