"""Pins of the fused-block oracle (oracle.window_qkv / window_proj / round_to /
layer_norm) against independent constructions: torch's own conversions,
LayerNorm, padding and Linear on the CPU, and the scalar C partition /
unpartition.  The reference has no such function (it composes norm1, F.pad,
the partition op and nn.Linear: torch-ext/crumpet/monai_patch.py:79-111 and
:153-197), so every check here is against library routines or invariants.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import seeded

CASES = [  # (B, D, H, W, C), ws, ss
    ((2, 12, 12, 12, 16), (7, 7, 7), (3, 3, 3)),  # padded to 14^3, shifted
    ((1, 7, 9, 5, 32), (7, 3, 5), (2, 1, 0)),  # non-cubic, one axis padded
    ((1, 6, 6, 6, 48), (6, 6, 6), (0, 0, 0)),  # MONAI stage-3 rule, no shift
]


def _pad(x: torch.Tensor, ws) -> torch.Tensor:
    D, H, W = x.shape[1:4]
    pd, ph, pw = ((w - d % w) % w for d, w in zip((D, H, W), ws))
    return F.pad(x, (0, 0, 0, pw, 0, ph, 0, pd))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_round_to_matches_torch_casts(oracle, dtype):
    g = torch.Generator().manual_seed(11)
    a = torch.randn(20000, generator=g, dtype=torch.float64) * torch.logspace(-6, 4, 20000, dtype=torch.float64)
    want = a.to(torch.float32).to(getattr(torch, dtype)).double().numpy()
    np.testing.assert_array_equal(oracle.round_to(a.numpy(), dtype), want)


def test_layer_norm_matches_torch(oracle):
    x = seeded((3, 5, 48), torch.float64, 12) * 3.0 + 2.0
    w = seeded((48,), torch.float64, 13)
    b = seeded((48,), torch.float64, 14)
    want = F.layer_norm(x, (48,), w, b, eps=1e-5).numpy()
    np.testing.assert_allclose(oracle.layer_norm(x.numpy(), w.numpy(), b.numpy(), 1e-5), want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("case", CASES, ids=["pad-shift", "noncubic", "ws6"])
def test_window_qkv_identity_is_padded_partition(oracle, case):
    """Identity weight, no norm: the zero-padded volume, window-partitioned
    by the C oracle."""
    shape, ws, ss = case
    C = shape[-1]
    x = seeded(shape, torch.float32, 20)
    got = oracle.window_qkv(x.numpy(), ws, ss, np.eye(C), None, normalize=False, dtype="float32")
    xp = _pad(x, ws)
    want = oracle.shift_partition(xp.numpy(), ws, ss)
    np.testing.assert_array_equal(got, want.astype(np.float64))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
@pytest.mark.parametrize("case", CASES, ids=["pad-shift", "noncubic", "ws6"])
def test_window_qkv_matches_torch_chain(oracle, case, dtype):
    """torch LayerNorm -> cast (the autocast rounding) -> F.pad -> C-oracle
    partition -> torch Linear in float64 -> cast."""
    shape, ws, ss = case
    C = shape[-1]
    td = getattr(torch, dtype)
    x = seeded(shape, torch.float32, 21) * 2.0 + 0.5
    gw = seeded((C,), torch.float32, 22) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 23) * 0.1
    lin = torch.nn.Linear(C, 3 * C)
    with torch.no_grad():
        lin.weight.copy_(seeded((3 * C, C), torch.float32, 24) / C ** 0.5)
        lin.bias.copy_(seeded((3 * C,), torch.float32, 25) * 0.1)
    wq, bq = lin.weight.detach().to(td).double(), lin.bias.detach().to(td).double()
    got = oracle.window_qkv(x.numpy(), ws, ss, wq.numpy(), bq.numpy(), gw.numpy(), gb.numpy(), 1e-5, True, dtype)

    a = F.layer_norm(x.double(), (C,), gw.double(), gb.double(), eps=1e-5).to(torch.float32).to(td).double()
    win = torch.from_numpy(oracle.shift_partition(_pad(a, ws).numpy(), ws, ss))
    want = F.linear(win, wq, bq).to(torch.float32).to(td).double().numpy()
    # float64 vs float64-then-float32 rounding of the LN output can differ by
    # one ulp of `dtype` near a rounding boundary; everything else is exact
    ulp = {"float16": 2 ** -10, "bfloat16": 2 ** -7, "float32": 2 ** -23}[dtype]
    np.testing.assert_allclose(got, want, rtol=4 * ulp, atol=4 * ulp)


def test_window_qkv_padding_projects_to_bias(oracle):
    shape, ws, ss = CASES[0]
    C = shape[-1]
    x = seeded(shape, torch.float32, 26)
    w = seeded((32, C), torch.float32, 27).double().numpy()
    b = seeded((32,), torch.float32, 28).double().numpy()
    got = oracle.window_qkv(x.numpy(), ws, ss, w, b, dtype="float32")
    # tokens whose shifted source lies in the padding: mark them through a
    # partition of an indicator volume
    ind = np.zeros(tuple(shape[:4]) + (1,), dtype=np.float32)
    ind[...] = 1.0
    inside = oracle.shift_partition(_pad(torch.from_numpy(ind), ws).numpy(), ws, ss)[..., 0] > 0
    assert (~inside).any() and inside.any()
    np.testing.assert_array_equal(got[~inside], np.broadcast_to(oracle.round_to(b, "float32"), got[~inside].shape))


@pytest.mark.parametrize("case", CASES, ids=["pad-shift", "noncubic", "ws6"])
def test_window_proj_identity_is_cropped_unpartition(oracle, case):
    shape, ws, ss = case
    B, D, H, W, C = shape
    Dp, Hp, Wp = (-(-d // w) * w for d, w in zip((D, H, W), ws))
    nwin = B * (Dp // ws[0]) * (Hp // ws[1]) * (Wp // ws[2])
    win = seeded((nwin, ws[0] * ws[1] * ws[2], C), torch.float32, 30).numpy()
    got = oracle.window_proj(win, B, D, H, W, ws, ss, np.eye(C), None, "float32")
    full = oracle.unshift_unpartition(win, B, Dp, Hp, Wp, C, ws, ss)
    np.testing.assert_array_equal(got, full[:, :D, :H, :W].astype(np.float64))


@pytest.mark.parametrize("case", CASES, ids=["pad-shift", "noncubic", "ws6"])
def test_window_proj_inverts_window_qkv(oracle, case):
    shape, ws, ss = case
    B, D, H, W, C = shape
    x = seeded(shape, torch.float32, 31).numpy()
    win = oracle.window_qkv(x, ws, ss, np.eye(C), None, normalize=False, dtype="float32")
    back = oracle.window_proj(win, B, D, H, W, ws, ss, np.eye(C), None, "float32")
    np.testing.assert_array_equal(back, x.astype(np.float64))
