"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

The CPU half checks that the oracle still reproduces the committed vectors
(so a change to the oracle cannot silently move the bar); the GPU half runs
the kernels on the same inputs: bit-exact for the partition round trip and
the masks, within 2e-3 of the fp64 output for fp16 attention.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / name, allow_pickle=False)


def test_oracle_reproduces_partition_fixture(oracle):
    g = _load("partition_f16.npz")
    win = oracle.shift_partition(g["x"], tuple(g["ws"]), tuple(g["ss"]))
    np.testing.assert_array_equal(win, g["windows"])
    B, D, H, W, C = g["x"].shape
    back = oracle.unshift_unpartition(win, B, D, H, W, C, tuple(g["ws"]), tuple(g["ss"]))
    np.testing.assert_array_equal(back, g["x"])


def test_oracle_reproduces_mask_fixture(oracle):
    g = _load("mask_bits.npz")
    for i in range(3):
        dims, ws, ss = tuple(g[f"dims{i}"]), tuple(g[f"ws{i}"]), tuple(g[f"ss{i}"])
        for dt in ("float16", "bfloat16", "float32"):
            np.testing.assert_array_equal(oracle.attn_mask_bits(*dims, ws, ss, dt), g[f"mask{i}_{dt}"])


def test_oracle_reproduces_attention_fixture(oracle):
    g = _load("attention_f16.npz")
    q, k, v, bias, mask = (g[n].view(np.float16) for n in ("q", "k", "v", "bias", "mask"))
    ref = oracle.attention(q, k, v, bias, mask, g["boundary"], scale=float(g["scale"]), dtype=np.float64)
    np.testing.assert_allclose(ref, g["out"], rtol=0, atol=1e-12)


@pytest.mark.gpu
def test_kernels_match_partition_fixture(dev):
    import crumpet_amd

    g = _load("partition_f16.npz")
    x = torch.from_numpy(g["x"].view(np.float16).copy()).to(dev)
    ws, ss = tuple(int(v) for v in g["ws"]), tuple(int(v) for v in g["ss"])
    win = crumpet_amd.fused_shift_partition_3d(x, ws, ss)
    np.testing.assert_array_equal(win.cpu().view(torch.int16).numpy().view(np.uint16), g["windows"])
    B, D, H, W, C = x.shape
    back = crumpet_amd.fused_unshift_unpartition_3d(win, B, D, H, W, C, ws, ss)
    assert torch.equal(back, x)


@pytest.mark.gpu
def test_kernels_match_mask_fixture(dev):
    import crumpet_amd

    g = _load("mask_bits.npz")
    for i in range(3):
        dims, ws, ss = (tuple(int(v) for v in g[f"{n}{i}"]) for n in ("dims", "ws", "ss"))
        for dt, tdt, view in (("float16", torch.float16, torch.int16), ("bfloat16", torch.bfloat16, torch.int16),
                              ("float32", torch.float32, torch.int32)):
            crumpet_amd.clear_mask_cache()
            m = crumpet_amd.compute_attn_mask_3d(*dims, ws, ss, tdt, dev)
            bits = m.cpu().view(view).numpy().view(g[f"mask{i}_{dt}"].dtype)
            np.testing.assert_array_equal(bits, g[f"mask{i}_{dt}"])


@pytest.mark.gpu
def test_kernel_matches_attention_fixture(dev):
    from crumpet_amd.fused_attention import fused_swin_attention

    g = _load("attention_f16.npz")
    q, k, v, bias, mask = (torch.from_numpy(g[n].view(np.float16).copy()).to(dev)
                           for n in ("q", "k", "v", "bias", "mask"))
    bnd = torch.from_numpy(g["boundary"].copy()).to(dev)
    # mask [3, N, N] with B = 6: window b reads mask[b mod 3] (the raw op's nW-periodic form)
    from crumpet_amd import _native

    out = torch.empty_like(q)
    _native.ops().fused_swin_attention(out, q, k, v, bias, mask, bnd, float(g["scale"]))
    err = np.abs(out.float().cpu().numpy() - g["out"]).max()
    assert err < 2e-3, err
    # the reference wrapper with a per-window mask [B, N, N] gives the same result
    full = mask[torch.arange(q.shape[0], device=dev) % mask.shape[0]].contiguous()
    out2 = fused_swin_attention(q, k, v, bias, full, bnd, scale=float(g["scale"]))
    assert torch.equal(out2, out)
