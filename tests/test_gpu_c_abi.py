"""Parity through the raw C ABI (include/crumpet_hip.h) called with ctypes:
device pointers from torch allocations, the current HIP stream, explicit
sizes.  This is the boundary a non-Python caller binds."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import CODE, bias_from_table, c_abi, raw, seeded, strides, trunc_normal_table

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_c_abi_partition_unpartition(oracle, dev):
    lib = c_abi()
    B, D, H, W, C = 2, 14, 14, 14, 48
    x = seeded((B, D, H, W, C), torch.float16, 1)
    xd = x.to(dev)
    out = torch.empty((B * 8, 343, C), dtype=torch.float16, device=dev)
    st = lib.crumpet_shift_partition_3d(out.data_ptr(), xd.data_ptr(), B, D, H, W, C, 2,
                                        7, 7, 7, 3, 3, 3, _stream())
    assert st == 0, lib.crumpet_last_error()
    back = torch.empty_like(xd)
    st = lib.crumpet_unshift_unpartition_3d(back.data_ptr(), out.data_ptr(), B, D, H, W, C, 2,
                                            7, 7, 7, 3, 3, 3, _stream())
    assert st == 0, lib.crumpet_last_error()
    torch.cuda.synchronize()
    assert np.array_equal(raw(out), oracle.shift_partition(raw(x), (7, 7, 7), (3, 3, 3)))
    assert np.array_equal(raw(back), raw(x))
    g = torch.empty_like(xd)
    assert lib.crumpet_shift_partition_3d_backward(g.data_ptr(), out.data_ptr(), B, D, H, W, C, 2,
                                                   7, 7, 7, 3, 3, 3, _stream()) == 0
    gw = torch.empty_like(out)
    assert lib.crumpet_unshift_unpartition_3d_backward(gw.data_ptr(), xd.data_ptr(), B, D, H, W, C, 2,
                                                       7, 7, 7, 3, 3, 3, _stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(g, xd) and torch.equal(gw, out)


def test_c_abi_mask(oracle, dev):
    lib = c_abi()
    out = torch.empty((343, 343, 343), dtype=torch.bfloat16, device=dev)
    st = lib.crumpet_compute_attn_mask_3d(out.data_ptr(), CODE[torch.bfloat16], 49, 49, 49,
                                          7, 7, 7, 3, 3, 3, _stream())
    assert st == 0, lib.crumpet_last_error()
    torch.cuda.synchronize()
    ref = oracle.attn_mask_bits(49, 49, 49, (7, 7, 7), (3, 3, 3), "bfloat16")
    assert np.array_equal(raw(out).view(np.uint16), ref)


def test_c_abi_attention(oracle, dev):
    lib = c_abi()
    B, H, N, Dh = 8, 3, 343, 16
    q, k, v = (seeded((B, H, N, Dh), torch.float16, s) for s in (10, 11, 12))
    bias = bias_from_table(trunc_normal_table(2197, H, 13), (7, 7, 7)).half()
    mask = torch.from_numpy(oracle.attn_mask(14, 14, 14, (7, 7, 7), (3, 3, 3), "float16"))
    qd, kd, vd, bd, md = (t.to(dev) for t in (q, k, v, bias, mask))
    out = torch.empty_like(qd)
    st = lib.crumpet_fused_swin_attention(
        out.data_ptr(), strides(out, 4), qd.data_ptr(), strides(qd, 4), kd.data_ptr(), strides(kd, 4),
        vd.data_ptr(), strides(vd, 4), CODE[torch.float16], B, H, N, Dh,
        bd.data_ptr(), CODE[torch.float16], strides(bd, 3),
        md.data_ptr(), CODE[torch.float16], 8, strides(md, 3), None, ctypes.c_float(0.25),
        _stream())
    assert st == 0, lib.crumpet_last_error()
    torch.cuda.synchronize()
    ref = oracle.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), bias.float().numpy(),
                           mask.float().numpy(), None, scale=0.25)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-3

    # the same windows through the geometry entry point (mask derived from the 14^3 volume)
    out2 = torch.empty_like(qd)
    st = lib.crumpet_fused_swin_attention_shifted(
        out2.data_ptr(), strides(out2, 4), qd.data_ptr(), strides(qd, 4), kd.data_ptr(), strides(kd, 4),
        vd.data_ptr(), strides(vd, 4), CODE[torch.float16], B, H, N, Dh,
        bd.data_ptr(), CODE[torch.float16], strides(bd, 3), 14, 14, 14, 7, 7, 7, 3, 3, 3,
        ctypes.c_float(0.25), _stream())
    assert st == 0, lib.crumpet_last_error()
    torch.cuda.synchronize()
    assert np.abs(out2.float().cpu().numpy() - ref).max() <= 2e-3


def test_c_abi_rejects_bad_arguments(dev):
    lib = c_abi()
    x = torch.empty((1, 14, 14, 14, 4), dtype=torch.float16, device=dev)
    st = lib.crumpet_shift_partition_3d(x.data_ptr(), x.data_ptr(), 1, 14, 14, 14, 4, 2,
                                        7, 7, 7, 7, 0, 0, _stream())
    assert st == 1 and b"shift" in lib.crumpet_last_error()
    st = lib.crumpet_compute_attn_mask_3d(x.data_ptr(), 9, 14, 14, 14, 7, 7, 7, 3, 3, 3, _stream())
    assert st == 1


def test_c_abi_window_projections(oracle, dev):
    """crumpet_window_qkv_3d / crumpet_window_proj_3d through the raw C ABI:
    LayerNorm + pad + shift + partition + qkv, then proj + reverse + crop,
    against the oracle chain (4 ulps of fp16)."""
    lib = c_abi()
    B, D, C, ws, ss = 2, 12, 48, (7, 7, 7), (3, 3, 3)
    x = seeded((B, D, D, D, C), torch.float32, 70)
    gw = seeded((C,), torch.float32, 71) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 72) * 0.1
    w = (seeded((3 * C, C), torch.float32, 73) / C ** 0.5).half()
    b = (seeded((3 * C,), torch.float32, 74) * 0.1).half()
    xd, gwd, gbd, wd, bd = (t.to(dev) for t in (x, gw, gb, w, b))
    qkv = torch.empty((B * 8, 343, 3 * C), dtype=torch.float16, device=dev)
    st = lib.crumpet_window_qkv_3d(qkv.data_ptr(), CODE[torch.float16], xd.data_ptr(), CODE[torch.float32],
                                   B, D, D, D, C, 1, gwd.data_ptr(), gbd.data_ptr(), CODE[torch.float32],
                                   ctypes.c_float(1e-5), wd.data_ptr(), bd.data_ptr(), 3 * C, *ws, *ss, _stream())
    assert st == 0, lib.crumpet_last_error()
    wp = (seeded((C, C), torch.float32, 75) / C ** 0.5).half()
    wpd = wp.to(dev)
    y = torch.empty((B, D, D, D, C), dtype=torch.float16, device=dev)
    win = qkv[:, :, :C].contiguous()
    st = lib.crumpet_window_proj_3d(y.data_ptr(), win.data_ptr(), CODE[torch.float16], B, D, D, D, C,
                                    wpd.data_ptr(), None, C, *ws, *ss, _stream())
    assert st == 0, lib.crumpet_last_error()
    torch.cuda.synchronize()
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), b.double().numpy(),
                             gw.double().numpy(), gb.double().numpy(), 1e-5, True, "float16")
    got = qkv.float().cpu().double().numpy()
    assert (np.abs(got - want) <= 4 * 2 ** -10 * np.maximum(np.abs(want), 1.0)).all()
    want_y = oracle.window_proj(win.float().cpu().double().numpy(), B, D, D, D, ws, ss, wp.double().numpy())
    got_y = y.float().cpu().double().numpy()
    assert (np.abs(got_y - want_y) <= 4 * 2 ** -10 * np.maximum(np.abs(want_y), 1.0)).all()
