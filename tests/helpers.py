"""Shared helpers of the test suite (seeded inputs, raw-byte views, C-ABI handle)."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}
CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
TOL = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-4}


def seeded(shape, dtype, seed):
    """N(0, 1) generated on the CPU from a seed, then cast (bit-identical on every box)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def raw(t: torch.Tensor) -> np.ndarray:
    """Raw element bits of a tensor as a numpy integer array (works for bf16)."""
    t = t.detach().cpu().contiguous()
    view = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.view(view).numpy()


def trunc_normal_table(rows, heads, seed, std=0.02):
    g = torch.Generator().manual_seed(seed)
    t = torch.empty((rows, heads), dtype=torch.float32)
    torch.nn.init.trunc_normal_(t, std=std, a=-2.0, b=2.0, generator=g)
    return t


def bias_from_table(table: torch.Tensor, ws, n=None):
    from oracle import oracle

    rpi = torch.from_numpy(oracle.relative_position_index(ws))
    if n is not None:
        rpi = rpi[:n, :n]
    m = rpi.shape[0]
    return table[rpi.reshape(-1)].reshape(m, m, -1).permute(2, 0, 1).contiguous()


def boundary_flags(D, H, W, ws, ss, outer=1):
    """1 for windows whose mask has a nonzero entry (last window on a shifted axis)."""
    nWd, nWh, nWw = D // ws[0], H // ws[1], W // ws[2]
    flags = []
    for wd in range(nWd):
        for wh in range(nWh):
            for ww in range(nWw):
                f = (wd == nWd - 1 and ss[0] > 0) or (wh == nWh - 1 and ss[1] > 0) or (
                    ww == nWw - 1 and ss[2] > 0)
                flags.append(1 if f else 0)
    return torch.tensor(flags * outer, dtype=torch.uint8)


def synthetic_ct(shape, seed):
    """Config 5 input: a CT-like volume, uniform intensities in [0, 0.5] plus
    12 smooth seeded Gaussian blobs, clamped to [0, 1] (float32, CPU)."""
    g = torch.Generator().manual_seed(seed)
    b, c, d, h, w = shape
    vol = torch.rand(shape, generator=g) * 0.5
    zz, yy, xx = torch.meshgrid(torch.arange(d), torch.arange(h), torch.arange(w), indexing="ij")
    for _ in range(12):
        ctr = torch.rand(3, generator=g) * torch.tensor([d, h, w])
        sigma = 4.0 + 8.0 * torch.rand(1, generator=g).item()
        amp = 0.3 + 0.5 * torch.rand(1, generator=g).item()
        r2 = (zz - ctr[0]) ** 2 + (yy - ctr[1]) ** 2 + (xx - ctr[2]) ** 2
        vol += amp * torch.exp(-r2 / (2 * sigma * sigma))
    return vol.clamp_(0.0, 1.0)


def c_abi():
    """ctypes handle of libcrumpet_hip.so with argument types from include/crumpet_hip.h."""
    from crumpet_amd import _native

    lib = _native.hip_library()
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    for name in ("crumpet_shift_partition_3d", "crumpet_unshift_unpartition_3d",
                 "crumpet_shift_partition_3d_backward", "crumpet_unshift_unpartition_3d_backward"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [vp, vp] + [i64] * 12 + [vp]
    lib.crumpet_compute_attn_mask_3d.restype = ctypes.c_int
    lib.crumpet_compute_attn_mask_3d.argtypes = [vp, ctypes.c_int32] + [i64] * 9 + [vp]
    p4 = ctypes.POINTER(ctypes.c_int64)
    lib.crumpet_fused_swin_attention.restype = ctypes.c_int
    lib.crumpet_fused_swin_attention.argtypes = [
        vp, p4, vp, p4, vp, p4, vp, p4, ctypes.c_int32, i64, i64, i64, i64,
        vp, ctypes.c_int32, p4, vp, ctypes.c_int32, i64, p4, vp, ctypes.c_float, vp,
    ]
    lib.crumpet_fused_swin_attention_shifted.restype = ctypes.c_int
    lib.crumpet_fused_swin_attention_shifted.argtypes = [
        vp, p4, vp, p4, vp, p4, vp, p4, ctypes.c_int32, i64, i64, i64, i64,
        vp, ctypes.c_int32, p4] + [i64] * 9 + [ctypes.c_float, vp]
    i32, f32 = ctypes.c_int32, ctypes.c_float
    lib.crumpet_window_qkv_3d.restype = ctypes.c_int
    lib.crumpet_window_qkv_3d.argtypes = ([vp, i32, vp, i32] + [i64] * 5 + [i32, vp, vp, i32, f32, vp, vp, i64]
                                          + [i64] * 6 + [vp])
    lib.crumpet_window_proj_3d.restype = ctypes.c_int
    lib.crumpet_window_proj_3d.argtypes = [vp, vp, i32] + [i64] * 5 + [vp, vp, i64] + [i64] * 6 + [vp]
    lib.crumpet_last_error.restype = ctypes.c_char_p
    lib.crumpet_status_string.restype = ctypes.c_char_p
    lib.crumpet_status_string.argtypes = [ctypes.c_int]
    lib.crumpet_version.restype = ctypes.c_char_p
    return lib


def strides(t: torch.Tensor, n: int):
    return (ctypes.c_int64 * n)(*t.stride())
