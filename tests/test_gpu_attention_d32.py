"""Head dim 32 on the tuned kernel (attention_kernel.h, D = 32): 2-byte
types, unit d stride, 129 <= N <= 352 (14 or 22 key tiles).  Everything
else at head dim 32 runs the general kernel (test_gpu_attention_wide.py).

Against the fp32 oracle formula softmax(q*scale @ k^T + bias +
[boundary]*mask) @ v (oracle/oracle.py) on the same low-precision inputs,
with the tolerances of the other attention tests (2e-3 fp16, 1e-2 bf16
max-abs), and against the general kernel on the same inputs (a non-unit d
stride sends a call there).  The reference's Triton kernel takes head dim
32 through the same entry point (torch-ext/crumpet/fused_attention.py:149-226).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crumpet_amd.fused_attention import fused_swin_attention_shifted, fused_swin_attention_windows
from helpers import TOL, bias_from_table, boundary_flags, seeded, trunc_normal_table

pytestmark = pytest.mark.gpu

DT = [torch.float16, torch.bfloat16]
IDS = ["f16", "bf16"]


def _f32(t):
    return t.float().numpy()


def _compare(out, ref, dtype, what):
    got = out.float().cpu().numpy()
    err = np.abs(got - ref).max()
    print(f"{what}: max-abs {err:.3e} (tol {TOL[dtype]})", flush=True)
    assert np.isfinite(got).all()
    assert err <= TOL[dtype], f"{what}: max-abs {err} > {TOL[dtype]}"


def _qkv_views(B, N, H, dtype, seed):
    """The [B, N, 3 * H * 32] qkv buffer and q, k, v as [B, H, N, 32] views
    of it (the MONAI qkv layout)."""
    qkv = seeded((B, N, 3 * H * 32), dtype, seed)
    t = qkv.reshape(B, N, 3, H, 32).permute(2, 0, 3, 1, 4)
    return qkv, t[0], t[1], t[2]


@pytest.mark.parametrize("dtype", DT, ids=IDS)
@pytest.mark.parametrize("N", [129, 200, 224, 225, 320, 321, 343, 352])
@pytest.mark.parametrize("mode", ["none", "mask_f16", "mask_bf16", "mask_f32", "mask_f16_noflags"])
def test_tile_edges_and_mask_kinds(oracle, dev, N, dtype, mode):
    """Both tile classes at their edges (14 tiles: 129..224, 22: 225..352;
    at 22 tiles, 21 and 22 strips (N >= 321) run three strip groups per
    workgroup without a mask or without boundary flags, N = 320 the 4-wave
    form), without a mask and with a per-window mask of each dtype read as
    mask[b mod 3] under boundary flags (fp16 also without flags), fp32 bias
    with -inf-free values."""
    B, H = 12, 2
    q, k, v = (seeded((B, H, N, 32), dtype, 5000 + N + i) for i in range(3))
    bias = seeded((H, N, N), torch.float32, 5010 + N) * 0.5
    mask = bnd = None
    if mode != "none":
        mdt = {"mask_bf16": torch.bfloat16, "mask_f32": torch.float32}.get(mode, torch.float16)
        m = torch.where(seeded((3, N, N), torch.float32, 5020 + N) > 0.8, -100.0, 0.0)
        mask = (m + seeded((3, N, N), torch.float32, 5030 + N) * 0.25).to(mdt)
        if mode != "mask_f16_noflags":
            bnd = torch.tensor([1, 0, 1, 1, 0, 1, 0, 0, 1, 1, 1, 0], dtype=torch.uint8)
    print(f"d32 N={N} {dtype} {mode}", flush=True)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None if mask is None else _f32(mask),
                           None if bnd is None else bnd.numpy(), scale=0.25)
    qd = q.to(dev)
    out = fused_swin_attention_windows(qd, k.to(dev), v.to(dev), bias.to(dev),
                                       None if mask is None else mask.to(dev),
                                       None if bnd is None else bnd.to(dev), 0.25, torch.empty_like(qd))
    _compare(out, ref, dtype, f"d32 N={N} {mode}")


@pytest.mark.parametrize("dtype", DT, ids=IDS)
def test_shifted_region_interleaved_qkv(oracle, dev, dtype):
    """Region mode (the shifted mask from the 14^3 geometry, never
    materialised) on q/k/v views of an interleaved qkv buffer, 3 heads, the
    model's bias gather, against the tiled compute_attn_mask_3d mask."""
    vol, ws, ss = (14, 14, 14), (7, 7, 7), (3, 3, 3)
    B, H, N = 8 * 2, 3, 343
    _, q, k, v = _qkv_views(B, N, H, dtype, 5100)
    bias = bias_from_table(trunc_normal_table(13 ** 3, H, 5101), ws).to(dtype)
    m = oracle.attn_mask(*vol, ws, ss, "float32")
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), m, None, scale=32 ** -0.5)
    out = torch.empty((B, N, H * 32), dtype=dtype, device=dev)
    ov = out.view(B, N, H, 32).permute(0, 2, 1, 3)
    fused_swin_attention_shifted(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), vol, ws, ss, None, ov)
    _compare(ov, ref, dtype, f"d32 region interleaved {dtype}")


@pytest.mark.parametrize("dtype", DT, ids=IDS)
def test_tuned_and_general_kernels_agree(oracle, dev, dtype):
    """The same tensor-mask problem through the tuned kernel (unit d stride)
    and the general one (a d stride of 2 over a wider buffer): each within
    the tolerance of the oracle and of the other."""
    B, H, N = 6, 3, 343
    q, k, v = (seeded((B, H, N, 32), dtype, 5200 + i) for i in range(3))
    bias = seeded((H, N, N), torch.float32, 5203) * 0.5
    mask = torch.where(seeded((2, N, N), torch.float32, 5204) > 0.7, -100.0, 0.0).to(dtype)
    bnd = torch.tensor([1, 1, 0, 1, 0, 1], dtype=torch.uint8)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(mask), bnd.numpy(), scale=0.25)
    args = (bias.to(dev), mask.to(dev), bnd.to(dev), 0.25)
    qd = q.to(dev)
    tuned = fused_swin_attention_windows(qd, k.to(dev), v.to(dev), *args, torch.empty_like(qd))
    wide_in = []
    for t in (q, k, v):
        w = torch.zeros((B, H, N, 64), dtype=dtype)
        w[..., ::2] = t
        wide_in.append(w.to(dev)[..., ::2])
    assert wide_in[0].stride(-1) == 2
    general = fused_swin_attention_windows(*wide_in, *args, torch.empty_like(qd))
    _compare(tuned, ref, dtype, f"tuned {dtype}")
    _compare(general, ref, dtype, f"general {dtype}")
    d = (tuned.float() - general.float()).abs().max().item()
    print(f"tuned vs general: {d:.3e}", flush=True)
    assert d <= TOL[dtype]


@pytest.mark.parametrize("dtype", DT, ids=IDS)
def test_config3_shape_all_windows(oracle, dev, dtype):
    """The config-3 window shape at head dim 32 (1372 windows x 3 heads of
    343 tokens, feature size 96), shifted mask of the 49^3 geometry as
    region mode (three strip groups per workgroup) and as the [343] mask
    tensor with boundary flags (4-wave workgroups): every window against
    the oracle."""
    vol, ws, ss = (49, 49, 49), (7, 7, 7), (3, 3, 3)
    B, H, N = 1372, 3, 343
    _, q, k, v = _qkv_views(B, N, H, dtype, 5300)
    bias = bias_from_table(trunc_normal_table(13 ** 3, H, 5301), ws).to(dtype)
    m = torch.from_numpy(oracle.attn_mask(*vol, ws, ss, "float32"))
    bnd = boundary_flags(*vol, ws, ss, outer=4)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), m.numpy(), None, scale=0.25)  # mask[b % 343]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out_r = fused_swin_attention_shifted(qd, kd, vd, bias.to(dev), vol, ws, ss, 0.25)
    out_t = fused_swin_attention_windows(qd, kd, vd, bias.to(dev), m.to(dtype).to(dev), bnd.to(dev), 0.25,
                                         torch.empty((B, H, N, 32), dtype=dtype, device=dev))
    for name, out in (("region", out_r), ("tensor", out_t)):
        _compare(out, ref, dtype, f"config-3 shape d32 {name} {dtype}")


@pytest.mark.parametrize("dtype", DT, ids=IDS)
@pytest.mark.parametrize("N", [300, 343])
def test_rows_8_byte_aligned(oracle, dev, dtype, N):
    """q, k, v and out with a row stride of 36 elements (unit d stride, rows
    8-byte but not 16-byte aligned), in the 4-wave form (N = 300) and with
    three strip groups per workgroup (N = 343): the 16-byte Q loads and K/V
    transfers then start at 8-byte-aligned offsets."""
    B, H = 5, 2
    bufs = [seeded((B, H, N, 36), dtype, 5400 + i) for i in range(3)]
    q, k, v = (t[..., :32] for t in bufs)
    bias = seeded((H, N, N), torch.float32, 5403) * 0.5
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None, None, scale=0.25)
    # slice on the device: .to() of a non-dense view would make it contiguous
    qd, kd, vd = (t.to(dev)[..., :32] for t in bufs)
    out_buf = torch.full((B, H, N, 36), float("nan"), dtype=dtype, device=dev)
    out = out_buf[..., :32]
    for t in (qd, kd, vd, out):
        assert t.stride(2) == 36 and t.stride(3) == 1 and t.data_ptr() % 16 == 0
    fused_swin_attention_windows(qd, kd, vd, bias.to(dev), None, None, 0.25, out)
    _compare(out, ref, dtype, f"d32 8-byte-aligned rows N={N} {dtype}")
    assert torch.isnan(out_buf[..., 32:].float()).all()  # nothing written past the head dim
