"""Parity of the HIP fused window attention with the fp32 oracle formula
softmax(q*scale @ k^T + bias + [boundary]*mask) @ v (oracle/oracle.py).

Tolerances (max-abs vs fp32 on the same low-precision inputs): 2e-3 fp16,
1e-2 bf16, 1e-4 fp32.  The reference has no attention test; the cases here
cover its wrapper semantics (torch-ext/crumpet/fused_attention.py:149-226):
mask None / broadcast [1,N,N] / per-window [B,N,N], boundary flags, default
scale, strided q/k/v, and the BASELINE shapes (N=343 with 3/6/12/24 heads,
the MONAI N=216 stage-3 case).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crumpet_amd.fused_attention import fused_swin_attention, fused_swin_attention_windows
from helpers import TOL, bias_from_table, boundary_flags, seeded, trunc_normal_table

pytestmark = pytest.mark.gpu


def _inputs(B, H, N, D, dtype, seed):
    q = seeded((B, H, N, D), dtype, seed)
    k = seeded((B, H, N, D), dtype, seed + 1)
    v = seeded((B, H, N, D), dtype, seed + 2)
    return q, k, v


def _ws_for(N):
    for w in range(1, 9):
        if w ** 3 == N:
            return (w, w, w)
    raise ValueError(N)


def _bias(H, N, dtype, seed):
    ws = _ws_for(N)
    rows = (2 * ws[0] - 1) * (2 * ws[1] - 1) * (2 * ws[2] - 1)
    return bias_from_table(trunc_normal_table(rows, H, seed), ws).to(dtype)


def _f32(t):
    return t.float().numpy()


def _compare(out, ref, dtype, what=""):
    err = np.abs(out.float().cpu().numpy() - ref).max()
    print(f"{what} max-abs {err:.3e} (tol {TOL[dtype]})", flush=True)
    assert np.isfinite(out.float().cpu().numpy()).all()
    assert err <= TOL[dtype], f"{what}: max-abs {err} > {TOL[dtype]}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_shifted_mask_per_window_with_boundary(oracle, dev, dtype):
    D = 14
    ws, ss = (7, 7, 7), (3, 3, 3)
    B, H, N, Dh = 8 * 2, 3, 343, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 100)
    bias = _bias(H, N, dtype, 101)
    m8 = torch.from_numpy(oracle.attn_mask(D, D, D, ws, ss, "float32")).to(dtype)
    mask = m8.repeat(2, 1, 1)
    bnd = boundary_flags(D, D, D, ws, ss, outer=2)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(mask), bnd.numpy(), scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev), bnd.to(dev), scale=0.25)
    assert out.dtype == dtype and out.shape == q.shape
    _compare(out, ref, dtype, f"shifted {dtype}")
    # boundary=None: every window reads its mask; same answer here
    out2 = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev), None, scale=0.25)
    _compare(out2, ref, dtype, "boundary None")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_no_mask_and_default_scale(oracle, dev, dtype):
    B, H, N, Dh = 5, 6, 343, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 200)
    bias = _bias(H, N, dtype, 201)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None, None, scale=None)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), None)
    _compare(out, ref, dtype, "no mask")


def test_boundary_flag_skips_mask(oracle, dev):
    dtype = torch.float16
    B, H, N, Dh = 4, 2, 64, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 300)
    bias = _bias(H, N, dtype, 301)
    g = torch.Generator().manual_seed(302)
    mask = torch.where(torch.rand((B, N, N), generator=g) < 0.4, -100.0, 0.0).to(dtype)
    bnd = torch.tensor([1, 0, 0, 1], dtype=torch.uint8)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(mask), bnd.numpy(), scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev),
                               bnd.to(dev).bool(), scale=0.25)
    _compare(out, ref, dtype, "boundary flags")


def test_broadcast_mask_and_fp32_mask(oracle, dev):
    dtype = torch.float16
    B, H, N, Dh = 6, 3, 125, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 400)
    bias = _bias(H, N, torch.float32, 401)  # fp32 bias with fp16 q/k/v
    g = torch.Generator().manual_seed(402)
    mask = torch.randn((1, N, N), generator=g) * 3.0  # arbitrary fp32 values
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), mask.numpy(), None, scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev), None, scale=0.25)
    _compare(out, ref, dtype, "broadcast fp32 mask")


def test_mask_repeat_by_window_index(oracle, dev):
    """mask [nW, N, N] with B = outer * nW: window b reads mask[b % nW]."""
    dtype = torch.bfloat16
    D, ws, ss = 14, (7, 7, 7), (3, 3, 3)
    B, H, N, Dh = 8 * 3, 3, 343, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 500)
    bias = _bias(H, N, dtype, 501)
    m8 = torch.from_numpy(oracle.attn_mask(D, D, D, ws, ss, "float32")).to(dtype)
    bnd = boundary_flags(D, D, D, ws, ss, outer=3)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(m8), bnd.numpy(), scale=0.25)
    out = torch.empty_like(q, device=dev)
    fused_swin_attention_windows(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), m8.to(dev), bnd.to(dev), 0.25, out)
    _compare(out, ref, dtype, "mask mod nW")


@pytest.mark.parametrize("N", [27, 125, 343])
@pytest.mark.parametrize("bdt", [torch.float16, torch.bfloat16, torch.float32], ids=["f16", "bf16", "f32"])
def test_bias_row_strides(oracle, dev, bdt, N):
    """The bias read through padded rows (odd row stride N + 3, so 16-bit rows
    start mid-dword) and through broadcast rows (row stride 0; the op makes
    such a bias contiguous, as it does a broadcast-row mask): every key's
    value reaches the scores, the last keys of the last row included.  Bias
    values ~N(0, 2) make a wrong or missing value visible."""
    dtype = torch.bfloat16 if bdt == torch.bfloat16 else torch.float16
    B, H, Dh = 4, 2, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 950 + N)
    g = torch.Generator().manual_seed(951 + N)
    wide = (torch.randn((H, N, N + 3), generator=g) * 2.0).to(bdt)
    row = (torch.randn((H, 1, N), generator=g) * 2.0).to(bdt)
    mrow = (torch.randn((1, 1, N), generator=g) * 3.0).to(dtype)
    cases = (
        ("padded bias rows", wide[:, :, :N], wide.to(dev)[:, :, :N], None, None),
        ("broadcast rows", row.expand(H, N, N), row.to(dev).expand(H, N, N),
         mrow.expand(1, N, N), mrow.to(dev).expand(1, N, N)),
    )
    for what, b_cpu, b_dev, m_cpu, m_dev in cases:
        if "padded" in what:
            assert b_dev.stride() == (N * (N + 3), N + 3, 1)
        ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(b_cpu), None if m_cpu is None else _f32(m_cpu),
                               None, scale=0.25)
        out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), b_dev, m_dev, None, scale=0.25)
        _compare(out, ref, dtype, f"{what} {bdt} N={N}")


@pytest.mark.parametrize("N", [27, 125, 343])
@pytest.mark.parametrize("mdt", [torch.float16, torch.bfloat16, torch.float32], ids=["f16", "bf16", "f32"])
def test_random_mask_dtypes_and_odd_row_stride(oracle, dev, mdt, N):
    """Arbitrary mask values in every position, the mask a column slice of a
    wider buffer (odd row stride N + 3), N not a multiple of 16: the last key
    tile of the last query row ends exactly at the end of the mask extent."""
    dtype = torch.bfloat16 if mdt == torch.bfloat16 else torch.float16
    B, H, Dh = 6, 2, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 900 + N)
    bias = _bias(H, N, dtype, 901 + N)
    g = torch.Generator().manual_seed(902 + N)
    wide = (torch.randn((3, N, N + 3), generator=g) * 3.0).to(mdt)
    mask = wide[:, :, :N]  # [3, N, N], row stride N + 3, read as mask[b mod 3]
    assert mask.stride() == (N * (N + 3), N + 3, 1)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(mask), None, scale=0.25)
    out = torch.empty_like(q, device=dev)
    fused_swin_attention_windows(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), wide.to(dev)[:, :, :N], None,
                                 0.25, out)
    _compare(out, ref, dtype, f"random {mdt} mask N={N}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_strided_qkv_views_and_strided_out(oracle, dev, dtype):
    """q, k, v as views of a [b, n, 3, H, d] qkv buffer (monai_patch.py:153-154) and
    the output written straight into a [b, n, H*d] buffer."""
    b, n, H, Dh = 8, 343, 3, 16
    qkv = seeded((b, n, 3 * H * Dh), dtype, 600)
    t = qkv.reshape(b, n, 3, H, Dh).permute(2, 0, 3, 1, 4)
    q, k, v = t[0], t[1], t[2]
    bias = _bias(H, n, dtype, 601)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None, None, scale=0.25)
    td = qkv.to(dev).reshape(b, n, 3, H, Dh).permute(2, 0, 3, 1, 4)
    out_bnc = torch.empty((b, n, H * Dh), dtype=dtype, device=dev)
    out = out_bnc.view(b, n, H, Dh).permute(0, 2, 1, 3)
    fused_swin_attention(td[0], td[1], td[2], bias.to(dev), None, scale=0.25, out=out)
    _compare(out, ref, dtype, "strided")
    assert torch.equal(out_bnc.view(b, n, H, Dh).permute(0, 2, 1, 3).cpu(), out.cpu())


@pytest.mark.parametrize("N", [8, 27, 64, 125, 216, 512])
def test_window_volumes(oracle, dev, N):
    dtype = torch.float16
    B, H, Dh = 4, 2, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 700 + N)
    bias = _bias(H, N, dtype, 701)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None, None, scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), None, scale=0.25)
    _compare(out, ref, dtype, f"N={N}")


def test_non_unit_d_stride(oracle, dev):
    dtype = torch.float16
    B, H, N, Dh = 3, 2, 64, 16
    big = seeded((B, H, N, Dh * 2), dtype, 800)
    q = big[..., ::2]
    k = seeded((B, H, N, Dh), dtype, 801)
    v = seeded((B, H, N, Dh), dtype, 802)
    bias = _bias(H, N, dtype, 803)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None, None, scale=0.25)
    out = fused_swin_attention(big.to(dev)[..., ::2], k.to(dev), v.to(dev), bias.to(dev), None, scale=0.25)
    _compare(out, ref, dtype, "non-unit d stride")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
def test_rows_8_byte_aligned(oracle, dev, dtype, masked):
    """q, k, v and out with a row stride of 20 elements (unit d stride, rows
    8-byte but not 16-byte aligned), without a mask (multi-head token
    records) and with a per-window mask under boundary flags: the 16-byte
    K/V transfers and Q loads then start at 8-byte-aligned offsets."""
    B, H, N = 6, 3, 343
    bufs = [seeded((B, H, N, 20), dtype, 820 + i) for i in range(3)]
    q, k, v = (t[..., :16] for t in bufs)
    bias = _bias(H, N, dtype, 823)
    mask = bnd = None
    if masked:
        mask = torch.where(seeded((2, N, N), torch.float32, 824) > 0.7, -100.0, 0.0).to(dtype)
        bnd = torch.tensor([1, 0, 1, 1, 0, 1], dtype=torch.uint8)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None if mask is None else _f32(mask),
                           None if bnd is None else bnd.numpy(), scale=0.25)
    # slice on the device: .to() of a non-dense view would make it contiguous
    qd, kd, vd = (t.to(dev)[..., :16] for t in bufs)
    out_buf = torch.full((B, H, N, 20), float("nan"), dtype=dtype, device=dev)
    out = out_buf[..., :16]
    for t in (qd, kd, vd, out):
        assert t.stride(2) == 20 and t.stride(3) == 1 and t.data_ptr() % 16 == 0
    fused_swin_attention_windows(qd, kd, vd, bias.to(dev), None if mask is None else mask.to(dev),
                                 None if bnd is None else bnd.to(dev), 0.25, out)
    _compare(out, ref, dtype, f"8-byte-aligned rows {dtype} masked={masked}")
    assert torch.isnan(out_buf[..., 16:].float()).all()  # nothing written past the head dim


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_config3_stage0_all_windows(oracle, dev, dtype):
    """qkv [1372, 343, 144] fp16, table [2197, 3] trunc-normal 0.02,
    49^3 shifted mask tiled over sw-batch 4, scale 0.25.  Every window against
    the oracle, through the reference API (contiguous q/k/v, the mask
    repeated to [1372, N, N]: one head per workgroup) and through the
    window-batch entry the MONAI patch uses (q/k/v views of the qkv tensor,
    the [343, N, N] mask read as mask[b mod 343] in mask-major window order);
    in the BASELINE dtype fp16, and in bf16."""
    D, ws, ss = 49, (7, 7, 7), (3, 3, 3)
    B, H, N, Dh = 1372, 3, 343, 16
    qkv = seeded((B, N, 3 * H * Dh), dtype, 900)
    table = trunc_normal_table(2197, H, 901)
    bias = bias_from_table(table, ws).to(dtype)
    m = torch.from_numpy(oracle.attn_mask(D, D, D, ws, ss, "float32")).to(dtype)
    mask = m.repeat(4, 1, 1)
    bnd = boundary_flags(D, D, D, ws, ss, outer=4)
    td = qkv.to(dev).reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4)
    out = fused_swin_attention(td[0].contiguous(), td[1].contiguous(), td[2].contiguous(), bias.to(dev),
                               mask.to(dev), bnd.to(dev), scale=0.25)
    assert torch.isfinite(out).all()
    t = qkv.reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4)
    ref = oracle.attention(_f32(t[0]), _f32(t[1]), _f32(t[2]), _f32(bias), _f32(m), bnd.numpy(), scale=0.25)
    _compare(out, ref, dtype, "config3 all windows, reference API")
    out_bnc = torch.empty((B, N, H * Dh), dtype=dtype, device=dev)
    ov = out_bnc.view(B, N, H, Dh).permute(0, 2, 1, 3)
    fused_swin_attention_windows(td[0], td[1], td[2], bias.to(dev), m.to(dev), bnd.to(dev), 0.25, ov)
    _compare(ov, ref, dtype, "config3 all windows, mask [343,N,N] on qkv views")


SHIFTED_CASES = [
    # (volume, window, shift, outer batch)
    ((14, 14, 14), (7, 7, 7), (3, 3, 3), 2),
    ((14, 7, 21), (7, 7, 7), (3, 0, 2), 1),
    ((14, 14, 14), (7, 7, 7), (0, 0, 0), 1),
    ((12, 12, 12), (6, 6, 6), (3, 3, 3), 1),
    ((8, 8, 8), (4, 4, 4), (2, 2, 2), 3),
    ((7, 7, 7), (7, 7, 7), (3, 3, 3), 4),
]


@pytest.mark.parametrize("case", SHIFTED_CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_shifted_region_mask_matches_oracle(oracle, dev, case, dtype):
    """fused_swin_attention_shifted == attention with the compute_attn_mask_3d mask
    tiled over the outer batch (window b uses mask[b % nW])."""
    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    vol, ws, ss, outer = case
    nW = (vol[0] // ws[0]) * (vol[1] // ws[1]) * (vol[2] // ws[2])
    N = ws[0] * ws[1] * ws[2]
    B, H, Dh = nW * outer, 3, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 1000 + N)
    rows = (2 * ws[0] - 1) * (2 * ws[1] - 1) * (2 * ws[2] - 1)
    bias = bias_from_table(trunc_normal_table(rows, H, 1001), ws).to(dtype)
    m = oracle.attn_mask(*vol, ws, ss, "float32")
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), m, None, scale=0.25)
    out = fused_swin_attention_shifted(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), vol, ws, ss,
                                       scale=0.25)
    _compare(out, ref, dtype, f"shifted {case} {dtype}")


def test_shifted_equals_tensor_mask_path(oracle, dev):
    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    dtype = torch.float16
    vol, ws, ss = (14, 14, 14), (7, 7, 7), (3, 3, 3)
    B, H, N, Dh = 16, 3, 343, 16
    q, k, v = (t.to(dev) for t in _inputs(B, H, N, Dh, dtype, 1100))
    bias = _bias(H, N, dtype, 1101).to(dev)
    import crumpet_amd

    mask = crumpet_amd.compute_attn_mask_3d(*vol, ws, ss, dtype, dev)
    a = fused_swin_attention_shifted(q, k, v, bias, vol, ws, ss, scale=0.25)
    b = torch.empty_like(q)
    fused_swin_attention_windows(q, k, v, bias, mask, None, 0.25, b)
    assert (a.float() - b.float()).abs().max().item() <= 1e-3


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_config3_stage0_shifted_all_windows(oracle, dev, dtype):
    """Config 3 through the region-mask path, every window vs the oracle
    (the BASELINE dtype fp16, and bf16)."""
    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    D, ws, ss = 49, (7, 7, 7), (3, 3, 3)
    B, H, N, Dh = 1372, 3, 343, 16
    qkv = seeded((B, N, 3 * H * Dh), dtype, 1200)
    bias = bias_from_table(trunc_normal_table(2197, H, 1201), ws).to(dtype)
    td = qkv.to(dev).reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4)
    out_bnc = torch.empty((B, N, H * Dh), dtype=dtype, device=dev)
    out = out_bnc.view(B, N, H, Dh).permute(0, 2, 1, 3)
    fused_swin_attention_shifted(td[0], td[1], td[2], bias.to(dev), (D, D, D), ws, ss, scale=0.25, out=out)
    assert torch.isfinite(out).all()
    m = oracle.attn_mask(D, D, D, ws, ss, "float32")
    t = qkv.reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4)
    ref = oracle.attention(_f32(t[0]), _f32(t[1]), _f32(t[2]), _f32(bias), m, None, scale=0.25)
    _compare(out, ref, dtype, "config3 shifted, all windows")


@pytest.mark.parametrize("N", [1, 2, 15, 16, 17, 63, 64, 65, 128, 129, 224, 225, 352, 353, 511, 512])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_tile_count_boundaries(oracle, dev, N, dtype):
    """Every tile-count class and its edges (N = 16 t and 16 t + 1, the
    smallest and largest N of each compiled NT), any N (no window shape
    implied), with a random fp32 bias and, for odd N, an fp32 mask with
    boundary flags."""
    B, H, Dh = 3, 2, 16
    q, k, v = _inputs(B, H, N, Dh, dtype, 900 + N)
    bias = seeded((H, N, N), torch.float32, 901 + N)
    mask = bnd = None
    if N % 2:
        mask = torch.where(seeded((B, N, N), torch.float32, 902 + N) > 0.7, -100.0, 0.0)
        bnd = torch.tensor([1, 0, 1], dtype=torch.uint8)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None if mask is None else mask.numpy(),
                           None if bnd is None else bnd.numpy(), scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev),
                               None if mask is None else mask.to(dev), None if bnd is None else bnd.to(dev),
                               scale=0.25)
    _compare(out, ref, dtype, f"N={N} {dtype}")


def _interleaved(B, N, H, dtype, seed):
    """q, k, v as views of one [B, N, 3, H, Dh] qkv tensor (the MONAI layout:
    a token's heads adjacent, head stride 16), plus the CPU tensor."""
    qkv = seeded((B, N, 3 * H * 16), dtype, seed)
    return qkv, qkv.reshape(B, N, 3, H, 16).permute(2, 0, 3, 1, 4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H", [3, 6])
@pytest.mark.parametrize("ws", [(6, 6, 6), (7, 7, 7)])
@pytest.mark.parametrize("mode", ["region", "nomask", "tensor"])
def test_head_records_interleaved_qkv(oracle, dev, dtype, H, ws, mode):
    """Interleaved qkv with H a multiple of 3 runs three heads per workgroup
    with K/V staged as token records (N = 216 and 343: both tile counts that
    have that variant), also with a mask tensor and no boundary flags (every
    window masked, paired key order); every window against the oracle, and
    against the same data in separate contiguous tensors (one head per
    workgroup)."""
    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    shifted = mode != "nomask"
    vol = tuple(2 * w for w in ws)
    ss = tuple(w // 2 for w in ws) if shifted else (0, 0, 0)
    N = ws[0] * ws[1] * ws[2]
    B = 8 * 2  # two outer batches of 8 windows
    qkv, t = _interleaved(B, N, H, dtype, 1300 + N + H)
    rows = (2 * ws[0] - 1) * (2 * ws[1] - 1) * (2 * ws[2] - 1)
    bias = bias_from_table(trunc_normal_table(rows, H, 1301 + H), ws).to(dtype)
    m = oracle.attn_mask(*vol, ws, ss, "float32") if shifted else None
    ref = oracle.attention(_f32(t[0]), _f32(t[1]), _f32(t[2]), _f32(bias), None if m is None else m[np.arange(B) % 8],
                           None, scale=0.25)
    td = qkv.to(dev).reshape(B, N, 3, H, 16).permute(2, 0, 3, 1, 4)
    out_bnc = torch.empty((B, N, H * 16), dtype=dtype, device=dev)
    out = out_bnc.view(B, N, H, 16).permute(0, 2, 1, 3)
    mask_t = None if m is None else torch.from_numpy(np.ascontiguousarray(m[np.arange(B) % 8])).to(dtype).to(dev)
    if mode == "region":
        fused_swin_attention_shifted(td[0], td[1], td[2], bias.to(dev), vol, ws, ss, scale=0.25, out=out)
    else:
        fused_swin_attention(td[0], td[1], td[2], bias.to(dev), mask_t, scale=0.25, out=out)
    _compare(out, ref, dtype, f"records H={H} N={N} {mode}")
    sep = [x.contiguous() for x in td]
    if mode == "region":
        other = fused_swin_attention_shifted(sep[0], sep[1], sep[2], bias.to(dev), vol, ws, ss, scale=0.25)
    else:
        other = fused_swin_attention(sep[0], sep[1], sep[2], bias.to(dev), mask_t, scale=0.25)
    diff = (out.float() - other.float()).abs().max().item()
    assert diff <= TOL[dtype], diff


@pytest.mark.parametrize("N", [209, 224, 337, 352])
def test_head_records_tile_edges(oracle, dev, N):
    """The record path at the smallest and largest N of its tile counts (14
    and 22), any N, no mask: padded key rows of the records repeat row N-1
    and are masked by the bias tiles."""
    dtype, H, B = torch.float16, 3, 5
    qkv, t = _interleaved(B, N, H, dtype, 1400 + N)
    bias = seeded((H, N, N), torch.float32, 1401 + N)
    ref = oracle.attention(_f32(t[0]), _f32(t[1]), _f32(t[2]), _f32(bias), None, None, scale=0.25)
    td = qkv.to(dev).reshape(B, N, 3, H, 16).permute(2, 0, 3, 1, 4)
    out = fused_swin_attention(td[0], td[1], td[2], bias.to(dev), None, scale=0.25)
    _compare(out, ref, dtype, f"records N={N}")


@pytest.mark.parametrize("N", [129, 131, 225, 353])
@pytest.mark.parametrize("dt16", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_last_key_of_last_row_16bit(oracle, dev, N, dt16):
    """16-bit bias and mask whose [N, N] extent ends in the middle of a dword,
    at N where the tile count is rounded up (key N-1 is not in the last
    tile): the last row's last key must keep its bias and mask values (a
    dword-granular range check would read them as 0)."""
    dtype, H, B = torch.float16, 2, 3
    q, k, v = _inputs(B, H, N, 16, dtype, 1500 + N)
    bias = (seeded((H, N, N), torch.float32, 1501 + N) * 0.5).to(dt16)
    bias[:, N - 1, N - 1] = 4.0  # a large bias on the last key of the last row
    mask = torch.where(seeded((B, N, N), torch.float32, 1502 + N) > 0.5, -100.0, 0.0).to(dt16)
    mask[:, N - 1, :] = 0.0
    mask[0, N - 1, N - 1] = -100.0  # window 0: the last key of the last row masked
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), _f32(mask), None, scale=0.25)
    out = fused_swin_attention(q.to(dev), k.to(dev), v.to(dev), bias.to(dev), mask.to(dev), None, scale=0.25)
    _compare(out, ref, dtype, f"N={N} {dt16} last key")
    _compare(out[:, :, N - 1], ref[:, :, N - 1], dtype, f"N={N} {dt16} last row")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("Dh", [16, 32])
@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
def test_row_sums_out_of_range_take_the_exact_pass(oracle, dev, dtype, Dh, masked):
    """Windows whose row sums leave the offset softmax's range, between
    ordinary ones: a head whose bias sits 20 below (natural units) the
    others, so its first window's row sums are near 2^-20, windows with
    q = 3k, whose dominant diagonal reaches 2^40 and more (fp16 P overflow),
    and windows with q = 12k (row sums past 2^64 with finite bf16 P).
    Each forces the exact pass and moves the offsets for the following
    windows; B = 96 gives every workgroup several windows (multi-head records
    and head-dim-32 strip groups without a mask, 4-wave workgroups with a
    mask tensor and boundary flags).  The results must match the fp32 oracle
    like any other window."""
    B, H, N = 96, 3, 343
    qkv = seeded((B, N, 3, H, Dh), dtype, 1300 + Dh)  # the MONAI layout: heads adjacent
    peaky = [4, 5, 30, 31, 32, 61, 90]
    qkv[peaky, :, 0] = (qkv[peaky, :, 1].float() * 3).to(dtype)
    sharper = [50, 51, 75]  # row sums near 2^70: finite bf16 P past the 2^64 bound
    qkv[sharper, :, 0] = (qkv[sharper, :, 1].float() * 12).to(dtype)
    # a dominant diagonal makes a row's output its own v (up to ~5 for N(0, 1)
    # values, where bf16 rounding alone exceeds 1e-2): v at a quarter scale
    qkv[:, :, 2] = (qkv[:, :, 2].float() * 0.25).to(dtype)
    q, k, v = qkv.permute(2, 0, 3, 1, 4)
    bias = seeded((H, N, N), torch.float32, 1310) * 0.5
    bias[1] -= 20.0
    mask = bnd = None
    if masked:
        mask = torch.where(seeded((3, N, N), torch.float32, 1320) > 0.8, -100.0, 0.0).to(dtype)
        bnd = (torch.arange(B) % 3 != 1).to(torch.uint8)
    ref = oracle.attention(_f32(q), _f32(k), _f32(v), _f32(bias), None if mask is None else _f32(mask),
                           None if bnd is None else bnd.numpy(), scale=0.25)
    qd, kd, vd = qkv.to(dev).permute(2, 0, 3, 1, 4)
    out = fused_swin_attention_windows(qd, kd, vd, bias.to(dev), None if mask is None else mask.to(dev),
                                       None if bnd is None else bnd.to(dev), 0.25,
                                       torch.empty((B, H, N, Dh), dtype=dtype, device=dev))
    _compare(out, ref, dtype, f"exact pass Dh={Dh} {dtype} masked={masked}")
