"""GPU parity of the fused window-MSA block projections (window_qkv_3d,
window_proj_3d) with the oracle, and of the whole fused forward_part1 with
the eager MONAI-style block.

Kernel vs oracle (oracle.window_qkv / window_proj, float64 with the
autocast roundings): within 4 ulps of the compute dtype relative to
max(|ref|, 1) -- the LayerNorm output may round to the neighbouring value
near a rounding boundary (fp32 vs float64 statistics), and fp32
accumulation differs from float64 by far less than one output ulp.
Shapes: the Swin UNETR stages at window 7 (padded 12^3, shifted 14^3, the
7^3 / 6^3 deep stages) and a non-cubic padded case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from crumpet_amd import fused_block, monai_patch
from crumpet_amd import swin_unetr_compat as sw
from helpers import seeded

pytestmark = pytest.mark.gpu

CASES = [  # name, (B, D, H, W, C), ws, ss
    ("s0pad", (2, 12, 12, 12, 48), (7, 7, 7), (3, 3, 3)),
    ("s1", (1, 14, 14, 14, 96), (7, 7, 7), (3, 3, 3)),
    ("s2", (1, 7, 7, 7, 192), (7, 7, 7), (0, 0, 0)),
    ("s3monai", (2, 6, 6, 6, 384), (6, 6, 6), (0, 0, 0)),
    ("noncubic", (1, 7, 9, 5, 32), (7, 3, 5), (2, 1, 0)),
    ("c16", (2, 9, 9, 9, 16), (7, 7, 7), (3, 3, 3)),        # smallest C, padded
    ("c224", (1, 7, 8, 7, 224), (7, 7, 7), (3, 3, 3)),      # widest C an fp32 tile takes
]
DTYPES = [  # (x dtype, compute dtype)
    (torch.float32, torch.float16),
    (torch.float32, torch.bfloat16),
    (torch.float32, torch.float32),
    (torch.float16, torch.float16),
    (torch.bfloat16, torch.bfloat16),
]
ULP = {torch.float16: 2 ** -10, torch.bfloat16: 2 ** -7, torch.float32: 2 ** -18}
NAME = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _compare(got: torch.Tensor, want: np.ndarray, dtype, what: str):
    g = got.float().cpu().double().numpy()
    assert np.isfinite(g).all()
    err = np.abs(g - want)
    bound = 4 * ULP[dtype] * np.maximum(np.abs(want), 1.0)
    worst = float((err / bound).max())
    print(f"{what}: max-abs {err.max():.3e}, worst err/bound {worst:.2f}", flush=True)
    assert worst <= 1.0, f"{what}: error {err.max()} beyond 4 ulps"


def _skip_unsupported(C, cdt):
    if not monai_patch._fits_staging_tile(C, torch.empty((), dtype=cdt).element_size()):
        pytest.skip(f"C={C} in {cdt} exceeds the staging tile (unfused path)")


@pytest.mark.parametrize("dts", DTYPES, ids=lambda d: f"{NAME[d[0]]}-{NAME[d[1]]}")
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_window_qkv_matches_oracle(oracle, dev, case, dts):
    name, shape, ws, ss = case
    xdt, cdt = dts
    C = shape[-1]
    _skip_unsupported(C, cdt)
    print(f"window_qkv {name} {xdt}->{cdt}", flush=True)
    x = (seeded(shape, torch.float32, 40) * 2.0 + 0.5).to(xdt)
    gw = seeded((C,), torch.float32, 41) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 42) * 0.1
    w = (seeded((3 * C, C), torch.float32, 43) / C ** 0.5).to(cdt)
    b = (seeded((3 * C,), torch.float32, 44) * 0.1).to(cdt)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), b.to(dev), ws, ss, gw.to(dev), gb.to(dev), 1e-5, True,
                                    cdt)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), b.double().numpy(),
                             gw.double().numpy(), gb.double().numpy(), 1e-5, True, NAME[cdt])
    assert got.shape == want.shape
    _compare(got, want, cdt, f"window_qkv {name}")


def test_window_qkv_options(oracle, dev):
    """No LayerNorm, no bias, LayerNorm parameters in the input's dtype."""
    _, shape, ws, ss = CASES[0]
    C = shape[-1]
    x = seeded(shape, torch.float16, 45)
    w = (seeded((32, C), torch.float32, 46) / C ** 0.5).to(torch.float16)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), None, ws, ss, normalize=False)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), None, normalize=False)
    _compare(got, want, torch.float16, "no norm, no bias")
    gw = (seeded((C,), torch.float32, 47) + 1.0).to(torch.float16)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), None, ws, ss, gw.to(dev), None, 1e-6)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), None, gw.double().numpy(), None, 1e-6)
    _compare(got, want, torch.float16, "fp16 LN weight, no LN bias")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16, torch.float32], ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_window_proj_matches_oracle(oracle, dev, case, cdt):
    name, shape, ws, ss = case
    B, D, H, W, C = shape
    _skip_unsupported(C, cdt)
    print(f"window_proj {name} {cdt}", flush=True)
    Dp, Hp, Wp = (-(-n // k) * k for n, k in zip((D, H, W), ws))
    nwin = B * (Dp // ws[0]) * (Hp // ws[1]) * (Wp // ws[2])
    win = seeded((nwin, ws[0] * ws[1] * ws[2], C), torch.float32, 50).to(cdt)
    w = (seeded((C, C), torch.float32, 51) / C ** 0.5).to(cdt)
    b = (seeded((C,), torch.float32, 52) * 0.1).to(cdt)
    got = fused_block.window_proj_3d(win.to(dev), w.to(dev), b.to(dev), B, D, H, W, ws, ss)
    want = oracle.window_proj(win.double().numpy(), B, D, H, W, ws, ss, w.double().numpy(), b.double().numpy(),
                              NAME[cdt])
    assert got.shape == want.shape
    _compare(got, want, cdt, f"window_proj {name}")


@pytest.mark.parametrize("dts", DTYPES[:2] + DTYPES[3:], ids=lambda d: f"{NAME[d[0]]}-{NAME[d[1]]}")
@pytest.mark.parametrize("C", [16, 32, 48, 96, 192])
@pytest.mark.parametrize("dims", [(1, 9, 10, 11), (1, 2, 3, 3)], ids=["9x10x11", "2x3x3"])
def test_window_qkv_register_path(oracle, dev, dims, C, dts):
    """2-byte compute types with n_out = 3 C take the streaming kernels
    (LayerNorm statistics over the 4 lanes of a token, permuted contraction
    and feature order, 16-token tiles): C at most 48 with the weights in
    registers, C = 96 and 192 with the weights in LDS (all three q/k/v
    chunks per workgroup, or one of six).  A partial last tile, fewer tiles
    than waves, LayerNorm off, and LayerNorm parameters in the input's
    dtype."""
    B, D, H, W = dims
    xdt, cdt = dts
    ws, ss = (7, 7, 7), (3, 3, 3)
    x = (seeded((B, D, H, W, C), torch.float32, 64) * 2.0 + 0.5).to(xdt)
    gw = seeded((C,), torch.float32, 65) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 66) * 0.1
    w = (seeded((3 * C, C), torch.float32, 67) / C ** 0.5).to(cdt)
    b = (seeded((3 * C,), torch.float32, 68) * 0.1).to(cdt)
    print(f"window_qkv register path {dims} C={C} {xdt}->{cdt}", flush=True)
    xd, wd, bd = x.to(dev), w.to(dev), b.to(dev)
    xn, wn, bn = x.double().numpy(), w.double().numpy(), b.double().numpy()
    got = fused_block.window_qkv_3d(xd, wd, bd, ws, ss, gw.to(dev), gb.to(dev), 1e-5, True, cdt)
    want = oracle.window_qkv(xn, ws, ss, wn, bn, gw.double().numpy(), gb.double().numpy(), 1e-5, True, NAME[cdt])
    assert got.shape == want.shape
    _compare(got, want, cdt, f"window_qkv {dims} C={C}")
    got = fused_block.window_qkv_3d(xd, wd, None, ws, ss, normalize=False, dtype=cdt)
    want = oracle.window_qkv(xn, ws, ss, wn, None, normalize=False, dtype=NAME[cdt])
    _compare(got, want, cdt, "no norm, no bias")
    if xdt != torch.float32:
        gwx = gw.to(xdt)
        got = fused_block.window_qkv_3d(xd, wd, bd, ws, ss, gwx.to(dev), None, 1e-6, True, cdt)
        want = oracle.window_qkv(xn, ws, ss, wn, bn, gwx.double().numpy(), None, 1e-6, True, NAME[cdt])
        _compare(got, want, cdt, "LN weight in the input dtype, no LN bias")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_window_qkv_stage0_full_size(oracle, dev, cdt):
    """Config-5 stage 0 at full size: fp32 [4, 48^3, 48] -> [1372, 343, 144],
    every window-ordered token (padding included) against the oracle."""
    B, D, C, ws, ss = 4, 48, 48, (7, 7, 7), (3, 3, 3)
    x = seeded((B, D, D, D, C), torch.float32, 69) * 1.5 + 0.25
    gw = seeded((C,), torch.float32, 70) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 71) * 0.1
    w = (seeded((3 * C, C), torch.float32, 72) / C ** 0.5).to(cdt)
    b = (seeded((3 * C,), torch.float32, 73) * 0.1).to(cdt)
    print(f"window_qkv stage 0 full size {cdt}", flush=True)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), b.to(dev), ws, ss, gw.to(dev), gb.to(dev), 1e-5, True,
                                    cdt)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), b.double().numpy(),
                             gw.double().numpy(), gb.double().numpy(), 1e-5, True, NAME[cdt])
    _compare(got, want, cdt, "window_qkv stage 0")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("D,C,nwin", [(24, 96, 256), (12, 192, 32)], ids=["s1", "s2"])
def test_window_qkv_stages_1_2_full_size(oracle, dev, cdt, D, C, nwin):
    """Config-5 stages 1 and 2 at full size on the LDS-weight streaming
    kernel: fp32 [4, 24^3, 96] -> [256, 343, 288] (5488 tiles, two steps of
    every wave, all three chunks per workgroup) and [4, 12^3, 192] ->
    [32, 343, 576] (686 tiles in six chunk groups), every window-ordered
    token (padding included) against the oracle."""
    B, ws, ss = 4, (7, 7, 7), (3, 3, 3)
    x = seeded((B, D, D, D, C), torch.float32, 74) * 1.5 + 0.25
    gw = seeded((C,), torch.float32, 75) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 76) * 0.1
    w = (seeded((3 * C, C), torch.float32, 77) / C ** 0.5).to(cdt)
    b = (seeded((3 * C,), torch.float32, 78) * 0.1).to(cdt)
    print(f"window_qkv full size C={C} {cdt}", flush=True)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), b.to(dev), ws, ss, gw.to(dev), gb.to(dev), 1e-5, True,
                                    cdt)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), b.double().numpy(),
                             gw.double().numpy(), gb.double().numpy(), 1e-5, True, NAME[cdt])
    assert got.shape == want.shape == (nwin, 343, 3 * C)
    _compare(got, want, cdt, f"window_qkv full size C={C}")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("C,n_out", [(16, 16), (32, 48), (48, 48), (64, 64), (48, 16), (16, 64), (96, 96)])
@pytest.mark.parametrize("dims", [(1, 9, 10, 11), (3, 9, 9, 9), (1, 2, 3, 3)], ids=["990tok", "2187tok", "18tok"])
def test_window_proj_register_path(oracle, dev, dims, C, n_out, cdt):
    """2-byte types with C and n_out at most 64, and 96 -> 96 (stage 1), take
    the register-resident kernel (weights in registers, permuted contraction
    and feature order, 16-token tiles): token counts that leave a partial
    last tile, fewer tiles than waves, and n_out != C."""
    B, D, H, W = dims
    ws, ss = (7, 7, 7), (3, 3, 3)
    Dp, Hp, Wp = (-(-n // k) * k for n, k in zip((D, H, W), ws))
    nwin = B * (Dp // 7) * (Hp // 7) * (Wp // 7)
    win = seeded((nwin, 343, C), torch.float32, 58).to(cdt)
    w = (seeded((n_out, C), torch.float32, 59) / C ** 0.5).to(cdt)
    b = (seeded((n_out,), torch.float32, 60) * 0.1).to(cdt)
    print(f"window_proj register path {dims} C={C} n_out={n_out} {cdt}", flush=True)
    got = fused_block.window_proj_3d(win.to(dev), w.to(dev), b.to(dev), B, D, H, W, ws, ss)
    want = oracle.window_proj(win.double().numpy(), B, D, H, W, ws, ss, w.double().numpy(), b.double().numpy(),
                              NAME[cdt])
    assert got.shape == want.shape
    _compare(got, want, cdt, f"window_proj {dims} C={C} n_out={n_out}")
    got_nb = fused_block.window_proj_3d(win.to(dev), w.to(dev), None, B, D, H, W, ws, ss)
    want_nb = oracle.window_proj(win.double().numpy(), B, D, H, W, ws, ss, w.double().numpy(), None, NAME[cdt])
    _compare(got_nb, want_nb, cdt, "no bias")


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
def test_window_proj_stage0_full_size(oracle, dev, cdt):
    """Config-5 stage 0 at full size: [1372, 343, 48] windows -> [4, 48^3, 48],
    every output token against the oracle (27,648 tiles over several steps
    per wave)."""
    B, D, C, ws, ss = 4, 48, 48, (7, 7, 7), (3, 3, 3)
    win = seeded((B * 343, 343, C), torch.float32, 61).to(cdt)
    w = (seeded((C, C), torch.float32, 62) / C ** 0.5).to(cdt)
    b = (seeded((C,), torch.float32, 63) * 0.1).to(cdt)
    print(f"window_proj stage 0 full size {cdt}", flush=True)
    got = fused_block.window_proj_3d(win.to(dev), w.to(dev), b.to(dev), B, D, D, D, ws, ss)
    want = oracle.window_proj(win.double().numpy(), B, D, D, D, ws, ss, w.double().numpy(), b.double().numpy(),
                              NAME[cdt])
    _compare(got, want, cdt, "window_proj stage 0")


def test_many_tiles_uneven_feature_chunks(oracle, dev):
    """Over 1024 token tiles (no feature split across the grid) and 208
    output features: two LDS chunks (192 + 16), so three of the four waves
    have no tile in the second chunk."""
    shape, ws, ss = (1, 40, 40, 40, 32), (7, 7, 7), (3, 3, 3)
    x = seeded(shape, torch.float16, 54)
    w = (seeded((208, 32), torch.float32, 55) / 32 ** 0.5).to(torch.float16)
    b = (seeded((208,), torch.float32, 56) * 0.1).to(torch.float16)
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), b.to(dev), ws, ss)
    want = oracle.window_qkv(x.double().numpy(), ws, ss, w.double().numpy(), b.double().numpy())
    _compare(got, want, torch.float16, "qkv 208 features")
    y = fused_block.window_proj_3d(got, (seeded((208, 208), torch.float32, 57) / 208 ** 0.5).to(torch.float16).to(dev),
                                   None, 1, 40, 40, 40, ws, ss)
    wp = (seeded((208, 208), torch.float32, 57) / 208 ** 0.5).to(torch.float16)
    want_y = oracle.window_proj(got.double().cpu().numpy(), 1, 40, 40, 40, ws, ss, wp.double().numpy())
    _compare(y, want_y, torch.float16, "proj 208 features")


def test_stage0_full_size_sampled(oracle, dev):
    """Config-5 stage 0 at full size ([4,48^3,48] fp32 block input, fp16
    compute, window 7, shift 3, padded to 49^3): 512 sampled tokens of qkv
    against the oracle (whose window order is the C oracle's partition), and
    the proj scatter checked as a permutation of a full-size identity."""
    B, D, C, ws, ss = 4, 48, 48, (7, 7, 7), (3, 3, 3)
    x = seeded((B, D, D, D, C), torch.float32, 80) * 1.5 + 0.25
    gw = seeded((C,), torch.float32, 81) * 0.5 + 1.0
    gb = seeded((C,), torch.float32, 82) * 0.1
    w = (seeded((3 * C, C), torch.float32, 83) / C ** 0.5).half()
    b = (seeded((3 * C,), torch.float32, 84) * 0.1).half()
    got = fused_block.window_qkv_3d(x.to(dev), w.to(dev), b.to(dev), ws, ss, gw.to(dev), gb.to(dev), 1e-5, True,
                                    torch.float16)
    nwin, n = B * 7 ** 3, 343
    assert got.shape == (nwin, n, 3 * C)
    # source row of every window-ordered token: partition an index volume
    # (padded with -1) with the C oracle
    idx = np.full((B, 49, 49, 49, 1), -1, dtype=np.int32)
    idx[:, :D, :D, :D, 0] = np.arange(B * D ** 3, dtype=np.int32).reshape(B, D, D, D)
    src = oracle.shift_partition(idx, ws, ss).reshape(-1)
    g = np.random.default_rng(85)
    pick = g.choice(nwin * n, size=512, replace=False)
    xs = x.reshape(-1, C).double().numpy()
    rows = np.zeros((512, C))
    inside = src[pick] >= 0
    rows[inside] = oracle.round_to(oracle.layer_norm(xs[src[pick][inside]], gw.double().numpy(),
                                                     gb.double().numpy(), 1e-5), "float16")
    want = oracle.round_to(rows @ w.double().numpy().T + b.double().numpy(), "float16")
    _compare(got.reshape(-1, 3 * C)[torch.from_numpy(pick).to(dev)], want, torch.float16, "stage 0 sampled")
    # proj with identity weights, fp32: the full window -> volume scatter with crop
    eye = torch.eye(C, device=dev)
    win = torch.from_numpy(np.where(src >= 0, src, -1).astype(np.float32)).to(dev)[:, None].expand(-1, C)
    y = fused_block.window_proj_3d(win.reshape(nwin, n, C).contiguous(), eye, None, B, D, D, D, ws, ss)
    want_y = torch.arange(B * D ** 3, dtype=torch.float32, device=dev)[:, None].expand(-1, C)
    assert torch.equal(y.reshape(-1, C), want_y)


def test_identity_round_trip_is_exact(dev):
    """Identity weights, no norm, fp32: proj(qkv(x)) reproduces x bit for bit."""
    shape, ws, ss = (2, 12, 12, 12, 48), (7, 7, 7), (3, 3, 3)
    x = seeded(shape, torch.float32, 53).to(dev)
    eye = torch.eye(48, device=dev)
    win = fused_block.window_qkv_3d(x, eye, None, ws, ss, normalize=False)
    back = fused_block.window_proj_3d(win, eye, None, 2, 12, 12, 12, ws, ss)
    assert torch.equal(back, x)


def test_invalid_arguments(dev):
    x = torch.zeros((1, 7, 7, 7, 24), device=dev)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        fused_block.window_qkv_3d(x, torch.zeros((48, 24), device=dev), None, (7, 7, 7), (3, 3, 3))
    x = torch.zeros((1, 7, 7, 7, 32), device=dev)
    with pytest.raises(RuntimeError, match="shift_size"):
        fused_block.window_qkv_3d(x, torch.zeros((48, 32), device=dev), None, (7, 7, 7), (7, 0, 0))
    with pytest.raises(RuntimeError, match="weight"):
        fused_block.window_qkv_3d(x, torch.zeros((48, 16), device=dev), None, (7, 7, 7), (3, 3, 3))
    empty = fused_block.window_qkv_3d(torch.zeros((0, 7, 7, 7, 32), device=dev),
                                      torch.zeros((48, 32), device=dev), None, (7, 7, 7), (3, 3, 3))
    assert empty.shape == (0, 343, 48)


@pytest.mark.parametrize("autocast", [False, True], ids=["fp32", "fp16-autocast"])
@pytest.mark.parametrize("dims,dim,heads,shift", [((12, 12, 12), 48, 3, 3), ((14, 14, 14), 96, 6, 3),
                                                  ((6, 6, 6), 384, 24, 0)])
def test_fused_forward_part1_matches_eager(dev, dims, dim, heads, shift, autocast):
    """The fused forward_part1 against the eager block's own forward_part1 with
    the MONAI mask (tensor path) and with the geometry (region path)."""
    torch.manual_seed(60)
    blk = sw.SwinTransformerBlock(dim=dim, num_heads=heads, window_size=(7, 7, 7),
                                  shift_size=(shift,) * 3).to(dev).eval()
    g = torch.Generator().manual_seed(61)
    x = torch.randn((2,) + dims + (dim,), generator=g).to(dev)
    ws, ss = sw.get_window_size(dims, blk.window_size, blk.shift_size)
    padded = tuple(-(-n // k) * k for n, k in zip(dims, ws))
    mask = sw.compute_mask(padded, ws, ss, dev) if any(s > 0 for s in ss) else None

    cdt = torch.float16 if autocast else torch.float32
    es = torch.empty((), dtype=cdt).element_size()
    if not monai_patch._fits_staging_tile(dim, es):  # C=384 in fp32: the patch keeps the unfused path
        with torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
            assert not monai_patch._fused_block_supported(blk, x)
        pytest.skip(f"C={dim} in {cdt} exceeds the staging tile (unfused path)")
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16, enabled=autocast):
        want = blk.forward_part1(x, mask).float()
        assert monai_patch._fused_block_supported(blk, x)
        got = monai_patch._fused_block_forward(blk, x, mask, sw).float()
        if mask is not None:
            setattr(mask, monai_patch._GEOMETRY_ATTR, (*padded, tuple(ws), tuple(ss)))
            got_region = monai_patch._fused_block_forward(blk, x, mask, sw).float()
            assert torch.equal(got_region, got) or (got_region - got).abs().max().item() < 1e-3
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"forward_part1 {dims} C={dim} autocast={autocast}: max-abs {err:.2e} (max {scale:.2f})", flush=True)
    assert err < (1e-2 * scale if autocast else 1e-4 * max(1.0, scale))


@pytest.mark.parametrize("cdt", [torch.float16, torch.bfloat16, torch.float32], ids=["f16", "bf16", "f32"])
@pytest.mark.parametrize("dims,C,heads,ws,ss", [((9, 10, 11), 48, 3, (7, 7, 7), (3, 3, 3)),
                                                 ((14, 14, 14), 96, 6, (7, 7, 7), (3, 3, 3)),
                                                 ((6, 6, 6), 192, 12, (6, 6, 6), (0, 0, 0))],
                         ids=["padded-shifted", "s1-shifted", "6cubed-noshift"])
def test_window_msa_op_equals_the_three_calls(dev, dims, C, heads, ws, ss, cdt):
    """window_msa_3d (one dispatcher call) runs the same three kernels as
    window_qkv_3d -> fused_swin_attention[_shifted] -> window_proj_3d called
    one by one: bit-identical output."""
    _skip_unsupported(C, cdt)
    print(f"window_msa_3d {dims} C={C} {cdt}", flush=True)
    B = 2
    x = seeded((B,) + dims + (C,), torch.float32, 70 + C).to(dev)
    wq = (seeded((3 * C, C), torch.float32, 71) / C ** 0.5).to(cdt).to(dev)
    bq = (seeded((3 * C,), torch.float32, 72) * 0.1).to(cdt).to(dev)
    wp = (seeded((C, C), torch.float32, 73) / C ** 0.5).to(cdt).to(dev)
    bp = (seeded((C,), torch.float32, 74) * 0.1).to(cdt).to(dev)
    nw = (1.0 + 0.1 * seeded((C,), torch.float32, 75)).to(dev)
    nb = (0.1 * seeded((C,), torch.float32, 76)).to(dev)
    n = ws[0] * ws[1] * ws[2]
    bias = (seeded((heads, n, n), torch.float32, 77) * 0.1).to(dev)
    scale = (C // heads) ** -0.5
    got = torch.ops.crumpet_ops.window_msa_3d(x, nw, nb, 1e-5, wq, bq, wp, bp, bias, heads, scale, *ws, *ss)

    qkv = fused_block.window_qkv_3d(x, wq, bq, ws, ss, nw, nb, 1e-5, True, cdt)
    nwin = qkv.shape[0]
    t = qkv.view(nwin, n, 3, heads, C // heads).permute(2, 0, 3, 1, 4)
    attn = torch.empty((nwin, n, heads, C // heads), dtype=cdt, device=dev)
    ov = attn.permute(0, 2, 1, 3)
    ops = torch.ops.crumpet_ops
    if any(ss):
        padded = tuple(-(-d // w) * w for d, w in zip(dims, ws))
        ops.fused_swin_attention_shifted(ov, t[0], t[1], t[2], bias, *padded, *ws, *ss, scale)
    else:
        ops.fused_swin_attention(ov, t[0], t[1], t[2], bias, None, None, scale)
    want = fused_block.window_proj_3d(attn.view(nwin, n, C), wp, bp, B, *dims, ws, ss)
    assert got.dtype == cdt and got.shape == (B,) + dims + (C,)
    assert torch.equal(got, want)
