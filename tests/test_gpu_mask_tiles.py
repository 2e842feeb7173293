"""The tiled copy of a 16-bit mask (attn_mask_tiles) and attention reading it
(fused_swin_attention_tiled), checked against the row-major path:

* the layout, bit-exact against its definition (numpy, and a per-element
  loop on a small case), for strided masks, N from 1 to 512 and M > 1;
* attention with the tiled copy equal bit for bit to attention reading the
  mask itself, at every N where the tiled form runs (14 and 22 key tiles),
  in both head dims of the tuned kernel, every q / mask dtype pair, with and
  without boundary flags, broadcast / per-position / per-window masks, and
  the three-heads-per-workgroup form (interleaved qkv, no flags);
* the Python wrapper's reuse policy: the copy is made on the second call
  with one mask tensor, reused after, remade when the mask changes in
  place, and never matched to another tensor.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import crumpet_amd
from crumpet_amd import fused_attention
from crumpet_amd.fused_attention import fused_swin_attention, mask_tiles
from helpers import raw, seeded

pytestmark = pytest.mark.gpu

TILE_COUNTS = (1, 2, 4, 8, 14, 22, 32)


def tile_count(N):
    """The kernel's tile count for N, made even (the layout is in tile pairs)."""
    need = -(-N // 16)
    nt = next(c for c in TILE_COUNTS if c >= need)
    return nt + nt % 2


def tiles_definition(mask: np.ndarray) -> np.ndarray:
    """tiles[m][s][p][16 g + c][j][r] = mask[m][min(16 s + c, N - 1)][16 (2p + j) + 4 g + r], 0 past N."""
    M, N, _ = mask.shape
    strips, NT = -(-N // 16), tile_count(N)
    lane = np.arange(64)
    col, g = lane % 16, lane // 16
    out = np.zeros((M, strips, NT // 2, 64, 2, 4), dtype=mask.dtype)
    for s in range(strips):
        q = np.minimum(16 * s + col, N - 1)
        for t in range(NT):
            k = 16 * t + 4 * g[:, None] + np.arange(4)[None, :]
            vals = mask[:, q[:, None], np.minimum(k, N - 1)]
            out[:, s, t // 2, :, t % 2] = np.where((k < N)[None], vals, 0)
    return out.reshape(-1)


def random_mask(M, N, dtype, seed, row_pad=0):
    """Values in {0, -100} and random normals, as a view with row stride N + row_pad."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn((M, N, N + row_pad), generator=g)
    base = torch.where(torch.rand((M, N, N + row_pad), generator=g) > 0.7, torch.full_like(base, -100.0), base)
    return base.to(dtype)[:, :, :N]


def test_layout_definition_by_hand():
    """The numpy definition against a per-element walk (N = 17: two strips, a
    partial second strip and tile)."""
    M, N = 2, 17
    mask = np.arange(M * N * N, dtype=np.int16).reshape(M, N, N)
    got = tiles_definition(mask)
    assert got.size == M * 2 * 2 * 256
    i = 0  # the flat order: m, strip, tile pair, lane, tile in pair, key
    for m in range(M):
        for s in range(2):
            for p in range(1):
                for lane in range(64):
                    for j in range(2):
                        for r in range(4):
                            q, k = min(16 * s + lane % 16, N - 1), 16 * (2 * p + j) + 4 * (lane // 16) + r
                            assert got[i] == (mask[m, q, k] if k < N else 0)
                            i += 1


@pytest.mark.parametrize("N", [1, 15, 16, 17, 129, 200, 224, 225, 343, 352, 512])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_tiles_layout(dev, N, dtype):
    M = 3
    mask = random_mask(M, N, dtype, 7000 + N, row_pad=3)
    got = mask_tiles(mask.to(dev))
    np.testing.assert_array_equal(raw(got), tiles_definition(raw(mask)))


def _qkv(B, H, N, Dh, dtype, seed):
    return [seeded((B, H, N, Dh), dtype, seed + i).to(dtype) for i in range(3)]


@pytest.mark.parametrize("N", [129, 200, 224, 225, 343, 352])
@pytest.mark.parametrize("Dh", [16, 32])
@pytest.mark.parametrize("dtype,mdtype", [(torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.bfloat16), (torch.bfloat16, torch.float16)],
                         ids=["f16-f16", "bf16-bf16", "f16-bf16", "bf16-f16"])
def test_tiled_equals_row_major(dev, N, Dh, dtype, mdtype):
    print(f"tiled attention N={N} Dh={Dh} {dtype} mask {mdtype}", flush=True)
    B, H, nW = 6, 2, 3
    q, k, v = (t.to(dev) for t in _qkv(B, H, N, Dh, dtype, 7100 + N))
    bias = (seeded((H, N, N), torch.float32, 7110 + N) * 0.1).to(dtype).to(dev)
    ops = crumpet_amd._native.ops()
    for M, flags in ((nW, torch.tensor([1, 0, 1, 1, 0, 0], dtype=torch.uint8)), (B, None), (1, None)):
        mask = random_mask(M, N, mdtype, 7120 + N + M).to(dev)
        bnd = flags.to(dev) if flags is not None else None
        tiles = mask_tiles(mask)
        want = torch.empty_like(q)
        got = torch.empty_like(q)
        ops.fused_swin_attention(want, q, k, v, bias, mask, bnd, 0.25)
        ops.fused_swin_attention_tiled(got, q, k, v, bias, mask, tiles, bnd, 0.25)
        assert torch.equal(got, want), (M, flags is not None)


@pytest.mark.parametrize("N", [216, 343])
def test_tiled_three_heads_per_workgroup(dev, N):
    """q, k, v as views of an interleaved [B, N, 3, 3, 16] qkv buffer with a
    per-position 16-bit mask and no boundary flags: the three-heads form."""
    B, H, Dh, nW = 8, 3, 16, 4
    print(f"tiled attention, 3 heads per workgroup, N={N}", flush=True)
    qkv = seeded((B, N, 3 * H * Dh), torch.float16, 7200 + N).to(dev)
    t = qkv.reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4)
    bias = (seeded((H, N, N), torch.float32, 7210 + N) * 0.1).half().to(dev)
    mask = random_mask(nW, N, torch.float16, 7220 + N).to(dev)
    ops = crumpet_amd._native.ops()
    want = torch.empty((B, H, N, Dh), dtype=torch.float16, device=dev)
    got = torch.empty_like(want)
    ops.fused_swin_attention(want, t[0], t[1], t[2], bias, mask, None, 0.25)
    ops.fused_swin_attention_tiled(got, t[0], t[1], t[2], bias, mask, mask_tiles(mask), None, 0.25)
    assert torch.equal(got, want)


def test_wrapper_reuse_policy(dev):
    """The copy is made at the second call with a mask and reused; an in-place
    change of the mask (a new version) is read, never a stale copy."""
    B, H, N, Dh = 4, 2, 343, 16
    q, k, v = (t.to(dev) for t in _qkv(B, H, N, Dh, torch.float16, 7300))
    bias = (seeded((H, N, N), torch.float32, 7310) * 0.1).half().to(dev)
    mask = random_mask(B, N, torch.float16, 7320).to(dev)
    ops = crumpet_amd._native.ops()

    def plain():
        out = torch.empty_like(q)
        ops.fused_swin_attention(out, q, k, v, bias, mask, None, 0.25)
        return out

    fused_attention._tiled.clear()
    fused_attention._seen.clear()
    first = fused_swin_attention(q, k, v, bias, mask, None, 0.25)
    assert not fused_attention._tiled
    second = fused_swin_attention(q, k, v, bias, mask, None, 0.25)
    assert len(fused_attention._tiled) == 1
    tiles = next(iter(fused_attention._tiled.values()))[2]
    third = fused_swin_attention(q, k, v, bias, mask, None, 0.25)
    assert next(iter(fused_attention._tiled.values()))[2] is tiles
    want = plain()
    assert torch.equal(first, want) and torch.equal(second, want) and torch.equal(third, want)

    mask[:, :, : N // 2] = -100.0  # in place: a new version of the same storage
    changed = fused_swin_attention(q, k, v, bias, mask, None, 0.25)
    assert torch.equal(changed, plain()) and not torch.equal(changed, want)
    again = fused_swin_attention(q, k, v, bias, mask, None, 0.25)  # second sight: a new copy
    assert torch.equal(again, changed)
    assert len(fused_attention._tiled) == 1
    assert next(iter(fused_attention._tiled.values()))[2] is not tiles

    # a new tensor with the same values (possibly at the recycled address of
    # a freed one) is a new mask: read as it is on its first call
    other = mask.clone()
    before = len(fused_attention._seen)
    assert torch.equal(fused_swin_attention(q, k, v, bias, other, None, 0.25), changed)
    assert len(fused_attention._seen) == before + 1
