"""CPU tests of the MONAI patch plumbing and of the in-repo MONAI-compatible model.

The reference's own test (tests/test_monai_patch.py:8-13) checks that
patch/unpatch are idempotent; here the in-repo model is always present, so
it runs unconditionally.  The compat model's window partition, mask and
relative-position index are pinned against the oracle (itself pinned in
test_oracle.py).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import crumpet_amd
from crumpet_amd import monai_patch
from crumpet_amd import swin_unetr_compat as sw
from oracle import oracle


def test_patch_unpatch_repeated_safe():
    assert crumpet_amd.patch_monai_swin_unetr() is True
    assert crumpet_amd.patch_monai_swin_unetr() is False
    assert crumpet_amd.unpatch_monai_swin_unetr() is True
    assert crumpet_amd.unpatch_monai_swin_unetr() is False


def test_patch_swaps_and_restores_methods():
    originals = (sw.SwinTransformerBlock.forward_part1, sw.BasicLayer.forward, sw.WindowAttention.forward)
    assert crumpet_amd.patch_monai_swin_unetr() is True
    try:
        patched = (sw.SwinTransformerBlock.forward_part1, sw.BasicLayer.forward, sw.WindowAttention.forward)
        for p, o in zip(patched, originals):
            assert p is not o
            assert p.__wrapped__ is o
        assert monai_patch.is_patched()
    finally:
        crumpet_amd.unpatch_monai_swin_unetr()
    restored = (sw.SwinTransformerBlock.forward_part1, sw.BasicLayer.forward, sw.WindowAttention.forward)
    assert all(r is o for r, o in zip(restored, originals))


def test_disable_fused_attention_env(monkeypatch):
    monkeypatch.setenv("CRUMPET_DISABLE_FUSED_ATTN", "1")
    original = sw.WindowAttention.forward
    assert crumpet_amd.patch_monai_swin_unetr() is True
    try:
        assert sw.WindowAttention.forward is original
        assert sw.BasicLayer.forward is not original
    finally:
        crumpet_amd.unpatch_monai_swin_unetr()


@pytest.mark.parametrize("dims,ws,ss", [((14, 14, 14), (7, 7, 7), (3, 3, 3)),
                                        ((12, 8, 6), (6, 4, 3), (3, 2, 1)),
                                        ((28, 28, 28), (7, 7, 7), (3, 3, 3))])
def test_compat_mask_equals_oracle(dims, ws, ss):
    got = sw.compute_mask(dims, ws, ss, "cpu").numpy()
    want = oracle.attn_mask(*dims, ws, ss, "float32")
    assert got.dtype == np.float32
    np.testing.assert_array_equal(got, want)


def test_compat_partition_and_reverse_equal_oracle():
    g = torch.Generator().manual_seed(3)
    x = torch.randn((2, 14, 7, 21, 5), generator=g)
    ws, ss = (7, 7, 7), (3, 2, 4)
    rolled = torch.roll(x, shifts=tuple(-s for s in ss), dims=(1, 2, 3))
    win = sw.window_partition(rolled, ws)
    np.testing.assert_array_equal(win.numpy(), oracle.shift_partition(x.numpy(), ws, ss))
    back = torch.roll(sw.window_reverse(win, ws, (2, 14, 7, 21)), shifts=ss, dims=(1, 2, 3))
    assert torch.equal(back, x)


def test_compat_relative_position_index_equals_oracle():
    att = sw.WindowAttention(48, 3, (7, 7, 7))
    np.testing.assert_array_equal(att.relative_position_index.numpy(),
                                  oracle.relative_position_index((7, 7, 7)))


def test_compat_get_window_size_matches_oracle():
    for size in [(49, 49, 49), (6, 6, 6), (7, 3, 9)]:
        assert sw.get_window_size(size, (7, 7, 7), (3, 3, 3)) == oracle.get_window_size(size, (7, 7, 7), (3, 3, 3))


def test_compat_swin_unetr_shapes_on_cpu():
    torch.manual_seed(0)
    m = sw.SwinUNETR(in_channels=1, out_channels=3, feature_size=12, depths=(1, 1, 1, 1),
                     num_heads=(3, 3, 3, 3)).eval()
    with torch.no_grad():
        y = m(torch.rand(1, 1, 64, 64, 64))
    assert y.shape == (1, 3, 64, 64, 64)
    assert torch.isfinite(y).all()


def test_compat_feature48_parameter_count():
    # MONAI's SwinUNETR(feature_size=48, depths (2,2,2,2), heads (3,6,12,24), out 14) has 62.19 M parameters
    m = sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=48)
    assert sum(p.numel() for p in m.parameters()) == 62_187_296


def test_module_cache_follows_parameter_updates():
    """The fused block's cached bias gather and weight casts are recomputed
    when a source tensor changes in place (version counter) or is replaced
    (storage), and reused otherwise."""
    import torch

    from crumpet_amd import monai_patch
    from crumpet_amd.swin_unetr_compat import WindowAttention

    torch.manual_seed(3)
    attn = WindowAttention(dim=48, num_heads=3, window_size=(7, 7, 7), qkv_bias=True)
    first = monai_patch._window_bias(attn, 343)
    assert first.shape == (3, 343, 343)
    assert monai_patch._window_bias(attn, 343) is first
    idx = attn.relative_position_index[:343, :343].reshape(-1)
    assert torch.equal(first, attn.relative_position_bias_table.t()[:, idx].view(3, 343, 343))
    with torch.no_grad():
        attn.relative_position_bias_table.add_(1.0)  # in place: version bump
    second = monai_patch._window_bias(attn, 343)
    assert second is not first and torch.equal(second, first + 1.0)
    # a smaller window (the 6^3 stage rule) is a separate entry
    assert monai_patch._window_bias(attn, 216).shape == (3, 216, 216)

    # the fused block's entry: bias and both projections in the compute dtype
    bias, (w, b), (wp, bp) = monai_patch._block_params(attn, 343, torch.float16)
    assert torch.equal(bias, second)
    assert w.dtype == torch.float16 and w.is_contiguous() and torch.equal(w, attn.qkv.weight.half())
    assert torch.equal(bp, attn.proj.bias.half())
    again = monai_patch._block_params(attn, 343, torch.float16)
    assert again[1][0] is w and again[0] is bias
    attn.qkv.weight = torch.nn.Parameter(torch.zeros_like(attn.qkv.weight))  # replaced: new storage
    _, (w2, _), _ = monai_patch._block_params(attn, 343, torch.float16)
    assert w2 is not w and not w2.any()
    with torch.no_grad():
        attn.proj.bias.mul_(2.0)  # in place: version bump
    _, _, (_, bp2) = monai_patch._block_params(attn, 343, torch.float16)
    assert torch.equal(bp2, attn.proj.bias.half())
    # the compute dtype equal to the parameters' returns them as they are
    _, (w3, b3), _ = monai_patch._block_params(attn, 343, torch.float32)
    assert w3 is attn.qkv.weight and b3 is attn.qkv.bias
