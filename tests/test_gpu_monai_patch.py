"""GPU parity of the patched MONAI-style Swin UNETR with its own eager forward.

The reference pins its patch only by idempotence (tests/test_monai_patch.py)
and by a hd=4 demo that bypasses fused attention
(tests/test_demo_btcv_smoke.py:37-39).  Here the patched forwards
(partition / attention / unpartition kernels, both attention mask modes)
are compared with the unpatched eager forwards of the same modules and
weights, at the Swin UNETR stage shapes (window 7, shift 3, padding to the
window grid, the 6^3 stage with window 6 and no shift):

* fp32: the kernels compute in fp32, so the patched block matches eager to
  1e-4 (absolute, activations of order 1);
* fp16 autocast: eager rounds the scores to fp16 before adding the bias,
  the kernel keeps them in fp32, so the bound is 1e-2 relative to the
  largest activation.

Each model-level test runs twice: through the fused block projections
(norm1 + pad + shift + partition + qkv, and proj + reverse + crop, as
kernels) and through the partition / attention / unpartition path with
torch's LayerNorm and Linear layers (CRUMPET_DISABLE_FUSED_BLOCK=1).
"""

from __future__ import annotations

import pytest
import torch

import crumpet_amd
from crumpet_amd import monai_patch
from crumpet_amd import swin_unetr_compat as sw

pytestmark = pytest.mark.gpu


@pytest.fixture
def patched():
    crumpet_amd.unpatch_monai_swin_unetr()
    yield
    crumpet_amd.unpatch_monai_swin_unetr()


def _run(module, *args, autocast=False, dtype=torch.float16):
    with torch.no_grad(), torch.autocast("cuda", dtype=dtype, enabled=autocast):
        return module(*args)


def _layer(dim, heads, seed, depth=2):
    torch.manual_seed(seed)
    return sw.BasicLayer(dim=dim, depth=depth, num_heads=heads, window_size=(7, 7, 7), drop_path=0.0,
                         qkv_bias=True, downsample=None)


@pytest.fixture(params=["fused-block", "unfused-block"])
def block_mode(request, monkeypatch):
    """Run a test through the fused block projections and through the
    partition / attention / unpartition path."""
    monkeypatch.setenv("CRUMPET_DISABLE_FUSED_BLOCK", "0" if request.param == "fused-block" else "1")
    return request.param


@pytest.mark.parametrize("dims,dim,heads", [((12, 12, 12), 48, 3),   # padded to 14^3, shifted
                                            ((14, 14, 14), 96, 6),   # no padding, shifted
                                            ((6, 6, 6), 384, 24)])   # window 6, no shift (N=216)
def test_patched_basic_layer_matches_eager_fp32(patched, dev, dims, dim, heads, block_mode):
    layer = _layer(dim, heads, 0).to(dev).eval()
    g = torch.Generator().manual_seed(1)
    x = torch.randn((2, dim) + dims, generator=g).to(dev)
    want = _run(layer, x)
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(layer, x)
    err = (got - want).abs().max().item()
    print(f"basic layer {dims} C={dim}: max-abs {err:.2e}", flush=True)
    assert err < 1e-4


def test_patched_basic_layer_fp16_autocast(patched, dev, block_mode):
    layer = _layer(48, 3, 2).to(dev).eval()
    g = torch.Generator().manual_seed(3)
    x = torch.randn((2, 48, 12, 12, 12), generator=g).to(dev)
    want = _run(layer, x, autocast=True).float()
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(layer, x, autocast=True).float()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"fp16 autocast: max-abs {err:.2e} (max |x| {scale:.2f})", flush=True)
    assert err < 1e-2 * scale


@pytest.mark.parametrize("dims,dim,heads", [((12, 12, 12), 48, 3), ((6, 6, 6), 384, 24)])
def test_patched_basic_layer_bf16_autocast(patched, dev, dims, dim, heads, block_mode):
    """bf16 autocast: eager rounds q k^T to bf16 before the bias and the
    softmax, the kernel keeps the scores in fp32, so the bound is 1e-2
    relative to the largest activation, the north-star bf16 tolerance
    (measured: about 1.6e-3)."""
    layer = _layer(dim, heads, 4).to(dev).eval()
    g = torch.Generator().manual_seed(5)
    x = torch.randn((2, dim) + dims, generator=g).to(dev)
    want = _run(layer, x, autocast=True, dtype=torch.bfloat16).float()
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(layer, x, autocast=True, dtype=torch.bfloat16).float()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"bf16 autocast {dims} C={dim}: max-abs {err:.2e} (max |x| {scale:.2f})", flush=True)
    assert err < 1e-2 * scale


@pytest.mark.parametrize("fused_block_on", [True, False], ids=["fused-block", "unfused-block"])
def test_region_mode_reads_no_mask(patched, dev, monkeypatch, fused_block_on):
    """A shifted block under the patched BasicLayer takes the geometry path,
    with and without the fused block projections (the fused block runs its
    kernels through the one-call window_msa_3d op, whose shift selects the
    geometry mask)."""
    from crumpet_amd import _native, fused_block

    monkeypatch.setenv("CRUMPET_DISABLE_FUSED_BLOCK", "0" if fused_block_on else "1")
    calls = []
    real_ops = _native.ops

    class OpsSpy:
        def window_msa_3d(self, *args):
            calls.append("msa-region" if any(args[-3:]) else "msa-none")
            return real_ops().window_msa_3d(*args)

        def __getattr__(self, name):
            return getattr(real_ops(), name)

    spy_ops = OpsSpy()
    monkeypatch.setattr(_native, "ops", lambda: spy_ops)
    for mod, names in ((monai_patch, ("fused_swin_attention_windows", "fused_swin_attention_shifted")),
                       (fused_block, ("fused_swin_attention_windows",))):
        for name in names:
            real = getattr(mod, name)
            tag = "region" if name.endswith("shifted") else None

            def spy(*args, _real=real, _tag=tag, **kw):
                calls.append(_tag or ("tensor" if args[4] is not None else "none"))
                return _real(*args, **kw)

            monkeypatch.setattr(mod, name, spy)
    layer = _layer(48, 3, 4).to(dev).eval()
    x = torch.randn((1, 48, 14, 14, 14), device=dev)
    assert crumpet_amd.patch_monai_swin_unetr()
    _run(layer, x)
    # block 0 has no shift; block 1 reads no mask
    assert calls == (["msa-none", "msa-region"] if fused_block_on else ["none", "region"])


def test_block_with_foreign_mask_uses_tensor_mask(patched, dev):
    """A mask that did not come from the patched BasicLayer is read as a tensor (mask[b mod nW])."""
    torch.manual_seed(5)
    blk = sw.SwinTransformerBlock(dim=48, num_heads=3, window_size=(7, 7, 7), shift_size=(3, 3, 3)).to(dev).eval()
    x = torch.randn((3, 14, 14, 14, 48), device=dev)
    mask = sw.compute_mask((14, 14, 14), (7, 7, 7), (3, 3, 3), dev)
    want = _run(blk, x, mask)
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(blk, x, mask)
    err = (got - want).abs().max().item()
    print(f"foreign mask: max-abs {err:.2e}", flush=True)
    assert err < 1e-4


def test_patched_swin_unetr_matches_eager_fp32(patched, dev, block_mode):
    torch.manual_seed(7)
    model = sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=48).to(dev).eval()
    g = torch.Generator().manual_seed(8)
    x = torch.rand((1, 1, 64, 64, 64), generator=g).to(dev)
    want = _run(model, x)
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(model, x)
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"SwinUNETR 64^3 fp32: max-abs logit delta {err:.2e} (max |logit| {scale:.2f})", flush=True)
    assert err < 1e-4 * max(1.0, scale)


def _config5_model(dev):
    torch.manual_seed(123)
    return sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=48, depths=(2, 2, 2, 2),
                        num_heads=(3, 6, 12, 24)).to(dev).eval()


def test_config5_swin_unetr_fp16_autocast(patched, dev, block_mode):
    """BASELINE config 5 as the reference benchmarks it
    (benchmarks/bench_e2e.py:27-53): SwinUNETR(1 -> 14, feature 48, depths
    2222, heads 3/6/12/24) on a [4,1,96,96,96] fp16 synthetic CT volume under
    fp16 autocast, patched against the unpatched eager forward of the same
    weights.  Eager rounds q k^T to fp16 before the bias, the kernels keep
    the scores in fp32, so the bound is 1e-2 of the largest logit."""
    from helpers import synthetic_ct

    model = _config5_model(dev)
    x = synthetic_ct((4, 1, 96, 96, 96), 77).half().to(dev)
    want = _run(model, x, autocast=True).float()
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(model, x, autocast=True).float()
    assert got.shape == (4, 14, 96, 96, 96)
    assert torch.isfinite(got).all()
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"config 5 fp16 autocast ({block_mode}): max-abs logit delta {err:.2e} "
          f"(max |logit| {scale:.2f})", flush=True)
    assert err <= 1e-2 * scale


def test_config5_swin_unetr_fp32(patched, dev, block_mode):
    """Config 5's model and input shape in fp32: the kernels compute in fp32,
    so patched and eager logits agree to 1e-4 of the largest logit."""
    from helpers import synthetic_ct

    model = _config5_model(dev)
    x = synthetic_ct((4, 1, 96, 96, 96), 77).to(dev)
    want = _run(model, x)
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(model, x)
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"config 5 fp32 ({block_mode}): max-abs logit delta {err:.2e} (max |logit| {scale:.2f})",
          flush=True)
    assert err <= 1e-4 * scale


def test_training_mode_falls_back_and_backpropagates(patched, dev):
    torch.manual_seed(9)
    layer = _layer(48, 3, 9, depth=2).to(dev).train()
    x = torch.randn((1, 48, 14, 14, 14), device=dev, requires_grad=True)
    want = layer(x)
    want.square().mean().backward()
    g_want = x.grad.clone()
    x.grad = None
    assert crumpet_amd.patch_monai_swin_unetr()
    got = layer(x)
    got.square().mean().backward()
    assert (got - want).abs().max().item() < 1e-4
    assert (x.grad - g_want).abs().max().item() < 1e-5


def test_unsupported_head_dim_is_bit_exact_fp16(patched, dev):
    """tests/test_demo_btcv_smoke.py:37-39 of the reference: with head_dim 4
    (feature size 12) the fused attention and the fused block are bypassed,
    the patched model runs the partition / unpartition kernels and the mask
    kernel around MONAI's own attention, and its fp16 logits equal the eager
    model's exactly."""
    torch.manual_seed(10)
    model = sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=12).to(dev).eval()
    g = torch.Generator().manual_seed(11)
    x = torch.rand((1, 1, 64, 64, 64), generator=g).half().to(dev)
    want = _run(model, x, autocast=True)
    assert crumpet_amd.patch_monai_swin_unetr()
    got = _run(model, x, autocast=True)
    print(f"hd=4 fp16: max-abs logit delta {(got - want).abs().max().item():.2e}", flush=True)
    assert torch.equal(got, want)
