"""Reversible patch of MONAI-style Swin UNETR models onto the gfx950 kernels.

Same entry points and patched methods as torch-ext/crumpet/monai_patch.py:
``patch_monai_swin_unetr()`` (idempotent; True when it installs the patch,
False when already active) and ``unpatch_monai_swin_unetr()`` (restores
the originals; True / False likewise) replace

* ``SwinTransformerBlock.forward_part1``: norm1, pad to the window grid,
  ``fused_shift_partition_3d``, window attention,
  ``fused_unshift_unpartition_3d``, crop (reference :72-114).  In inference
  mode, with a LayerNorm norm1 and Linear qkv / proj, the whole method runs
  as three kernels instead (``crumpet_amd.fused_block``): norm1 + pad +
  shift + partition + qkv in one, the fused attention, and proj + reverse +
  unshift + crop in one (opt out with ``CRUMPET_DISABLE_FUSED_BLOCK=1``);
* ``BasicLayer.forward``: channels-last stage loop with the cached
  ``compute_attn_mask_3d`` mask (reference :201-232);
* ``WindowAttention.forward``: the eager ``q k^T + bias + mask -> softmax
  -> @ v`` chain becomes one gfx950 kernel call (reference :117-198).  It
  falls back to the original in training mode, with attention dropout,
  when ``CRUMPET_DISABLE_FUSED_ATTN=1``, or for a head dimension other
  than 16, 32, 64, 128 or 256 (the kernels' head dimensions; every stage of
  the feature-size-48 Swin UNETR has 16, feature size 96 gives 32).  The
  reference takes the fused path for any head dimension from 16 up
  (reference :144-149), which its Triton kernel compiles for powers of two.

Differences from the reference's patched attention, none of which changes
the math:

* q, k and v are passed to the kernel as strided views of the qkv linear's
  output (no ``.contiguous()`` copies), and the kernel writes straight into
  a ``[b, n, H, hd]`` buffer, so the ``transpose(1, 2).reshape`` copy
  disappears;
* in a shifted block whose mask came from the patched ``BasicLayer`` the
  kernel derives the shifted-window mask from the window geometry
  (``fused_swin_attention_shifted``): nothing is tiled with
  ``mask.repeat`` and no mask or boundary flags are read.  Any other mask is
  read as ``mask[b mod nW]`` with boundary flags computed on the ``nW``
  distinct windows only;
* the relative-position bias stays in the table's dtype (fp32), as in the
  eager MONAI chain, instead of being rounded to the activation dtype.

MONAI is optional: the patch applies to ``monai.networks.nets.swin_unetr``
when it is importable, and always to ``crumpet_amd.swin_unetr_compat`` (the
in-repo MONAI-compatible model used when MONAI is absent).
"""

from __future__ import annotations

import functools
import os
from typing import Any

import torch
import torch.nn.functional as F

from . import compute_attn_mask_3d, fused_shift_partition_3d, fused_unshift_unpartition_3d
from .fused_attention import fused_swin_attention_shifted, fused_swin_attention_windows
from .fused_block import fused_window_msa_3d

_STATE: dict[str, Any] = {}
_REQUIRED = ("SwinTransformerBlock", "BasicLayer", "WindowAttention", "get_window_size")
# Attribute names: the mask geometry tag set by the patched BasicLayer, and the
# per-call region handed from forward_part1 to the attention module.
_GEOMETRY_ATTR = "_crumpet_geometry"
_REGION_ATTR = "_crumpet_region"


def _fused_attn_enabled() -> bool:
    """Opt-out via ``CRUMPET_DISABLE_FUSED_ATTN=1`` (reference monai_patch.py:47-51)."""
    return os.environ.get("CRUMPET_DISABLE_FUSED_ATTN", "0") != "1"


def _swin_modules() -> list:
    """Modules to patch: MONAI's swin_unetr if importable, plus the in-repo one."""
    mods = []
    try:
        import monai.networks.nets.swin_unetr as monai_swin  # noqa: F401

        if all(hasattr(monai_swin, n) for n in _REQUIRED):
            mods.append(monai_swin)
    except Exception:
        pass
    from . import swin_unetr_compat

    mods.append(swin_unetr_compat)
    return mods


def _as_triple(value) -> tuple[int, int, int]:
    if len(value) != 3:
        raise RuntimeError("CRUMPET MONAI patch only supports 3D Swin blocks")
    return tuple(int(v) for v in value)


def _fused_block_enabled() -> bool:
    """Opt-out of the fused block projections via ``CRUMPET_DISABLE_FUSED_BLOCK=1``."""
    return os.environ.get("CRUMPET_DISABLE_FUSED_BLOCK", "0") != "1"


def _compute_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype the block's Linear layers run in: autocast's, else x's."""
    if torch.is_autocast_enabled(x.device.type):
        return torch.get_autocast_dtype(x.device.type)
    return x.dtype


_ESIZE = {torch.float32: 4, torch.float16: 2, torch.bfloat16: 2}
# head dimensions of the fused attention kernels
_HEAD_DIMS = (16, 32, 64, 128, 256)


def _fits_staging_tile(c: int, esize: int) -> bool:
    """The projections' LDS tile (window_linear.hip plan_tile): 64 staged rows
    of C channels, an output chunk of at least 16 features (rows padded by
    16 bytes each) and 64 row indices within 64 KiB."""
    pad = 16 // esize
    return 64 * (c + pad) * esize + 64 * (16 + pad) * esize + 64 * 4 <= 64 * 1024


def _fused_block_supported(block, x: torch.Tensor) -> bool:
    """Inference-mode blocks whose attention half the fused block kernels
    cover: LayerNorm norm1 over C, Linear qkv / proj, a head dimension the
    attention kernels take, no attention dropout, C a multiple of 16 that
    fits the staging tile."""
    attn = block.attn
    c = x.shape[-1]
    if block.training or not (_fused_attn_enabled() and _fused_block_enabled()):
        return False
    if x.device.type != "cuda" or x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        return False
    norm = block.norm1
    if not isinstance(norm, torch.nn.LayerNorm) or tuple(norm.normalized_shape) != (c,):
        return False
    if not isinstance(attn.qkv, torch.nn.Linear) or not isinstance(attn.proj, torch.nn.Linear):
        return False
    if attn.qkv.out_features != 3 * c or attn.proj.in_features != c or attn.proj.out_features != c:
        return False
    if attn.attn_drop.p != 0.0 or c % attn.num_heads != 0 or c // attn.num_heads not in _HEAD_DIMS:
        return False
    return c % 16 == 0 and c <= 384 and _fits_staging_tile(c, _ESIZE[_compute_dtype(x)])


def _cached(module, key, sources, make):
    """``make()`` for ``key``, kept on ``module`` until a tensor in ``sources``
    changes: an in-place update bumps its version counter, reassigning it
    changes its storage.  Under graph capture nothing is cached or reused:
    the value is recomputed by kernels the graph records, so every replay
    reads the parameters as they are then (the reference recomputes the bias
    on every call for that reason, torch-ext/crumpet/monai_patch.py:157-162)."""
    if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
        return make()
    stamp = tuple((t._version, t.data_ptr()) for t in sources)
    cache = module.__dict__.setdefault("_crumpet_cache", {})
    hit = cache.get(key)
    if hit is not None and hit[0] == stamp:
        return hit[1]
    with torch.no_grad():
        value = make()
    cache[key] = (stamp, value)
    return value


def _window_bias(attn, n):
    """``[heads, n, n]`` relative-position bias of the first ``n`` window
    tokens, gathered from the transposed table (unit stride along keys) and
    kept in the table's dtype; cached on the module (``_cached``)."""
    def make():
        idx = attn.relative_position_index[:n, :n].reshape(-1)
        return attn.relative_position_bias_table.t()[:, idx].view(attn.num_heads, n, n)

    return _cached(attn, ("bias", n), (attn.relative_position_bias_table, attn.relative_position_index), make)


def _block_params(attn, n, dtype):
    """``(bias, (w_qkv, b_qkv), (w_proj, b_proj))`` of a window-attention
    module for the fused block: the gathered ``[heads, n, n]`` bias and both
    projections cast to ``dtype``, kept as one entry on the module
    (``_cached``), so a call checks the sources' versions once."""
    def make():
        idx = attn.relative_position_index[:n, :n].reshape(-1)
        bias = attn.relative_position_bias_table.t()[:, idx].view(attn.num_heads, n, n)
        cast = lambda t: None if t is None else t.to(dtype).contiguous()  # noqa: E731
        return bias, (cast(attn.qkv.weight), cast(attn.qkv.bias)), (cast(attn.proj.weight), cast(attn.proj.bias))

    sources = tuple(t for t in (attn.relative_position_bias_table, attn.relative_position_index,
                                attn.qkv.weight, attn.qkv.bias, attn.proj.weight, attn.proj.bias)
                    if t is not None)
    return _cached(attn, ("block", n, dtype), sources, make)


def _fused_block_forward(block, x, mask_matrix, swin):
    """forward_part1 as three kernels: window_qkv_3d (norm1, pad, shift,
    partition, qkv), the fused attention, window_proj_3d (proj, reverse,
    unshift, crop), launched by one dispatcher call unless a mask tensor
    without the geometry tag is passed.  The gathered bias and the cast
    projection weights are cached per module."""
    b, d, h, w, c = x.shape
    window_size, shift_size = swin.get_window_size((d, h, w), block.window_size, block.shift_size)
    ws = _as_triple(window_size)
    ss = _as_triple(shift_size)
    padded = tuple(-(-n // k) * k for n, k in zip((d, h, w), ws))
    attn = block.attn
    n = ws[0] * ws[1] * ws[2]
    dtype = _compute_dtype(x)
    bias, qkv, proj = _block_params(attn, n, dtype)
    shifted = any(s > 0 for s in ss)
    region = shifted and getattr(mask_matrix, _GEOMETRY_ATTR, None) == (*padded, ws, ss)
    return fused_window_msa_3d(x, block.norm1, qkv, proj, bias, attn.num_heads, attn.scale, ws, ss,
                               mask=mask_matrix if shifted else None, region=region, dtype=dtype)


def _patched_forward_part1(original, swin):
    @functools.wraps(original)
    def forward_part1(self, x, mask_matrix):
        if x.dim() != 5:
            return original(self, x, mask_matrix)
        if _fused_block_supported(self, x):
            return _fused_block_forward(self, x, mask_matrix, swin)
        x = self.norm1(x)
        b, d, h, w, c = x.shape
        window_size, shift_size = swin.get_window_size((d, h, w), self.window_size, self.shift_size)
        window_size = _as_triple(window_size)
        shift_size = _as_triple(shift_size)
        pad_d1 = (window_size[0] - d % window_size[0]) % window_size[0]
        pad_b = (window_size[1] - h % window_size[1]) % window_size[1]
        pad_r = (window_size[2] - w % window_size[2]) % window_size[2]
        if pad_d1 > 0 or pad_b > 0 or pad_r > 0:
            x = F.pad(x, (0, 0, 0, pad_r, 0, pad_b, 0, pad_d1))
        _, dp, hp, wp, _ = x.shape

        shifted = any(s > 0 for s in shift_size)
        attn_mask = mask_matrix if shifted else None
        region = None
        if shifted and getattr(mask_matrix, _GEOMETRY_ATTR, None) == (dp, hp, wp, window_size, shift_size):
            region = ((dp, hp, wp), window_size, shift_size)

        x_windows = fused_shift_partition_3d(x, window_size, shift_size)
        setattr(self.attn, _REGION_ATTR, region)
        try:
            attn_windows = self.attn(x_windows, mask=attn_mask)
        finally:
            setattr(self.attn, _REGION_ATTR, None)
        x = fused_unshift_unpartition_3d(attn_windows, B=b, D=dp, H=hp, W=wp, C=c,
                                         window_size=window_size, shift_size=shift_size)
        if pad_d1 > 0 or pad_r > 0 or pad_b > 0:
            x = x[:, :d, :h, :w, :].contiguous()
        return x

    return forward_part1


def _patched_window_attention_forward(original):
    @functools.wraps(original)
    def forward(self, x, mask):
        if self.training or self.attn_drop.p != 0.0 or not _fused_attn_enabled():
            return original(self, x, mask)
        b, n, c = x.shape
        heads = self.num_heads
        hd = c // heads
        if hd not in _HEAD_DIMS or hd * heads != c:
            return original(self, x, mask)

        qkv = self.qkv(x)  # [b, n, 3c]; channel = s*c + h*hd + d
        t = qkv.view(b, n, 3, heads, hd).permute(2, 0, 3, 1, 4)  # views [b, H, n, hd]
        bias = _window_bias(self, n)
        out = torch.empty((b, n, heads, hd), dtype=qkv.dtype, device=qkv.device)
        ov = out.permute(0, 2, 1, 3)
        region = getattr(self, _REGION_ATTR, None)
        if mask is not None and region is not None:
            volume, ws, ss = region
            fused_swin_attention_shifted(t[0], t[1], t[2], bias, volume, ws, ss, self.scale, ov)
        elif mask is not None:
            nw = mask.shape[0]
            flags = (mask.reshape(nw, -1).abs().amax(dim=1) > 0).to(torch.uint8)
            boundary = flags.repeat(b // nw).contiguous()
            fused_swin_attention_windows(t[0], t[1], t[2], bias, mask, boundary, self.scale, ov)
        else:
            fused_swin_attention_windows(t[0], t[1], t[2], bias, None, None, self.scale, ov)
        x = self.proj(out.view(b, n, c))
        return self.proj_drop(x)

    return forward


def _patched_basic_layer_forward(original, swin):
    @functools.wraps(original)
    def forward(self, x):
        if x.dim() != 5:
            return original(self, x)
        b, c, d, h, w = x.shape
        window_size, shift_size = swin.get_window_size((d, h, w), self.window_size, self.shift_size)
        window_size = _as_triple(window_size)
        shift_size = _as_triple(shift_size)
        x = x.permute(0, 2, 3, 4, 1).contiguous()
        dp = -(-d // window_size[0]) * window_size[0]
        hp = -(-h // window_size[1]) * window_size[1]
        wp = -(-w // window_size[2]) * window_size[2]
        attn_mask = compute_attn_mask_3d(D=dp, H=hp, W=wp, window_size=window_size,
                                         shift_size=shift_size, dtype=x.dtype, device=x.device)
        setattr(attn_mask, _GEOMETRY_ATTR, (dp, hp, wp, window_size, shift_size))
        for blk in self.blocks:
            x = blk(x, attn_mask)
        x = x.view(b, d, h, w, -1)
        if self.downsample is not None:
            x = self.downsample(x)
        return x.permute(0, 4, 1, 2, 3).contiguous()

    return forward


def patch_monai_swin_unetr() -> bool:
    """Install the patch.  Returns True on the call that installs it and False
    if it is already active (reference monai_patch.py:235-261)."""
    if _STATE.get("patched"):
        return False
    saved = []
    for swin in _swin_modules():
        orig = (swin.SwinTransformerBlock.forward_part1, swin.BasicLayer.forward,
                swin.WindowAttention.forward)
        saved.append((swin, orig))
        swin.SwinTransformerBlock.forward_part1 = _patched_forward_part1(orig[0], swin)
        swin.BasicLayer.forward = _patched_basic_layer_forward(orig[1], swin)
        if _fused_attn_enabled():
            swin.WindowAttention.forward = _patched_window_attention_forward(orig[2])
    _STATE.update({"patched": True, "saved": saved})
    return True


def unpatch_monai_swin_unetr() -> bool:
    """Restore the original methods.  Returns True if a patch was removed
    (reference monai_patch.py:264-275)."""
    if not _STATE.get("patched"):
        return False
    for swin, orig in _STATE["saved"]:
        swin.SwinTransformerBlock.forward_part1 = orig[0]
        swin.BasicLayer.forward = orig[1]
        swin.WindowAttention.forward = orig[2]
    _STATE.clear()
    return True


def is_patched() -> bool:
    return bool(_STATE.get("patched"))
