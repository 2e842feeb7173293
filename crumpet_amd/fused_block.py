"""Fused window-MSA block of a 3D Swin transformer on MI355X.

A Swin block's attention half (MONAI ``SwinTransformerBlock.forward_part1``,
patched by torch-ext/crumpet/monai_patch.py:72-114 in the reference) is

    norm1 -> zero-pad to the window grid -> roll(-shift) -> window partition
    -> qkv Linear -> window attention -> proj Linear
    -> window reverse -> roll(+shift) -> crop

Here it is three gfx950 kernels:

* ``window_qkv_3d``: LayerNorm, padding, shift, partition and the qkv
  projection in one pass over the block input (``crumpet_window_qkv_3d``);
* the fused window attention (``crumpet_fused_swin_attention[_shifted]``),
  reading q, k, v as strided views of the qkv buffer;
* ``window_proj_3d``: the proj projection in output (volume) order, the
  reverse partition, shift and crop folded into its row gathers
  (``crumpet_window_proj_3d``).

The layout changes never touch HBM as separate passes.  Numerics follow the
eager chain under autocast: LayerNorm in fp32, its output rounded once to
the compute dtype, fp32 accumulation, bias added before the final rounding.
"""

from __future__ import annotations

from typing import Sequence

import torch

from . import _native
from ._geometry import as_triple, padded_dims, require_float_dtype
from .fused_attention import fused_swin_attention_windows

def _check(x: torch.Tensor, what: str) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(f"{what}: crumpet_amd runs only on HIP (MI355X) devices; got '{x.device}'")
    require_float_dtype(x.dtype)


def _num_windows(padded, window_size):
    return (padded[0] // window_size[0]) * (padded[1] // window_size[1]) * (padded[2] // window_size[2])


def window_qkv_3d(
    x: torch.Tensor,  # [B, D, H, W, C]
    weight: torch.Tensor,  # [n_out, C]
    bias: torch.Tensor | None,  # [n_out]
    window_size: Sequence[int],
    shift_size: Sequence[int],
    norm_weight: torch.Tensor | None = None,
    norm_bias: torch.Tensor | None = None,
    eps: float = 1e-5,
    normalize: bool = True,
    dtype: torch.dtype | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``[B*nW, N, n_out]``: ``LN(x)`` zero-padded to the window grid, shifted
    by ``-shift_size``, partitioned into windows and projected by
    ``weight``/``bias``, in ``dtype`` (default ``x.dtype``; ``weight`` and
    ``bias`` are cast to it, as autocast casts a Linear's parameters)."""
    _check(x, "window_qkv_3d")
    ws = as_triple("window_size", window_size, signed=True)
    ss = as_triple("shift_size", shift_size, signed=True)
    if x.dim() != 5:
        raise ValueError("x must have shape [B, D, H, W, C]")
    dtype = x.dtype if dtype is None else dtype
    require_float_dtype(dtype)
    B, D, H, W, _ = x.shape
    padded = padded_dims((D, H, W), ws)
    n = ws[0] * ws[1] * ws[2]
    w = weight.to(dtype).contiguous()
    b = bias.to(dtype).contiguous() if bias is not None else None
    if out is None:
        out = torch.empty((B * _num_windows(padded, ws), n, w.shape[0]), dtype=dtype, device=x.device)
    _native.ops().window_qkv_3d(out, x.contiguous(), norm_weight, norm_bias, float(eps), bool(normalize),
                                w, b, *ws, *ss)
    return out


def window_proj_3d(
    windows: torch.Tensor,  # [B*nW, N, C]
    weight: torch.Tensor,  # [n_out, C]
    bias: torch.Tensor | None,
    B: int,
    D: int,
    H: int,
    W: int,
    window_size: Sequence[int],
    shift_size: Sequence[int],
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``[B, D, H, W, n_out]``: ``windows @ weight^T + bias`` put back in volume
    order (inverse partition over the padded grid, shift by ``+shift_size``)
    and cropped to ``D, H, W``; in the dtype of ``windows``."""
    _check(windows, "window_proj_3d")
    ws = as_triple("window_size", window_size, signed=True)
    ss = as_triple("shift_size", shift_size, signed=True)
    dtype = windows.dtype
    w = weight.to(dtype).contiguous()
    b = bias.to(dtype).contiguous() if bias is not None else None
    if out is None:
        out = torch.empty((int(B), int(D), int(H), int(W), w.shape[0]), dtype=dtype, device=windows.device)
    _native.ops().window_proj_3d(out, windows.contiguous(), w, b, *ws, *ss)
    return out


def _linear(m):
    """(weight, bias) of a Linear module, or the pair itself."""
    return (m.weight, m.bias) if isinstance(m, torch.nn.Linear) else tuple(m)


def fused_window_msa_3d(
    x: torch.Tensor,  # [B, D, H, W, C] block input (before norm1)
    norm: torch.nn.LayerNorm,
    qkv,  # torch.nn.Linear, or its (weight, bias)
    proj,  # torch.nn.Linear, or its (weight, bias)
    relative_position_bias: torch.Tensor,  # [heads, N, N]
    num_heads: int,
    scale: float,
    window_size: Sequence[int],
    shift_size: Sequence[int],
    mask: torch.Tensor | None = None,
    region: bool = True,
    dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """The attention half of a Swin block, ``[B, D, H, W, C]`` in ``dtype``.

    With a non-zero shift the shifted-window mask is derived from the padded
    volume's geometry (``region=True``, nothing is read) or taken from
    ``mask`` (``[nW, N, N]``, window b reads ``mask[b mod nW]``).  ``qkv`` and
    ``proj`` are Linear modules or ``(weight, bias)`` pairs; weights already
    in ``dtype`` and contiguous are used as they are (no cast kernel).
    Without a mask tensor the three kernels run from one dispatcher call
    (``window_msa_3d``); with one, the boundary flags are computed and the
    kernels are called one by one.
    """
    ws = as_triple("window_size", window_size, signed=True)
    ss = as_triple("shift_size", shift_size, signed=True)
    B, D, H, W, C = x.shape
    dtype = x.dtype if dtype is None else dtype
    wq, bq = _linear(qkv)
    wp, bp = _linear(proj)
    shifted = any(s > 0 for s in ss)
    if region or not shifted:
        # the three kernels in one dispatcher call (window_msa_3d), which
        # allocates the qkv and attention intermediates itself
        _check(x, "fused_window_msa_3d")
        require_float_dtype(dtype)
        wq, bq, wp, bp = (None if t is None else t.to(dtype).contiguous() for t in (wq, bq, wp, bp))
        return _native.ops().window_msa_3d(x, norm.weight, norm.bias, float(norm.eps), wq, bq, wp, bp,
                                           relative_position_bias, int(num_heads), float(scale), *ws, *ss)
    hd = C // num_heads
    n = ws[0] * ws[1] * ws[2]
    qkv_out = window_qkv_3d(x, wq, bq, ws, ss, norm.weight, norm.bias, norm.eps, True, dtype)
    nwin = qkv_out.shape[0]
    t = qkv_out.view(nwin, n, 3, num_heads, hd).permute(2, 0, 3, 1, 4)
    attn = torch.empty((nwin, n, num_heads, hd), dtype=dtype, device=x.device)
    ov = attn.permute(0, 2, 1, 3)
    if mask is not None:
        nw = mask.shape[0]
        flags = (mask.reshape(nw, -1).abs().amax(dim=1) > 0).to(torch.uint8)
        fused_swin_attention_windows(t[0], t[1], t[2], relative_position_bias, mask,
                                     flags.repeat(nwin // nw).contiguous(), scale, ov)
    else:
        fused_swin_attention_windows(t[0], t[1], t[2], relative_position_bias, None, None, scale, ov)
    return window_proj_3d(attn.view(nwin, n, C), wp, bp, B, D, H, W, ws, ss)
