"""Fused 3D Swin window attention on MI355X.

``fused_swin_attention`` keeps the signature and argument semantics of the
reference wrapper (torch-ext/crumpet/fused_attention.py:149-226); the
computation runs in the gfx950 HIP kernel behind the
``crumpet_ops::fused_swin_attention`` dispatcher op:

    out[b, h] = softmax(q[b,h] * scale @ k[b,h]^T + bias[h]
                        + (boundary[b] ? mask[b] : 0)) @ v[b,h]

The kernel reads q, k, v through their strides (no ``.contiguous()``
copies are needed) and writes ``out`` through its strides.  ``block_m`` and
``block_n`` are accepted for API compatibility; the HIP kernels' tiling is
fixed by the MFMA shape (16-query strips, 16-key tiles).  Head dim 16 with
up to 512 tokens per window (every Swin UNETR stage) runs the tuned kernel;
head dims 32, 64, 128 and 256, and larger windows, run the general kernel
(the head dims the reference's Triton kernel takes: powers of two from 16).
"""

from __future__ import annotations

import ctypes
import weakref
from collections import OrderedDict

import torch

from . import _native

# Tiled copies of 16-bit masks (``attn_mask_tiles``): in the tiled layout a
# wave's mask words of one key tile are 512 contiguous bytes instead of 16
# row pieces, which the tuned kernels read faster (config 3: about 7% of the
# tensor-mask launch).  A copy is made the second time one mask tensor
# object is passed and kept for the most recent masks only.  It is used
# while that object is alive and its version counter (bumped by every
# in-place torch op on it or on a view of it) and storage are unchanged;
# writes that bypass torch's version counter (raw pointers, DLPack) are not
# seen.  A new tensor, even at a recycled address, is never matched.
_TILED_KEEP = 2
_tiled: "OrderedDict[int, tuple]" = OrderedDict()  # id -> (weakref, stamp, tiles)
_seen: "OrderedDict[int, tuple]" = OrderedDict()  # id -> (weakref, stamp)


def _stamp(mask: torch.Tensor) -> tuple | None:
    try:
        return (mask.device, mask.data_ptr(), mask._version, tuple(mask.shape), tuple(mask.stride()), mask.dtype)
    except (RuntimeError, NotImplementedError):  # fake / functional tensors while tracing
        return None


def _matches(entry, mask: torch.Tensor, stamp: tuple) -> bool:
    return entry is not None and entry[0]() is mask and entry[1] == stamp


def _tiles_elements(M: int, N: int) -> int:
    f = _native.hip_library().crumpet_attn_mask_tiles_elements
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64, ctypes.c_int64]
    return int(f(M, N))


def mask_tiles(mask: torch.Tensor) -> torch.Tensor:
    """The tiled copy of a 16-bit ``[M, N, N]`` mask that
    ``fused_swin_attention`` reads when it can (one launch; 1 <= N <= 512)."""
    M, N = int(mask.shape[0]), int(mask.shape[1])
    n = _tiles_elements(M, N)
    if n < 0:
        raise ValueError(f"attn_mask_tiles: N = {N} is outside 1 .. 512")
    out = torch.empty(n, dtype=mask.dtype, device=mask.device)
    _native.ops().attn_mask_tiles(out, mask)
    return out


def _cached_tiles(q: torch.Tensor, mask: torch.Tensor | None) -> torch.Tensor | None:
    """The kept tiled copy of ``mask`` for this call, or None (read the mask
    itself): only 16-bit masks with 2-byte q at head dim 16 or 32 and
    129 <= N <= 352 (the tuned kernels' 14- and 22-tile forms), never while
    a graph is captured or traced."""
    if mask is None or mask.dtype not in (torch.float16, torch.bfloat16):
        return None
    if q.dtype not in (torch.float16, torch.bfloat16) or q.shape[3] not in (16, 32):
        return None
    N = q.shape[2]
    if not 129 <= N <= 352 or mask.dim() != 3 or mask.shape[1] != N or mask.shape[2] != N:
        return None
    if torch.compiler.is_compiling() or (torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()):
        return None
    stamp = _stamp(mask)
    if stamp is None:
        return None
    key = id(mask)
    hit = _tiled.get(key)
    if _matches(hit, mask, stamp):
        _tiled.move_to_end(key)
        return hit[2]
    if not _matches(_seen.get(key), mask, stamp):
        _seen[key] = (weakref.ref(mask), stamp)
        _seen.move_to_end(key)
        while len(_seen) > 4 * _TILED_KEEP:
            _seen.popitem(last=False)
        return None
    del _seen[key]
    tiles = mask_tiles(mask)
    _tiled[key] = (weakref.ref(mask), stamp, tiles)
    _tiled.move_to_end(key)
    while len(_tiled) > _TILED_KEEP:
        _tiled.popitem(last=False)
    return tiles


def _attend(out, q, k, v, bias, mask, boundary, scale) -> None:
    tiles = _cached_tiles(q, mask)
    if tiles is not None:
        _native.ops().fused_swin_attention_tiled(out, q, k, v, bias, mask, tiles, boundary, float(scale))
    else:
        _native.ops().fused_swin_attention(out, q, k, v, bias, mask, boundary, float(scale))


def fused_swin_attention(
    q: torch.Tensor,  # [B, H, N, D]
    k: torch.Tensor,  # [B, H, N, D]
    v: torch.Tensor,  # [B, H, N, D]
    relative_position_bias: torch.Tensor,  # [H, N, N]
    mask: torch.Tensor | None,  # [num_windows (== B) or 1, N, N] or None
    boundary: torch.Tensor | None = None,  # [B] uint8 / bool
    scale: float | None = None,
    block_m: int = 64,
    block_n: int = 32,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Compute fused 3D Swin window attention.

    ``q``, ``k``, ``v`` have shape ``[B * num_windows, num_heads, N, head_dim]``.
    ``relative_position_bias`` is ``[num_heads, N, N]`` and broadcasts over the
    batch.  ``mask`` is ``[B, N, N]`` or ``[1, N, N]`` (broadcast), or ``None``.
    ``boundary`` is a per-window uint8/bool flag; a zero flag skips that
    window's mask.  With a mask and no flags every window reads its mask.
    ``out`` (optional, any strides, same shape/dtype as q) receives the result;
    by default a tensor like ``q`` is allocated.
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda
    assert q.shape == k.shape == v.shape, "Q/K/V shape mismatch"
    B, H, N, D = q.shape
    assert relative_position_bias.shape == (H, N, N)

    if scale is None:
        scale = 1.0 / (D ** 0.5)

    bnd = None
    if mask is not None:
        if mask.shape[0] != 1:
            assert mask.shape[0] == B, f"mask shape {mask.shape[0]} incompatible with B={B}"
        if boundary is not None:
            bnd = boundary if boundary.dtype == torch.uint8 else boundary.to(torch.uint8)
            bnd = bnd.contiguous()

    if out is None:
        out = torch.empty_like(q)
    _attend(out, q, k, v, relative_position_bias, mask, bnd, scale)
    return out


def fused_swin_attention_windows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    relative_position_bias: torch.Tensor,
    mask: torch.Tensor | None,
    boundary: torch.Tensor | None,
    scale: float,
    out: torch.Tensor,
) -> torch.Tensor:
    """Raw form used by the MONAI integration: ``mask`` may hold one mask per
    window position ``[nW, N, N]`` with ``nW`` dividing ``B``; window ``b``
    then reads ``mask[b % nW]`` (the layout MONAI's ``mask.repeat`` tiling
    produces, without materialising the repeat)."""
    _attend(out, q, k, v, relative_position_bias, mask, boundary, scale)
    return out


def fused_swin_attention_shifted(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    relative_position_bias: torch.Tensor,
    volume,
    window_size,
    shift_size,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Window attention with the shifted-window mask of a ``volume = (D, H, W)``.

    Equivalent to ``fused_swin_attention(q, k, v, bias, mask, None, scale)``
    with ``mask = compute_attn_mask_3d(D, H, W, window_size, shift_size)``
    repeated over the outer batch (window ``b`` uses the mask of window
    ``b % nW``), without materialising, repeating or reading the mask: the
    mask of a window depends only on which axes it is the last window along,
    and the kernel folds it into its register bias tiles whenever that
    window type changes.  ``q``'s batch must be a multiple of ``nW`` and
    ``N`` the window volume.
    """
    assert q.is_cuda and k.is_cuda and v.is_cuda
    assert q.shape == k.shape == v.shape, "Q/K/V shape mismatch"
    B, H, N, D = q.shape
    assert relative_position_bias.shape == (H, N, N)
    if scale is None:
        scale = 1.0 / (D ** 0.5)
    if out is None:
        out = torch.empty_like(q)
    Dv, Hv, Wv = (int(x) for x in volume)
    ws = tuple(int(x) for x in window_size)
    ss = tuple(int(x) for x in shift_size)
    _native.ops().fused_swin_attention_shifted(
        out, q, k, v, relative_position_bias, Dv, Hv, Wv, *ws, *ss, float(scale))
    return out


__all__ = ["fused_swin_attention", "fused_swin_attention_shifted", "mask_tiles"]
