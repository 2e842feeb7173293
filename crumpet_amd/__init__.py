"""crumpet_amd: MI355X (gfx950) shifted-window kernels behind the crumpet API.

Public functions keep the reference's names, arguments, validation and
error types (torch-ext/crumpet/__init__.py:89-378):

* ``compute_attn_mask_3d(D, H, W, window_size, shift_size, dtype, device)``
* ``fused_shift_partition_3d(x, window_size, shift_size)``
* ``fused_unshift_unpartition_3d(windows, B, D, H, W, C, window_size, shift_size)``
* ``crumpet_amd.fused_attention.fused_swin_attention(q, k, v, bias, mask, boundary, scale)``
* ``patch_monai_swin_unetr()`` / ``unpatch_monai_swin_unetr()``
* ``clear_mask_cache()`` / ``mask_cache_info()``

All tensors are channels-last ``[B, D, H, W, C]``.  Compute runs only in the
hand-written HIP kernels of libcrumpet_hip.so, reached through the
``torch.ops.crumpet_ops`` dispatcher ops.  There is no eager or CPU
fallback: a tensor on another device, or a missing extension, raises
``RuntimeError``.  Meta tensors are supported for shape propagation.
"""

from __future__ import annotations

import contextlib
import functools
import os
from typing import Sequence

import torch

from . import _native
from ._geometry import WindowGrid, as_triple, require_float_dtype
from .cache import clear_mask_cache, get_or_compute_mask, make_mask_key, mask_cache_info

__version__ = "0.1.0"

_HAS_HIP_EXT = _native.ops_or_none() is not None


class _RoctxRange:
    """A roctx range (``torch.cuda.nvtx`` is roctx on ROCm builds of torch)."""

    __slots__ = ("_name",)

    def __init__(self, name: str):
        self._name = name

    def __enter__(self):
        torch.cuda.nvtx.range_push(self._name)
        return self

    def __exit__(self, *exc) -> bool:
        torch.cuda.nvtx.range_pop()
        return False


def _op_range(name: str):
    """A roctx range around one op call when CRUMPET_ENABLE_NVTX=1 (none
    while torch.compile traces)."""
    if (os.environ.get("CRUMPET_ENABLE_NVTX", "0") != "1" or torch.compiler.is_compiling()
            or not torch.cuda.is_available()):
        return contextlib.nullcontext()
    return _RoctxRange(name)


@functools.lru_cache(maxsize=256)
def _checked_grid(D, H, W, window_size, shift_size) -> WindowGrid:
    return WindowGrid.checked(D, H, W, window_size, shift_size)


def _grid(D: int, H: int, W: int, window_size, shift_size) -> WindowGrid:
    """``WindowGrid.checked``, kept for hashable arguments: the deep Swin
    stages are host-bound, and validating the same geometry on every call
    was about half of a gather call's Python time.  Invalid arguments raise
    every time (exceptions are not cached); lists are validated each call,
    and so is everything under torch.compile, which traces the check."""
    if torch.compiler.is_compiling():
        return WindowGrid.checked(D, H, W, window_size, shift_size)
    try:
        return _checked_grid(D, H, W, window_size, shift_size)
    except TypeError:  # unhashable window / shift sizes
        return WindowGrid.checked(D, H, W, window_size, shift_size)


def _device_ops(device: torch.device, what: str):
    """The op namespace for a HIP tensor; any other device raises."""
    if device.type != "cuda":
        raise RuntimeError(
            f"{what}: crumpet_amd runs only on HIP (MI355X) devices; got a tensor on '{device}'"
        )
    return _native.ops()


def compute_attn_mask_3d(
    D: int,
    H: int,
    W: int,
    window_size: Sequence[int],
    shift_size: Sequence[int],
    dtype: torch.dtype,
    device: torch.device | str,
) -> torch.Tensor:
    """Shifted 3D Swin attention mask ``[nW, vol, vol]``: 0 where region ids match, -100 elsewhere.

    Cached per ``(D, H, W, window_size, shift_size, dtype, device)``
    (reference: torch-ext/crumpet/__init__.py:139-182).
    """
    window_size = as_triple("window_size", window_size)
    shift_size = as_triple("shift_size", shift_size)
    require_float_dtype(dtype)
    grid = WindowGrid.checked(D, H, W, window_size, shift_size)
    dev = torch.device(device)
    shape = (grid.num_windows, grid.volume, grid.volume)
    if dev.type == "meta":
        return torch.empty(shape, dtype=dtype, device=dev)
    ops = _device_ops(dev, "compute_attn_mask_3d")

    def build() -> torch.Tensor:
        mask = torch.empty(shape, dtype=dtype, device=dev)
        with _op_range("crumpet.compute_attn_mask_3d"):
            ops.compute_attn_mask_3d(mask, *grid.dims, *grid.op_args)
        return mask

    key = make_mask_key(*grid.dims, grid.window, grid.shift, dtype, dev)
    return get_or_compute_mask(key, build)


def _to_windows(x: torch.Tensor, grid: WindowGrid) -> torch.Tensor:
    """Shift-partition gather of a contiguous ``[B, D, H, W, C]`` volume."""
    batch, channels = x.shape[0], x.shape[4]
    out = x.new_empty(grid.windows_shape(batch, channels))
    _native.ops().fused_shift_partition_3d(out, x, *grid.op_args)
    return out


def _to_volume(windows: torch.Tensor, grid: WindowGrid, batch: int) -> torch.Tensor:
    """Unshift-unpartition gather of contiguous ``[B*nW, vol, C]`` windows."""
    channels = windows.shape[2]
    out = windows.new_empty(grid.volume_shape(batch, channels))
    _native.ops().fused_unshift_unpartition_3d(out, windows, batch, *grid.dims, channels, *grid.op_args)
    return out


class _WindowPermute(torch.autograd.Function):
    """One of the two window permutations with autograd.

    Partition and unpartition are permutations of the same elements, each
    the inverse of the other, so the gradient of one is the other applied to
    the incoming gradient (the reference's ``*_backward`` ops are exactly
    these gathers, torch_binding.cpp:22-24,29-31).
    """

    @staticmethod
    def forward(ctx, src: torch.Tensor, grid: WindowGrid, to_windows: bool, batch: int):
        ctx.grid, ctx.to_windows, ctx.batch = grid, to_windows, batch
        src = src.contiguous()
        return _to_windows(src, grid) if to_windows else _to_volume(src, grid, batch)

    @staticmethod
    def backward(ctx, grad: torch.Tensor):
        grad = grad.contiguous()
        if ctx.to_windows:
            grad_src = _to_volume(grad, ctx.grid, ctx.batch)
        else:
            grad_src = _to_windows(grad, ctx.grid)
        return grad_src, None, None, None


def fused_shift_partition_3d(
    x: torch.Tensor,
    window_size: Sequence[int],
    shift_size: Sequence[int],
) -> torch.Tensor:
    """Cyclic shift by ``-shift_size`` plus 3D window partition of ``[B, D, H, W, C]``.

    Returns ``[B * nW, ws_d * ws_h * ws_w, C]`` (reference:
    torch-ext/crumpet/__init__.py:257-290).  Zero shift runs the same kernel.
    """
    if x.ndim != 5:
        raise ValueError("x must have shape [B, D, H, W, C]")
    require_float_dtype(x.dtype)
    batch, D, H, W, channels = map(int, x.shape)
    grid = _grid(D, H, W, window_size, shift_size)
    if x.device.type == "meta":
        return x.new_empty(grid.windows_shape(batch, channels))
    _device_ops(x.device, "fused_shift_partition_3d")
    with _op_range("crumpet.fused_shift_partition_3d"):
        if torch.is_grad_enabled() and x.requires_grad:
            return _WindowPermute.apply(x, grid, True, batch)
        return _to_windows(x.contiguous(), grid)


def fused_unshift_unpartition_3d(
    windows: torch.Tensor,
    B: int,
    D: int,
    H: int,
    W: int,
    C: int,
    window_size: Sequence[int],
    shift_size: Sequence[int],
) -> torch.Tensor:
    """3D window reverse plus cyclic shift by ``+shift_size``: ``[B*nW, vol, C] -> [B, D, H, W, C]``.

    Reference: torch-ext/crumpet/__init__.py:293-351.
    """
    if windows.ndim != 3:
        raise ValueError("windows must have shape [B * num_windows, window_volume, C]")
    require_float_dtype(windows.dtype)
    grid = _grid(D, H, W, window_size, shift_size)
    batch, channels = int(B), int(C)
    expected = grid.windows_shape(batch, channels)
    if tuple(map(int, windows.shape)) != expected:
        raise ValueError(f"windows must have shape {expected}")
    if windows.device.type == "meta":
        return windows.new_empty(grid.volume_shape(batch, channels))
    _device_ops(windows.device, "fused_unshift_unpartition_3d")
    with _op_range("crumpet.fused_unshift_unpartition_3d"):
        if torch.is_grad_enabled() and windows.requires_grad:
            return _WindowPermute.apply(windows, grid, False, batch)
        return _to_volume(windows.contiguous(), grid, batch)


def patch_monai_swin_unetr() -> bool:
    from .monai_patch import patch_monai_swin_unetr as patch

    return patch()


def unpatch_monai_swin_unetr() -> bool:
    from .monai_patch import unpatch_monai_swin_unetr as unpatch

    return unpatch()


__all__ = [
    "compute_attn_mask_3d",
    "fused_shift_partition_3d",
    "fused_unshift_unpartition_3d",
    "patch_monai_swin_unetr",
    "unpatch_monai_swin_unetr",
    "clear_mask_cache",
    "mask_cache_info",
]
