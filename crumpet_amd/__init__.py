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
import os
from typing import Sequence

import torch

from . import _native
from .cache import clear_mask_cache, get_or_compute_mask, make_mask_key, mask_cache_info

__version__ = "0.1.0"

_ops = _native.ops_or_none()
_HAS_HIP_EXT = _ops is not None

_SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def _register_fake_impls() -> None:
    """No-op fake kernels so the mutating ops trace under torch.compile / FakeTensor."""
    if not _HAS_HIP_EXT:
        return
    register = getattr(torch.library, "register_fake", None)
    if register is None:
        return

    def _noop(*args, **kwargs):
        return None

    for name in _native.OP_NAMES:
        try:
            register(f"crumpet_ops::{name}")(_noop)
        except (RuntimeError, AttributeError, ValueError):
            pass


_register_fake_impls()


@contextlib.contextmanager
def _range(name: str):
    """roctx range around an op when CRUMPET_ENABLE_NVTX=1 (torch.cuda.nvtx is roctx on ROCm)."""
    if os.environ.get("CRUMPET_ENABLE_NVTX", "0") == "1" and torch.cuda.is_available():
        torch.cuda.nvtx.range_push(name)
        try:
            yield
        finally:
            torch.cuda.nvtx.range_pop()
    else:
        yield


def _triple(name: str, value: Sequence[int]) -> tuple[int, int, int]:
    if len(value) != 3:
        raise ValueError(f"{name} must contain exactly three values")
    out = tuple(int(v) for v in value)
    if any(v < 0 for v in out):
        raise ValueError(f"{name} values must be non-negative")
    return out


def _validate_shape(D: int, H: int, W: int, window_size, shift_size) -> None:
    if D <= 0 or H <= 0 or W <= 0:
        raise ValueError("D, H and W must be positive")
    if any(v <= 0 for v in window_size):
        raise ValueError("window_size values must be positive")
    if D % window_size[0] or H % window_size[1] or W % window_size[2]:
        raise ValueError(
            "standalone CRUMPET kernels require D, H and W to be divisible by window_size"
        )
    for axis, (shift, window) in enumerate(zip(shift_size, window_size)):
        if shift < 0 or shift >= window:
            raise ValueError(f"shift_size[{axis}] must satisfy 0 <= shift < window_size[{axis}]")


def _check_dtype(dtype: torch.dtype) -> None:
    if dtype not in _SUPPORTED_DTYPES:
        raise TypeError("CRUMPET supports torch.float32, torch.float16 and torch.bfloat16")


def _hip_ops(device: torch.device, what: str):
    """The op namespace for a HIP tensor; raises for any other device."""
    if device.type != "cuda":
        raise RuntimeError(
            f"{what}: crumpet_amd runs only on HIP (MI355X) devices; got a tensor on '{device}'"
        )
    return _native.ops()


def _windows_geometry(D, H, W, window_size):
    volume = window_size[0] * window_size[1] * window_size[2]
    num_windows = (D // window_size[0]) * (H // window_size[1]) * (W // window_size[2])
    return volume, num_windows


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
    window_size = _triple("window_size", window_size)
    shift_size = _triple("shift_size", shift_size)
    _check_dtype(dtype)
    D, H, W = int(D), int(H), int(W)
    _validate_shape(D, H, W, window_size, shift_size)
    dev = torch.device(device)
    volume, num_windows = _windows_geometry(D, H, W, window_size)
    if dev.type == "meta":
        return torch.empty((num_windows, volume, volume), dtype=dtype, device=dev)
    ops = _hip_ops(dev, "compute_attn_mask_3d")

    def compute() -> torch.Tensor:
        out = torch.empty((num_windows, volume, volume), dtype=dtype, device=dev)
        with _range("crumpet.compute_attn_mask_3d"):
            ops.compute_attn_mask_3d(out, D, H, W, *window_size, *shift_size)
        return out

    return get_or_compute_mask(make_mask_key(D, H, W, window_size, shift_size, dtype, dev), compute)


class _ShiftPartitionFn(torch.autograd.Function):
    """Partition forward; backward is the inverse gather (adjoint of a permutation)."""

    @staticmethod
    def forward(ctx, x, window_size, shift_size):
        x = x.contiguous()
        B, D, H, W, C = (int(v) for v in x.shape)
        volume, num_windows = _windows_geometry(D, H, W, window_size)
        out = torch.empty((B * num_windows, volume, C), dtype=x.dtype, device=x.device)
        _native.ops().fused_shift_partition_3d(out, x, *window_size, *shift_size)
        ctx.shape = (B, D, H, W, C)
        ctx.window_size = window_size
        ctx.shift_size = shift_size
        return out

    @staticmethod
    def backward(ctx, grad_output):
        B, D, H, W, C = ctx.shape
        grad_x = torch.empty((B, D, H, W, C), dtype=grad_output.dtype, device=grad_output.device)
        _native.ops().fused_shift_partition_3d_backward(
            grad_x, grad_output.contiguous(), B, D, H, W, C, *ctx.window_size, *ctx.shift_size
        )
        return grad_x, None, None


class _UnshiftUnpartitionFn(torch.autograd.Function):
    """Unpartition forward; backward is the partition gather."""

    @staticmethod
    def forward(ctx, windows, B, D, H, W, C, window_size, shift_size):
        windows = windows.contiguous()
        out = torch.empty((B, D, H, W, C), dtype=windows.dtype, device=windows.device)
        _native.ops().fused_unshift_unpartition_3d(
            out, windows, B, D, H, W, C, *window_size, *shift_size
        )
        ctx.window_size = window_size
        ctx.shift_size = shift_size
        return out

    @staticmethod
    def backward(ctx, grad_output):
        B, D, H, W, C = (int(v) for v in grad_output.shape)
        volume, num_windows = _windows_geometry(D, H, W, ctx.window_size)
        grad_windows = torch.empty(
            (B * num_windows, volume, C), dtype=grad_output.dtype, device=grad_output.device
        )
        _native.ops().fused_unshift_unpartition_3d_backward(
            grad_windows, grad_output.contiguous(), *ctx.window_size, *ctx.shift_size
        )
        return grad_windows, None, None, None, None, None, None, None


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
    window_size = _triple("window_size", window_size)
    shift_size = _triple("shift_size", shift_size)
    _check_dtype(x.dtype)
    B, D, H, W, C = (int(v) for v in x.shape)
    _validate_shape(D, H, W, window_size, shift_size)
    volume, num_windows = _windows_geometry(D, H, W, window_size)
    if x.device.type == "meta":
        return torch.empty((B * num_windows, volume, C), dtype=x.dtype, device=x.device)
    ops = _hip_ops(x.device, "fused_shift_partition_3d")
    with _range("crumpet.fused_shift_partition_3d"):
        if torch.is_grad_enabled() and x.requires_grad:
            return _ShiftPartitionFn.apply(x, window_size, shift_size)
        out = torch.empty((B * num_windows, volume, C), dtype=x.dtype, device=x.device)
        ops.fused_shift_partition_3d(out, x.contiguous(), *window_size, *shift_size)
        return out


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
    window_size = _triple("window_size", window_size)
    shift_size = _triple("shift_size", shift_size)
    _check_dtype(windows.dtype)
    B, D, H, W, C = (int(B), int(D), int(H), int(W), int(C))
    _validate_shape(D, H, W, window_size, shift_size)
    volume, num_windows = _windows_geometry(D, H, W, window_size)
    expected = (B * num_windows, volume, C)
    if tuple(int(v) for v in windows.shape) != expected:
        raise ValueError(f"windows must have shape {expected}")
    if windows.device.type == "meta":
        return torch.empty((B, D, H, W, C), dtype=windows.dtype, device=windows.device)
    ops = _hip_ops(windows.device, "fused_unshift_unpartition_3d")
    with _range("crumpet.fused_unshift_unpartition_3d"):
        if torch.is_grad_enabled() and windows.requires_grad:
            return _UnshiftUnpartitionFn.apply(
                windows, B, D, H, W, C, window_size, shift_size
            )
        out = torch.empty((B, D, H, W, C), dtype=windows.dtype, device=windows.device)
        ops.fused_unshift_unpartition_3d(
            out, windows.contiguous(), B, D, H, W, C, *window_size, *shift_size
        )
        return out


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
