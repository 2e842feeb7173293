"""Loader of the native libraries built by crumpet_amd._build.

``torch`` is imported before either library is opened so that the HIP
library binds to torch's HIP runtime.  Nothing here falls back to another
implementation: when the libraries are missing every compute entry point of
the package raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

PKG = Path(__file__).resolve().parent
HIP_LIB = PKG / "libcrumpet_hip.so"
OPS_LIB = PKG / "_crumpet_ops.so"

# Entry points declared in include/crumpet_hip.h.
C_ABI_SYMBOLS = (
    "crumpet_version",
    "crumpet_last_error",
    "crumpet_status_string",
    "crumpet_shift_partition_3d",
    "crumpet_unshift_unpartition_3d",
    "crumpet_shift_partition_3d_backward",
    "crumpet_unshift_unpartition_3d_backward",
    "crumpet_compute_attn_mask_3d",
    "crumpet_fused_swin_attention",
    "crumpet_fused_swin_attention_tiled",
    "crumpet_attn_mask_tiles",
    "crumpet_attn_mask_tiles_elements",
    "crumpet_fused_swin_attention_shifted",
    "crumpet_window_qkv_3d",
    "crumpet_window_proj_3d",
)

OP_NAMES = (
    "compute_attn_mask_3d",
    "fused_shift_partition_3d",
    "fused_shift_partition_3d_backward",
    "fused_unshift_unpartition_3d",
    "fused_unshift_unpartition_3d_backward",
    "fused_swin_attention",
    "fused_swin_attention_shifted",
    "fused_swin_attention_tiled",
    "attn_mask_tiles",
    "window_qkv_3d",
    "window_proj_3d",
    "window_msa_3d",
)

_hip = None
_ops = None
_error: str | None = None


def _load() -> None:
    # Only success is cached: after a failed attempt (e.g. the libraries were
    # not built yet) the next call tries again.
    global _hip, _ops, _error
    if _ops is not None:
        return
    _error = None
    try:
        if not HIP_LIB.exists() or not OPS_LIB.exists():
            raise OSError(
                f"{HIP_LIB.name} / {OPS_LIB.name} are not built; run "
                "`python -m crumpet_amd._build` or __graft_entry__.build()"
            )
        _hip = ctypes.CDLL(str(HIP_LIB), mode=ctypes.RTLD_GLOBAL)
        torch.ops.load_library(str(OPS_LIB))
        _ops = torch.ops.crumpet_ops
    except (OSError, RuntimeError) as exc:  # pragma: no cover - depends on the build
        _error = f"{type(exc).__name__}: {exc}"
        return
    _declare_fake_kernels()


def _mutating_op_fake(*args, **kwargs) -> None:
    """The crumpet_ops ops other than window_msa_3d write into a
    caller-allocated output and return nothing, so their fake (meta) kernel
    has nothing to do."""
    return None


def _window_msa_fake(x, norm_weight, norm_bias, eps, w_qkv, b_qkv, w_proj, b_proj, bias, heads, scale,
                     ws_d, ws_h, ws_w, ss_d, ss_h, ss_w):
    """window_msa_3d returns the block half's output, [B, D, H, W, C_out] in
    the weights' dtype."""
    B, D, H, W, _ = x.shape
    return x.new_empty((B, D, H, W, w_proj.shape[0]), dtype=w_qkv.dtype)


def _declare_fake_kernels() -> None:
    """Fake kernels for FakeTensor / torch.compile tracing of the ops (the
    reference registers the same no-op fakes: torch-ext/crumpet/__init__.py:50-73)."""
    for name in OP_NAMES:
        fake = _window_msa_fake if name == "window_msa_3d" else _mutating_op_fake
        try:
            torch.library.register_fake(f"crumpet_ops::{name}")(fake)
        except (RuntimeError, ValueError):
            pass  # already registered in this process


def ops():
    """The ``torch.ops.crumpet_ops`` namespace; raises if the extension is missing."""
    _load()
    if _ops is None:
        raise RuntimeError(f"crumpet_amd HIP extension is not available ({_error})")
    return _ops


def ops_or_none():
    _load()
    return _ops


def hip_library() -> ctypes.CDLL:
    """ctypes handle of libcrumpet_hip.so (the C ABI of include/crumpet_hip.h)."""
    _load()
    if _hip is None:
        raise RuntimeError(f"crumpet_amd HIP library is not available ({_error})")
    return _hip


def load_error() -> str | None:
    _load()
    return _error
