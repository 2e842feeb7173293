"""LRU cache of shifted-window attention masks, keyed per device.

Same keys, limits and environment switches as the reference cache
(torch-ext/crumpet/cache.py:13-96):

* key ``(D, H, W, window_size, shift_size, dtype, device)``;
* ``CRUMPET_DISABLE_MASK_CACHE=1`` computes on every call;
* ``CRUMPET_MASK_CACHE_SIZE`` (default 64 entries) and
  ``CRUMPET_MASK_CACHE_MAX_BYTES`` (default 1 GiB) bound the cache, evicting
  least-recently-used entries; a single mask above the byte cap is returned
  without being stored.

Like the reference, the cache is a module-level ordered dict without a lock:
it is not thread-safe, and it is a convenience, not a lifetime guarantee.
"""

from __future__ import annotations

import os
from collections import OrderedDict
from typing import Callable

import torch

MaskKey = tuple

_entries: "OrderedDict[MaskKey, torch.Tensor]" = OrderedDict()
_bytes = 0

_DEFAULT_MAX_ENTRIES = 64
_DEFAULT_MAX_BYTES = 1 << 30


def _env_int(name: str, default: int) -> int:
    raw = os.environ.get(name)
    if raw is None:
        return default
    try:
        return int(raw)
    except ValueError:
        return default


def _disabled() -> bool:
    return os.environ.get("CRUMPET_DISABLE_MASK_CACHE", "0") == "1"


def _device_key(device) -> str:
    dev = torch.device(device)
    if dev.type == "cuda":
        index = dev.index
        if index is None:
            index = torch.cuda.current_device() if torch.cuda.is_available() else 0
        return f"cuda:{index}"
    return str(dev)


def make_mask_key(D, H, W, window_size, shift_size, dtype, device) -> MaskKey:
    return (int(D), int(H), int(W), tuple(window_size), tuple(shift_size), dtype, _device_key(device))


def clear_mask_cache() -> None:
    global _bytes
    _entries.clear()
    _bytes = 0


def mask_cache_info() -> dict[str, int]:
    return {
        "entries": len(_entries),
        "bytes": _bytes,
        "max_entries": _env_int("CRUMPET_MASK_CACHE_SIZE", _DEFAULT_MAX_ENTRIES),
        "max_bytes": _env_int("CRUMPET_MASK_CACHE_MAX_BYTES", _DEFAULT_MAX_BYTES),
    }


def get_or_compute_mask(key: MaskKey, compute: Callable[[], torch.Tensor]) -> torch.Tensor:
    """Return the cached mask for ``key`` or compute, store and return it."""
    global _bytes
    if _disabled():
        return compute()
    hit = _entries.get(key)
    if hit is not None:
        _entries.move_to_end(key)
        return hit
    value = compute()
    size = value.numel() * value.element_size()
    max_bytes = _env_int("CRUMPET_MASK_CACHE_MAX_BYTES", _DEFAULT_MAX_BYTES)
    max_entries = _env_int("CRUMPET_MASK_CACHE_SIZE", _DEFAULT_MAX_ENTRIES)
    if size > max_bytes or max_entries <= 0:
        return value
    _entries[key] = value
    _bytes += size
    while len(_entries) > max_entries or _bytes > max_bytes:
        _, old = _entries.popitem(last=False)
        _bytes -= old.numel() * old.element_size()
    return value
