"""Window-grid arithmetic and argument checks shared by the public API.

The error types and the key words of the messages are part of the
interface: callers (and the reference's tests, tests/test_padding.py:11,17)
match ``ValueError`` with "divisible" and "shift_size", and a dtype outside
fp32/fp16/bf16 raises ``TypeError`` (torch-ext/crumpet/__init__.py:98-122
is the behaviour followed).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import torch

FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
DTYPE_MESSAGE = "CRUMPET supports torch.float32, torch.float16 and torch.bfloat16"


def as_triple(name: str, value: Sequence[int], *, signed: bool = False) -> tuple[int, int, int]:
    """Three ints from a sequence; negatives are rejected unless ``signed``."""
    if len(value) != 3:
        raise ValueError(f"{name} must contain exactly three values")
    d, h, w = (int(v) for v in value)
    if not signed and min(d, h, w) < 0:
        raise ValueError(f"{name} values must be non-negative")
    return d, h, w


def require_float_dtype(dtype: torch.dtype) -> None:
    if dtype not in FLOAT_DTYPES:
        raise TypeError(DTYPE_MESSAGE)


def padded_dims(dims: Sequence[int], window: Sequence[int]) -> tuple[int, int, int]:
    """Each extent rounded up to a whole number of windows."""
    return tuple(-(-int(d) // int(w)) * int(w) for d, w in zip(dims, window))


@dataclass(frozen=True)
class WindowGrid:
    """A ``D x H x W`` volume tiled by ``window`` with a cyclic ``shift``."""

    dims: tuple[int, int, int]
    window: tuple[int, int, int]
    shift: tuple[int, int, int]

    @classmethod
    def checked(cls, D: int, H: int, W: int, window_size: Sequence[int],
                shift_size: Sequence[int]) -> "WindowGrid":
        """Validate a standalone (unpadded) grid as the kernels require it."""
        window = as_triple("window_size", window_size)
        shift = as_triple("shift_size", shift_size)
        dims = (int(D), int(H), int(W))
        if min(dims) <= 0:
            raise ValueError("D, H and W must be positive")
        if min(window) <= 0:
            raise ValueError("window_size values must be positive")
        if any(d % w for d, w in zip(dims, window)):
            raise ValueError(
                "standalone CRUMPET kernels require D, H and W to be divisible by window_size"
            )
        for axis in range(3):
            if not 0 <= shift[axis] < window[axis]:
                raise ValueError(
                    f"shift_size[{axis}] must satisfy 0 <= shift < window_size[{axis}]"
                )
        return cls(dims, window, shift)

    @property
    def volume(self) -> int:
        """Tokens per window."""
        return self.window[0] * self.window[1] * self.window[2]

    @property
    def num_windows(self) -> int:
        """Windows per volume."""
        return ((self.dims[0] // self.window[0]) * (self.dims[1] // self.window[1])
                * (self.dims[2] // self.window[2]))

    def windows_shape(self, batch: int, channels: int) -> tuple[int, int, int]:
        return (batch * self.num_windows, self.volume, channels)

    def volume_shape(self, batch: int, channels: int) -> tuple[int, int, int, int, int]:
        return (batch, *self.dims, channels)

    @property
    def op_args(self) -> tuple[int, ...]:
        """``ws_d, ws_h, ws_w, ss_d, ss_h, ss_w`` as the ops take them."""
        return (*self.window, *self.shift)
