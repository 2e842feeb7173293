"""CPU oracle of the crumpet shifted-window hot path.

TEST INFRASTRUCTURE ONLY.  Only tests/, bench.py's ``cpu_baseline`` leg and
``__graft_entry__.smoke()`` may import this module, and only as the checker
(or the timed CPU baseline), never as the thing measured or shipped.  The
product package ``crumpet_amd`` never imports it and has no CPU fallback.

Two independent restatements of each integer/byte function live here so
that tests can pin one against the other:

* the scalar C closed forms in ``crumpet_oracle.c`` (fast, used at full
  BASELINE sizes), reached through ctypes; and
* numpy restatements of the textbook tensor ops the reference composes
  (``np.roll`` + reshape/transpose, vectorised region ``where``, MONAI slice
  assignment), following the cited reference lines.

The attention oracle is the plain formula
``softmax(q*scale @ k^T + bias + [boundary]*mask) @ v`` in float32 (or
float64), following the semantics of
torch-ext/crumpet/fused_attention.py:82-146 and the wrapper :149-226.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path
from typing import Sequence

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_LIB = None

NEG100_BITS = {"float16": 0xD640, "bfloat16": 0xC2C8, "float32": 0xC2C80000}


def build_oracle(force: bool = False) -> Path:
    """Compile crumpet_oracle.c with gcc into oracle/liboracle.so."""
    src = ORACLE_DIR / "crumpet_oracle.c"
    if force or not LIB_PATH.exists() or LIB_PATH.stat().st_mtime < src.stat().st_mtime:
        tmp = LIB_PATH.with_suffix(".so.tmp")
        subprocess.check_call(
            ["gcc", "-O2", "-std=c99", "-fPIC", "-shared", str(src), "-o", str(tmp)]
        )
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build_oracle()
        lib = ctypes.CDLL(str(LIB_PATH))
        i64 = ctypes.c_int64
        arr3 = ctypes.POINTER(ctypes.c_int64)
        for name in ("oracle_shift_partition_3d", "oracle_unshift_unpartition_3d"):
            fn = getattr(lib, name)
            fn.restype = None
            fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, i64, i64, i64, i64, i64, i64, arr3, arr3]
        lib.oracle_attn_mask_3d.restype = None
        lib.oracle_attn_mask_3d.argtypes = [
            ctypes.c_void_p, i64, ctypes.c_uint32, i64, i64, i64, arr3, arr3,
        ]
        _LIB = lib
    return _LIB


def _triple(v: Sequence[int]) -> tuple[int, int, int]:
    t = tuple(int(x) for x in v)
    if len(t) != 3:
        raise ValueError("expected three values")
    return t


def _arr3(v):
    return (ctypes.c_int64 * 3)(*_triple(v))


def _check(D, H, W, ws, ss):
    for dim, w, s in zip((D, H, W), ws, ss):
        if w <= 0 or dim % w:
            raise ValueError("D, H and W must be divisible by window_size")
        if s < 0 or s >= w:
            raise ValueError("shift_size must satisfy 0 <= shift < window_size")


# --------------------------------------------------------------------------
# C closed forms (byte-exact, any element type)
# --------------------------------------------------------------------------

def shift_partition(x: np.ndarray, ws, ss) -> np.ndarray:
    """[B,D,H,W,C] -> [B*nW, vol, C]; reference.py:141-160."""
    ws, ss = _triple(ws), _triple(ss)
    B, D, H, W, C = x.shape
    _check(D, H, W, ws, ss)
    x = np.ascontiguousarray(x)
    nW = (D // ws[0]) * (H // ws[1]) * (W // ws[2])
    vol = ws[0] * ws[1] * ws[2]
    out = np.empty((B * nW, vol, C), dtype=x.dtype)
    _lib().oracle_shift_partition_3d(
        out.ctypes.data, x.ctypes.data, B, D, H, W, C, x.itemsize, _arr3(ws), _arr3(ss)
    )
    return out


def unshift_unpartition(windows: np.ndarray, B, D, H, W, C, ws, ss) -> np.ndarray:
    """[B*nW, vol, C] -> [B,D,H,W,C]; reference.py:163-184."""
    ws, ss = _triple(ws), _triple(ss)
    _check(D, H, W, ws, ss)
    windows = np.ascontiguousarray(windows)
    nW = (D // ws[0]) * (H // ws[1]) * (W // ws[2])
    if windows.shape != (B * nW, ws[0] * ws[1] * ws[2], C):
        raise ValueError("windows has the wrong shape")
    out = np.empty((B, D, H, W, C), dtype=windows.dtype)
    _lib().oracle_unshift_unpartition_3d(
        out.ctypes.data, windows.ctypes.data, B, D, H, W, C, windows.itemsize, _arr3(ws), _arr3(ss)
    )
    return out


def attn_mask_bits(D, H, W, ws, ss, dtype: str = "float16") -> np.ndarray:
    """Mask [nW, vol, vol] as raw element bits (uint16 or uint32).

    reference.py:50-98 and cuda/attn_mask_3d.cu:42-123.  ``dtype`` is one of
    "float16", "bfloat16", "float32"; -100 is exact in all three.
    """
    ws, ss = _triple(ws), _triple(ss)
    _check(D, H, W, ws, ss)
    vol = ws[0] * ws[1] * ws[2]
    if vol > 4096:
        raise ValueError("oracle supports window volumes up to 4096")
    nW = (D // ws[0]) * (H // ws[1]) * (W // ws[2])
    esize = 4 if dtype == "float32" else 2
    out = np.empty((nW, vol, vol), dtype=np.uint32 if esize == 4 else np.uint16)
    _lib().oracle_attn_mask_3d(
        out.ctypes.data, esize, NEG100_BITS[dtype], D, H, W, _arr3(ws), _arr3(ss)
    )
    return out


def attn_mask(D, H, W, ws, ss, dtype: str = "float32") -> np.ndarray:
    """Mask as float16/float32 values (bfloat16 has no numpy type; use attn_mask_bits)."""
    bits = attn_mask_bits(D, H, W, ws, ss, dtype)
    return bits.view(np.float16 if dtype == "float16" else np.float32)


# --------------------------------------------------------------------------
# numpy restatements of the reference's tensor-op compositions
# --------------------------------------------------------------------------

def np_window_partition(x: np.ndarray, ws) -> np.ndarray:
    """reference.py:101-118: view(B,D/ws,ws,H/ws,ws,W/ws,ws,C).permute(0,1,3,5,2,4,6,7)."""
    ws = _triple(ws)
    B, D, H, W, C = x.shape
    y = x.reshape(B, D // ws[0], ws[0], H // ws[1], ws[1], W // ws[2], ws[2], C)
    return np.ascontiguousarray(y.transpose(0, 1, 3, 5, 2, 4, 6, 7)).reshape(
        -1, ws[0] * ws[1] * ws[2], C
    )


def np_window_reverse(windows: np.ndarray, ws, dims) -> np.ndarray:
    """reference.py:121-138: view(B,D/ws,H/ws,W/ws,ws,ws,ws,C).permute(0,1,4,2,5,3,6,7)."""
    ws = _triple(ws)
    B, D, H, W = (int(v) for v in dims[:4])
    y = windows.reshape(B, D // ws[0], H // ws[1], W // ws[2], ws[0], ws[1], ws[2], -1)
    return np.ascontiguousarray(y.transpose(0, 1, 4, 2, 5, 3, 6, 7)).reshape(B, D, H, W, -1)


def np_shift_partition(x: np.ndarray, ws, ss) -> np.ndarray:
    """reference.py:141-160: torch.roll(x, -ss, dims=(1,2,3)) then partition."""
    ss = _triple(ss)
    if any(ss):
        x = np.roll(x, shift=(-ss[0], -ss[1], -ss[2]), axis=(1, 2, 3))
    return np_window_partition(x, ws)


def np_unshift_unpartition(windows: np.ndarray, B, D, H, W, C, ws, ss) -> np.ndarray:
    """reference.py:163-184: window reverse then torch.roll(x, +ss, dims=(1,2,3))."""
    ss = _triple(ss)
    x = np_window_reverse(windows, ws, (B, D, H, W))
    if any(ss):
        x = np.roll(x, shift=ss, axis=(1, 2, 3))
    return x


def np_mask_where(D, H, W, ws, ss) -> np.ndarray:
    """reference.py:50-98: torch.where region labels -> partition -> pairwise != -> where.

    Returns the boolean "labels differ" array [nW, vol, vol].
    """
    ws, ss = _triple(ws), _triple(ss)
    if not any(ss):
        nW = (D // ws[0]) * (H // ws[1]) * (W // ws[2])
        vol = ws[0] * ws[1] * ws[2]
        return np.zeros((nW, vol, vol), dtype=bool)

    def regions(n, w, s):
        a = np.arange(n)
        return np.where(a < n - w, 0, np.where(a < n - s, 1, 2))

    labels = (
        9 * regions(D, ws[0], ss[0])[:, None, None]
        + 3 * regions(H, ws[1], ss[1])[None, :, None]
        + regions(W, ws[2], ss[2])[None, None, :]
    ).astype(np.int16)
    win = np_window_partition(labels.reshape(1, D, H, W, 1), ws)[..., 0]
    return win[:, None, :] != win[:, :, None]


def np_mask_monai_slices(D, H, W, ws, ss) -> np.ndarray:
    """benchmarks/bench_kernel.py:63-86 (MONAI compute_mask): fp32 img_mask filled
    with cnt 0..26 over slice(-ws), slice(-ws,-ss), slice(-ss,None) per axis,
    partitioned, pairwise difference, nonzero -> -100.  Returns float32 values.
    """
    ws, ss = _triple(ws), _triple(ss)
    img = np.zeros((1, D, H, W, 1), dtype=np.float32)
    cnt = 0
    for d in (slice(-ws[0]), slice(-ws[0], -ss[0]), slice(-ss[0], None)):
        for h in (slice(-ws[1]), slice(-ws[1], -ss[1]), slice(-ss[1], None)):
            for w in (slice(-ws[2]), slice(-ws[2], -ss[2]), slice(-ss[2], None)):
                img[:, d, h, w, :] = cnt
                cnt += 1
    win = np_window_partition(img, ws)[..., 0]
    diff = win[:, None, :] - win[:, :, None]
    return np.where(diff != 0, np.float32(-100.0), np.float32(0.0)).astype(np.float32)


# --------------------------------------------------------------------------
# Swin / MONAI helpers used by the attention path
# --------------------------------------------------------------------------

def get_window_size(x_size, window_size, shift_size=None):
    """MONAI get_window_size rule (called at monai_patch.py:81,210): an axis whose
    extent is <= the window uses the extent as window and no shift."""
    use_w = list(window_size)
    use_s = list(shift_size) if shift_size is not None else None
    for i in range(len(x_size)):
        if x_size[i] <= window_size[i]:
            use_w[i] = x_size[i]
            if use_s is not None:
                use_s[i] = 0
    if use_s is None:
        return tuple(use_w)
    return tuple(use_w), tuple(use_s)


def relative_position_index(ws) -> np.ndarray:
    """Closed form of the 3D relative position index [vol, vol]:
    ((dd + ws_d-1)*(2ws_h-1) + (dh + ws_h-1))*(2ws_w-1) + (dw + ws_w-1),
    with d* = coord_i - coord_j (Swin, Liu et al. 2021; MONAI WindowAttention)."""
    ws = _triple(ws)
    coords = np.stack(
        np.meshgrid(np.arange(ws[0]), np.arange(ws[1]), np.arange(ws[2]), indexing="ij")
    ).reshape(3, -1)
    vol = coords.shape[1]
    idx = np.empty((vol, vol), dtype=np.int64)
    for i in range(vol):
        dd = coords[:, i][:, None] - coords
        idx[i] = ((dd[0] + ws[0] - 1) * (2 * ws[1] - 1) + (dd[1] + ws[1] - 1)) * (2 * ws[2] - 1) + (
            dd[2] + ws[2] - 1
        )
    return idx


def relative_position_index_swin(ws) -> np.ndarray:
    """The textbook Swin/MONAI construction: relative coords, shift to start at
    0, multiply by the mixed-radix strides, sum."""
    ws = _triple(ws)
    coords = np.stack(np.meshgrid(*[np.arange(w) for w in ws], indexing="ij"))
    flat = coords.reshape(3, -1)
    rel = (flat[:, :, None] - flat[:, None, :]).transpose(1, 2, 0).copy()
    rel[:, :, 0] += ws[0] - 1
    rel[:, :, 1] += ws[1] - 1
    rel[:, :, 2] += ws[2] - 1
    rel[:, :, 0] *= (2 * ws[1] - 1) * (2 * ws[2] - 1)
    rel[:, :, 1] *= 2 * ws[2] - 1
    return rel.sum(-1)


def gather_bias(table: np.ndarray, ws, n: int | None = None) -> np.ndarray:
    """table [(2ws-1)^3, H] -> bias [H, n, n], as monai_patch.py:160-162."""
    rpi = relative_position_index(ws)
    if n is not None:
        rpi = rpi[:n, :n]
    n_ = rpi.shape[0]
    return np.ascontiguousarray(table[rpi.reshape(-1)].reshape(n_, n_, -1).transpose(2, 0, 1))


def attention(q, k, v, bias, mask=None, boundary=None, scale=None, dtype=np.float32,
              window_chunk: int = 256) -> np.ndarray:
    """out[b,h] = softmax(q[b,h]*scale @ k[b,h]^T + bias[h] + [bnd_b]*mask[b % M]) @ v[b,h].

    q, k, v: [B, H, N, D]; bias [H, N, N]; mask [M, N, N] with M | B, or None;
    boundary [B] (nonzero = add the mask) or None (= all windows read the
    mask).  Computed in ``dtype`` (float32 by default) in window chunks.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    bias = np.asarray(bias, dtype=dtype)
    B, Hh, N, Dh = q.shape
    if scale is None:
        scale = Dh ** -0.5
    scale = dtype(scale)
    out = np.empty((B, Hh, N, Dh), dtype=dtype)
    if mask is not None:
        mask = np.asarray(mask, dtype=dtype)
        M = mask.shape[0]
        if B % M:
            raise ValueError("mask batch must divide B")
    for b0 in range(0, B, window_chunk):
        b1 = min(B, b0 + window_chunk)
        s = np.matmul(q[b0:b1] * scale, np.swapaxes(k[b0:b1], -1, -2)) + bias[None]
        if mask is not None:
            idx = np.arange(b0, b1) % mask.shape[0]
            m = mask[idx][:, None]
            if boundary is not None:
                flag = (np.asarray(boundary[b0:b1]) != 0)[:, None, None, None]
                m = np.where(flag, m, dtype(0))
            s = s + m
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[b0:b1] = np.matmul(p, v[b0:b1])
    return out


def attention_reference_numerics(q, k, v, bias, mask=None, scale=None, block_n: int = 32):
    """The attention formula with the rounding steps of the reference's Triton
    kernel (torch-ext/crumpet/fused_attention.py:82-146), for 2-byte inputs:
    q * scale computed in fp32 and rounded to the input dtype (:88); scores
    and bias + mask in fp32 (:109-128); an online softmax over ``block_n``-key
    chunks (:133-140) whose P is rounded to the input dtype before P V, with
    the row sum taken over the unrounded fp32 P and the accumulator rescaled
    in fp32; the result rounded to the input dtype (:142-148).

    q, k, v: torch tensors [B, H, N, D] (float16 / bfloat16 / float32, CPU);
    bias [H, N, N]; mask [B, N, N] (already tiled per window) or None.
    Returns a torch tensor of q's dtype.  Used to bound what the input
    dtype's rounding alone costs against the exact formula (``attention``).
    """
    import torch

    dt = q.dtype
    B, H, N, D = q.shape
    if scale is None:
        scale = D ** -0.5
    qs = (q.float() * scale).to(dt).float()
    m = torch.full((B, H, N), -float("inf"))
    l = torch.zeros((B, H, N))
    acc = torch.zeros((B, H, N, D))
    for n0 in range(0, N, block_n):
        n1 = min(N, n0 + block_n)
        s = qs @ k[:, :, n0:n1].float().transpose(-1, -2) + bias[None, :, :, n0:n1].float()
        if mask is not None:
            s = s + mask[:, None, :, n0:n1].float()
        m_new = torch.maximum(m, s.amax(-1))
        alpha = torch.exp(m - m_new)
        p = torch.exp(s - m_new[..., None])
        l = l * alpha + p.sum(-1)
        acc = acc * alpha[..., None] + p.to(dt).float() @ v[:, :, n0:n1].float()
        m = m_new
    return (acc / l[..., None]).to(dt)


# --------------------------------------------------------------------------
# fused window-MSA block projections (the chain around the attention)
# --------------------------------------------------------------------------

def round_to(a, dtype: str) -> np.ndarray:
    """Round to float16 / bfloat16 / float32 (nearest even) and return float64.

    The 16-bit types are reached through float32, as in the kernels and the
    autocast chain, whose values are float32 before the cast.  bfloat16 (no
    numpy type) keeps the upper 16 bits of the float32 value after adding
    0x7FFF plus the lowest kept bit (round half to even).
    """
    a = np.asarray(a, dtype=np.float64)
    if dtype == "float64":
        return a
    if dtype == "float32":
        return a.astype(np.float32).astype(np.float64)
    if dtype == "float16":
        return a.astype(np.float32).astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
        u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
        return u.astype(np.uint32).view(np.float32).astype(np.float64)
    raise ValueError(dtype)


def _padded_dims(D, H, W, ws):
    ws = _triple(ws)
    return tuple(-(-d // w) * w for d, w in zip((D, H, W), ws))


def layer_norm(x, weight=None, bias=None, eps: float = 1e-5) -> np.ndarray:
    """torch.nn.LayerNorm over the last axis in float64: biased variance, eps
    inside the square root, optional affine weight / bias."""
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = np.square(x - mean).mean(axis=-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, dtype=np.float64)
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def window_qkv(x, ws, ss, weight, bias=None, norm_weight=None, norm_bias=None, eps: float = 1e-5,
               normalize: bool = True, dtype: str = "float16") -> np.ndarray:
    """[B*nW, N, n_out]: the eager chain of monai_patch.py:79-97 plus the qkv
    Linear of :153 -- norm1, zero padding at the end of each axis to the
    window grid (after the norm), roll by -ss, window partition, Linear.

    float64 arithmetic, with the two roundings of the autocast chain: the
    LayerNorm output (the Linear's input) and the Linear's output are rounded
    to ``dtype``.  ``weight`` / ``bias`` are taken as given (pass values
    already rounded to ``dtype``).
    """
    x = np.asarray(x, dtype=np.float64)
    B, D, H, W, C = x.shape
    a = layer_norm(x, norm_weight, norm_bias, eps) if normalize else x
    a = round_to(a, dtype)
    Dp, Hp, Wp = _padded_dims(D, H, W, ws)
    ap = np.zeros((B, Dp, Hp, Wp, C), dtype=np.float64)
    ap[:, :D, :H, :W] = a
    win = np_shift_partition(ap, ws, ss)
    y = win @ np.asarray(weight, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return round_to(y, dtype)


def window_proj(windows, B, D, H, W, ws, ss, weight, bias=None, dtype: str = "float16") -> np.ndarray:
    """[B, D, H, W, n_out]: the proj Linear of monai_patch.py:196-197, then the
    window reverse on the padded grid, roll by +ss and the crop of :98-111.
    float64 arithmetic, output rounded to ``dtype``."""
    y = np.asarray(windows, dtype=np.float64) @ np.asarray(weight, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    y = round_to(y, dtype)
    Dp, Hp, Wp = _padded_dims(D, H, W, ws)
    vol = np_unshift_unpartition(y, B, Dp, Hp, Wp, y.shape[-1], ws, ss)
    return np.ascontiguousarray(vol[:, :D, :H, :W])
