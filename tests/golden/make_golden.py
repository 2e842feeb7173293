"""Write the small golden fixtures of tests/golden/ from the pinned oracle.

The reference ships no golden vectors for this path (its tests re-derive
everything from the eager PyTorch restatement), so these fixtures freeze the
oracle's outputs - each already pinned against independent constructions in
tests/test_oracle.py - on small seeded inputs:

* partition_f16.npz   : x [2,14,7,21,5] fp16 bits, ws (7,7,7), ss (3,2,4)
                        -> windows bits (and the identity round trip)
* mask_bits.npz       : masks (raw bits) for fp16 / bf16 / fp32 at
                        (14,14,14) ws7 ss3, (12,8,6) ws(6,4,3) ss(3,2,1), zero shift
* attention_f16.npz   : q, k, v [6,2,27,16] fp16, bias [2,27,27] fp16,
                        mask [3,27,27] fp16 (b mod 3), boundary [6]
                        -> fp64 oracle output

Run from the repository root: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import oracle  # noqa: E402


def f16_bits(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16).view(np.uint16)


def main() -> None:
    rng = np.random.default_rng(20261201)

    x = rng.standard_normal((2, 14, 7, 21, 5)).astype(np.float16)
    ws, ss = (7, 7, 7), (3, 2, 4)
    win = oracle.shift_partition(x.view(np.uint16), ws, ss)
    np.savez_compressed(HERE / "partition_f16.npz", x=x.view(np.uint16), windows=win,
                        ws=np.array(ws), ss=np.array(ss))

    cases = [((14, 14, 14), (7, 7, 7), (3, 3, 3)), ((12, 8, 6), (6, 4, 3), (3, 2, 1)),
             ((14, 14, 14), (7, 7, 7), (0, 0, 0))]
    out = {}
    for i, (dims, w, s) in enumerate(cases):
        out[f"dims{i}"] = np.array(dims)
        out[f"ws{i}"] = np.array(w)
        out[f"ss{i}"] = np.array(s)
        for dt in ("float16", "bfloat16", "float32"):
            out[f"mask{i}_{dt}"] = oracle.attn_mask_bits(*dims, w, s, dt)
    np.savez_compressed(HERE / "mask_bits.npz", **out)

    B, H, N, D = 6, 2, 27, 16
    q, k, v = (rng.standard_normal((B, H, N, D)).astype(np.float16) for _ in range(3))
    bias = (0.02 * rng.standard_normal((H, N, N))).astype(np.float16)
    mask = oracle.attn_mask(6, 3, 3, (3, 3, 3), (1, 1, 1), "float16").astype(np.float16)  # [2,27,27]
    mask = np.concatenate([mask, np.zeros((1, N, N), np.float16)])  # [3,27,27]
    boundary = np.array([1, 1, 0, 1, 0, 1], dtype=np.uint8)
    ref = oracle.attention(q, k, v, bias, mask, boundary, scale=0.25, dtype=np.float64)
    np.savez_compressed(HERE / "attention_f16.npz", q=q.view(np.uint16), k=k.view(np.uint16),
                        v=v.view(np.uint16), bias=bias.view(np.uint16), mask=mask.view(np.uint16),
                        boundary=boundary, scale=np.array(0.25), out=ref)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
