"""Config 4: the full shifted-window block path at the deeper Swin UNETR
stages (B=4, fp16 and bf16): shift-partition -> fused attention (mask from
the geometry) -> unshift-unpartition, each stage checked against the oracle.

* partition and unpartition: bit-exact against the C oracle on the whole
  volume (the unpartition check runs on the kernel's own attention output,
  so it isolates the gather);
* attention: every window of the stage against the fp32 oracle formula with
  the dense shifted mask, within 2e-3 (fp16) / 1e-2 (bf16).  q is the
  partitioned tokens read as H heads of 16; k and v are the same tokens
  with the heads rotated by one and two (independent of q,
  as a qkv projection makes them; with k = q every row's softmax peaks on
  its own key and the input-dtype rounding of P alone approaches the bf16
  tolerance).
Stage 3 runs both as BASELINE states it ([4,7^3,384], window 7, shift 0) and
as MONAI executes it ([4,6^3,384]: window 6, N=216, no shift).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import crumpet_amd
from crumpet_amd.fused_attention import fused_swin_attention_shifted
from helpers import TOL, bias_from_table, raw, seeded, trunc_normal_table

pytestmark = pytest.mark.gpu

STAGES = [("s1", 28, 96, 6, (7, 7, 7), (3, 3, 3)),
          ("s2", 14, 192, 12, (7, 7, 7), (3, 3, 3)),
          ("s3", 7, 384, 24, (7, 7, 7), (0, 0, 0)),
          ("s3_monai", 6, 384, 24, (6, 6, 6), (0, 0, 0))]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("stage", STAGES, ids=[s[0] for s in STAGES])
def test_stage_block_path(oracle, dev, stage, dtype):
    name, dim, C, H, ws, ss = stage
    B = 4
    N = ws[0] * ws[1] * ws[2]
    print(f"block path {name} {dtype}", flush=True)
    x = seeded((B, dim, dim, dim, C), dtype, 600 + dim)
    xd = x.to(dev)
    w = crumpet_amd.fused_shift_partition_3d(xd, ws, ss)
    np.testing.assert_array_equal(raw(w), oracle.shift_partition(raw(x), ws, ss))

    table = trunc_normal_table((2 * ws[0] - 1) * (2 * ws[1] - 1) * (2 * ws[2] - 1), H, 610 + dim)
    bias = bias_from_table(table, ws).to(dtype)
    nwin = w.shape[0]
    t = w.view(nwin, N, H, 16).permute(0, 2, 1, 3)
    tk = torch.roll(t, 1, dims=1)
    tv = torch.roll(t, 2, dims=1)
    o = torch.empty_like(w)
    ov = o.view(nwin, N, H, 16).permute(0, 2, 1, 3)
    fused_swin_attention_shifted(t, tk, tv, bias.to(dev), (dim,) * 3, ws, ss, 0.25, ov)

    back = crumpet_amd.fused_unshift_unpartition_3d(o, B, dim, dim, dim, C, ws, ss)
    np.testing.assert_array_equal(raw(back), oracle.unshift_unpartition(raw(o), B, dim, dim, dim, C, ws, ss))

    # every window: the mask tensor tiles the nW per-volume masks over the batch
    tq, tkn, tvn = (a.float().cpu().numpy() for a in (t, tk, tv))
    mask = oracle.attn_mask(dim, dim, dim, ws, ss, "float32")
    want = oracle.attention(tq, tkn, tvn, bias.float().numpy(), mask, None, scale=0.25, window_chunk=32)
    got = ov.float().cpu().numpy()
    err = float(np.abs(got - want).max())
    print(f"  {name} {dtype}: attention max-abs {err:.2e} over all {nwin} windows", flush=True)
    assert err < TOL[dtype]
