"""The raw dispatcher ops under torch.compile and torch.library.opcheck.

Mirrors tests/test_compile.py:9-22 of the reference (a fullgraph-compiled
partition -> unpartition round trip must return its input) and checks each
crumpet_ops schema with opcheck: schema and mutation annotations, the fake
(meta) kernels registered in crumpet_amd/_native.py, and AOT dispatch.
The compile test uses the aot_eager backend: it traces through Dynamo, fake
tensors and AOTAutograd exactly as inductor would, without generating any
kernels of its own, so the ops run as the HIP kernels they are.
"""

from __future__ import annotations

import pytest
import torch

import crumpet_amd
from helpers import seeded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


class _RoundTrip(torch.nn.Module):
    def forward(self, x):
        w = crumpet_amd.fused_shift_partition_3d(x, (2, 2, 2), (1, 1, 1))
        return crumpet_amd.fused_unshift_unpartition_3d(w, x.shape[0], 4, 4, 4, x.shape[-1], (2, 2, 2),
                                                        (1, 1, 1))


def test_torch_compile_fullgraph_round_trip(dev):
    x = seeded((1, 4, 4, 4, 3), torch.float32, 1).to(dev)
    compiled = torch.compile(_RoundTrip(), fullgraph=True, backend="aot_eager")
    assert torch.equal(compiled(x), x)
    # a second shape recompiles and stays exact
    x2 = seeded((2, 4, 4, 4, 5), torch.float16, 2).to(dev)
    assert torch.equal(compiled(x2), x2)


def test_torch_compile_matches_eager_windows(dev):
    class Part(torch.nn.Module):
        def forward(self, x):
            return crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3))

    x = seeded((2, 14, 14, 14, 8), torch.bfloat16, 3).to(dev)
    compiled = torch.compile(Part(), fullgraph=True, backend="aot_eager")
    assert torch.equal(compiled(x), crumpet_amd.fused_shift_partition_3d(x, (7, 7, 7), (3, 3, 3)))


def _opcheck(op, args):
    torch.library.opcheck(op, args, test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))


def test_opcheck_reference_ops(dev):
    ops = torch.ops.crumpet_ops
    B, D, H, W, C = 2, 8, 8, 8, 6
    ws, ss = (4, 4, 4), (1, 2, 3)
    x = seeded((B, D, H, W, C), torch.float16, 4).to(dev)
    wins = torch.empty((B * 8, 64, C), dtype=torch.float16, device=dev)
    back = torch.empty_like(x)
    mask = torch.empty((8, 64, 64), dtype=torch.float32, device=dev)
    _opcheck(ops.fused_shift_partition_3d.default, (wins, x, *ws, *ss))
    _opcheck(ops.fused_unshift_unpartition_3d.default, (back, wins, B, D, H, W, C, *ws, *ss))
    _opcheck(ops.fused_shift_partition_3d_backward.default, (back, wins, B, D, H, W, C, *ws, *ss))
    _opcheck(ops.fused_unshift_unpartition_3d_backward.default, (wins, x, *ws, *ss))
    _opcheck(ops.compute_attn_mask_3d.default, (mask, D, H, W, *ws, *ss))
    # the last calls left real results behind: the round trip is exact
    ops.fused_shift_partition_3d(wins, x, *ws, *ss)
    ops.fused_unshift_unpartition_3d(back, wins, B, D, H, W, C, *ws, *ss)
    assert torch.equal(back, x)


def test_opcheck_attention_and_block_ops(dev):
    ops = torch.ops.crumpet_ops
    B, H, N = 8, 2, 27
    qkv = seeded((B, N, 3, H, 16), torch.float16, 5).to(dev)
    q, k, v = (qkv[:, :, j].permute(0, 2, 1, 3) for j in range(3))
    bias = (seeded((H, N, N), torch.float32, 6) * 0.1).to(dev)
    mask = torch.where(seeded((2, N, N), torch.float32, 7) > 0.5, -100.0, 0.0).to(dev)
    bnd = torch.tensor([1, 0] * 4, dtype=torch.uint8, device=dev)
    out = torch.empty((B, H, N, 16), dtype=torch.float16, device=dev)
    _opcheck(ops.fused_swin_attention.default, (out, q, k, v, bias, mask, bnd, 0.25))
    _opcheck(ops.fused_swin_attention.default, (out, q, k, v, bias, None, None, 0.25))
    _opcheck(ops.fused_swin_attention_shifted.default, (out, q, k, v, bias, 6, 6, 6, 3, 3, 3, 1, 1, 1, 0.25))
    hmask = mask.half()
    tiles = torch.empty(2 * 2 * 2 * 256, dtype=torch.float16, device=dev)  # M=2, N=27: 2 strips x 2 tiles
    _opcheck(ops.attn_mask_tiles.default, (tiles, hmask))
    _opcheck(ops.fused_swin_attention_tiled.default, (out, q, k, v, bias, hmask, tiles, bnd, 0.25))

    x = seeded((1, 6, 6, 6, 16), torch.float16, 8).to(dev)
    w = (seeded((48, 16), torch.float32, 9) / 4).half().to(dev)
    b = seeded((48,), torch.float32, 10).half().to(dev)
    nw = torch.ones(16, device=dev)
    nb = torch.zeros(16, device=dev)
    qo = torch.empty((8, 27, 48), dtype=torch.float16, device=dev)
    _opcheck(ops.window_qkv_3d.default, (qo, x, nw, nb, 1e-5, True, w, b, 3, 3, 3, 1, 1, 1))
    wp = (seeded((16, 16), torch.float32, 11) / 4).half().to(dev)
    y = torch.empty((1, 6, 6, 6, 16), dtype=torch.float16, device=dev)
    _opcheck(ops.window_proj_3d.default, (y, qo[:, :, :16].contiguous(), wp, None, 3, 3, 3, 1, 1, 1))
    rb = (seeded((1, 27, 27), torch.float32, 12) * 0.1).to(dev)
    _opcheck(ops.window_msa_3d.default, (x, nw, nb, 1e-5, w, b, wp, None, rb, 1, 0.25, 3, 3, 3, 1, 1, 1))
