"""The hot path under HIP graph capture.

The kernels neither allocate nor synchronise, so a caller can capture the
shifted-window path (partition -> shifted attention -> unpartition, and the
fused block projections) in a graph and replay it.  Each replay is checked
bit-exactly against the eager result of the same inputs, with eager work and
synchronisations between the replays; the inputs change between replays so
that a replay that reran stale work would be caught.
"""

from __future__ import annotations

import pytest
import torch

from crumpet_amd.fused_attention import fused_swin_attention_shifted
from helpers import seeded

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    return torch.device("cuda:0")


def _path(ops, x, wins, attn, back, bias, dims, ws, ss, H):
    B, D, Hh, W, C = x.shape
    ops.fused_shift_partition_3d(wins, x, *ws, *ss)
    nwin, n = wins.shape[0], wins.shape[1]
    t = wins.view(nwin, n, H, 16).permute(0, 2, 1, 3)
    fused_swin_attention_shifted(t, t, t, bias, dims, ws, ss, 0.25, attn.view(nwin, n, H, 16).permute(0, 2, 1, 3))
    ops.fused_unshift_unpartition_3d(back, attn, B, D, Hh, W, C, *ws, *ss)


def test_graph_replays_match_eager(dev):
    ops = torch.ops.crumpet_ops
    B, D, H, C = 2, 14, 3, 48
    ws, ss, dims = (7, 7, 7), (3, 3, 3), (D, D, D)
    x = seeded((B, D, D, D, C), torch.float16, 1).to(dev)
    bias = (seeded((H, 343, 343), torch.float32, 2) * 0.1).half().to(dev)
    wins = torch.empty((B * 8, 343, C), dtype=torch.float16, device=dev)
    attn = torch.empty_like(wins)
    back = torch.empty_like(x)

    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm-up on the capture stream
        _path(ops, x, wins, attn, back, bias, dims, ws, ss, H)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        _path(ops, x, wins, attn, back, bias, dims, ws, ss, H)
    torch.cuda.synchronize()

    e_wins, e_attn, e_back = torch.empty_like(wins), torch.empty_like(attn), torch.empty_like(back)
    for seed in (11, 12, 13):
        x.copy_(seeded((B, D, D, D, C), torch.float16, seed).to(dev))
        g.replay()
        torch.cuda.synchronize()
        _path(ops, x, e_wins, e_attn, e_back, bias, dims, ws, ss, H)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(wins, e_wins), seed
        assert torch.equal(attn, e_attn), seed
        assert torch.equal(back, e_back), seed


def test_graph_replays_fused_block_projections(dev):
    C = 48
    x = seeded((2, 12, 12, 12, C), torch.float32, 20).to(dev)
    w = (seeded((3 * C, C), torch.float32, 21) / C ** 0.5).half().to(dev)
    b = (seeded((3 * C,), torch.float32, 22) * 0.1).half().to(dev)
    wp = (seeded((C, C), torch.float32, 23) / C ** 0.5).half().to(dev)
    gw = torch.ones(C, device=dev)
    gb = torch.zeros(C, device=dev)
    ops = torch.ops.crumpet_ops
    qkv = torch.empty((2 * 8, 343, 3 * C), dtype=torch.float16, device=dev)
    y = torch.empty((2, 12, 12, 12, C), dtype=torch.float16, device=dev)

    def run(qkv_out, y_out):
        ops.window_qkv_3d(qkv_out, x, gw, gb, 1e-5, True, w, b, 7, 7, 7, 3, 3, 3)
        ops.window_proj_3d(y_out, qkv_out[:, :, :C].contiguous(), wp, None, 7, 7, 7, 3, 3, 3)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run(qkv, y)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        run(qkv, y)
    torch.cuda.synchronize()
    e_qkv, e_y = torch.empty_like(qkv), torch.empty_like(y)
    for seed in (30, 31, 32):
        x.copy_(seeded(tuple(x.shape), torch.float32, seed).to(dev))
        g.replay()
        torch.cuda.synchronize()
        run(e_qkv, e_y)
        torch.cuda.synchronize()
        assert torch.equal(qkv, e_qkv), seed
        assert torch.equal(y, e_y), seed


def test_graph_replays_window_msa_op(dev):
    """window_msa_3d allocates its intermediates and output inside the call:
    captured, they come from the graph's pool, and every replay matches an
    eager call on the same input."""
    C, H = 48, 3
    x = seeded((2, 12, 12, 12, C), torch.float32, 40).to(dev)
    w = (seeded((3 * C, C), torch.float32, 41) / C ** 0.5).half().to(dev)
    b = (seeded((3 * C,), torch.float32, 42) * 0.1).half().to(dev)
    wp = (seeded((C, C), torch.float32, 43) / C ** 0.5).half().to(dev)
    gw = torch.ones(C, device=dev)
    gb = torch.zeros(C, device=dev)
    bias = (seeded((H, 343, 343), torch.float32, 44) * 0.1).to(dev)
    ops = torch.ops.crumpet_ops

    def run():
        return ops.window_msa_3d(x, gw, gb, 1e-5, w, b, wp, None, bias, H, 0.25, 7, 7, 7, 3, 3, 3)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        y = run()
    torch.cuda.synchronize()
    for seed in (50, 51, 52):
        x.copy_(seeded(tuple(x.shape), torch.float32, seed).to(dev))
        g.replay()
        torch.cuda.synchronize()
        want = run()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(y, want), seed
