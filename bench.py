"""Benchmark of the MI355X shifted-window hot path (one GPU).

A step is one pass of the hot path over one batch: the shift-partition plus
unshift-unpartition round trip of BASELINE config 1 ([1, 98^3, 48] fp16,
window 7, shift 3), called through the public crumpet API with the input
resident in HBM.  ``value`` is the round trip's algorithmic bytes
(2 x 180,708,864 B) per step time, in GB/s.

The same run also measures, each on its own BASELINE config:
  * the partition and unpartition kernels alone (per-launch HIP events,
    rotating buffer sets so no launch reads what the 256 MB MALL still holds);
  * the mask kernel (config 2, 98^3 fp16, 645,657,712 B written);
  * fused window attention (config 3, 1372 windows x 3 heads, N=343, hd 16),
    in TFLOP/s, with the eager ROCm PyTorch chain timed beside it;
  * the CPU oracle on the host cores as the reported CPU baseline, and each
    config's eager path on the host cores beside its GPU figure.

Prints ONE JSON line.  Only one GPU is supported: --gpus above 1 exits.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def synthetic_ct(shape, seed):
    """Config-5 input volume; the generator is shared with the test suite."""
    sys.path.insert(0, str(ROOT / "tests"))
    try:
        from helpers import synthetic_ct as make
    finally:
        sys.path.remove(str(ROOT / "tests"))
    return make(shape, seed)


HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0

C1 = dict(B=1, D=98, H=98, W=98, C=48, ws=(7, 7, 7), ss=(3, 3, 3))
C1_BYTES = 2 * 1 * 98 * 98 * 98 * 48 * 2  # read + write per direction: 180,708,864
C2_BYTES = 2744 * 343 * 343 * 2  # 645,657,712
C3 = dict(B=1372, H=3, N=343, Dh=16, D=49)
C3_FLOPS = 4 * 343 * 343 * 16 * 3 * 1372  # 30,991,570,176
C3_BYTES = 1372 * 343 * 144 * 2 + 1372 * 343 * 48 * 2  # qkv in + out: 180,708,864


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-attention", action="store_true")
    p.add_argument("--no-eager", action="store_true", help="skip the eager GPU attention chain")
    p.add_argument("--no-blocks", action="store_true", help="skip the config-4 stage block paths")
    p.add_argument("--no-e2e", action="store_true", help="skip the config-5 Swin UNETR forward")
    p.add_argument("--no-fused-block", action="store_true",
                   help="skip the fused window-MSA block at the config-5 stage shapes")
    p.add_argument("--profile", action="store_true",
                   help="short fixed launch sequence for rocprofv3 (plus a copy of known size)")
    return p.parse_args()


def _events_time(fn, iters):
    """Average ms per call of fn over iters back-to-back calls, HIP events on
    the current stream.  Python's cyclic garbage collector is paused over the
    timed calls (as timeit does): a full collection in a process holding a
    model takes tens of milliseconds and would land in whichever call
    happened to trigger it."""
    import gc

    import torch

    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    enabled = gc.isenabled()
    gc.disable()
    try:
        s.record()
        for i in range(iters):
            fn(i)
        e.record()
        torch.cuda.synchronize()
    finally:
        if enabled:
            gc.enable()
    return s.elapsed_time(e) / iters


_BUSY = {}


def _settle_clock(dev, seconds=0.15):
    """Keep the GPU busy for `seconds` with long torch matmuls (no kernel of
    this package, few dispatches in a profiler's records).  The shader clock
    ramps up over the first tens of milliseconds of load and drops while the
    host prepares inputs, so a kernel timed right after host-side work would
    otherwise be timed partly at a lower clock."""
    import torch

    busy = _BUSY.get(str(dev))
    if busy is None:
        busy = _BUSY[str(dev)] = torch.full((8192, 8192), 1e-3, dtype=torch.float16, device=dev)
    end = time.perf_counter() + seconds
    while time.perf_counter() < end:
        for _ in range(4):
            torch.matmul(busy, busy)
        torch.cuda.synchronize()


def _steady_time(fn, warmup, iters, dev):
    """_events_time after a clock settle and `warmup` untimed calls."""
    _settle_clock(dev)
    _events_time(fn, warmup)
    return _events_time(fn, iters)


def seeded(shape, dtype, seed):
    import torch

    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def bench_partition(args, dev):
    import torch

    import crumpet_amd

    ops = torch.ops.crumpet_ops
    B, D, H, W, C, ws, ss = (C1[k] for k in ("B", "D", "H", "W", "C", "ws", "ss"))
    R = 4  # 4 x 180 MB rotating sets > 256 MB MALL
    xs = [seeded((B, D, H, W, C), torch.float16, 100 + r).to(dev) for r in range(R)]
    wins = [torch.empty((B * 2744, 343, C), dtype=torch.float16, device=dev) for _ in range(R)]
    backs = [torch.empty_like(xs[0]) for _ in range(R)]

    # correctness gate on the measured buffers: round trip restores the input
    w0 = crumpet_amd.fused_shift_partition_3d(xs[0], ws, ss)
    assert torch.equal(crumpet_amd.fused_unshift_unpartition_3d(w0, B, D, H, W, C, ws, ss), xs[0])
    del w0

    def part(i):
        ops.fused_shift_partition_3d(wins[i % R], xs[i % R], *ws, *ss)

    def unpart(i):
        ops.fused_unshift_unpartition_3d(backs[i % R], wins[i % R], B, D, H, W, C, *ws, *ss)

    def step(i):
        w = crumpet_amd.fused_shift_partition_3d(xs[i % R], ws, ss)
        crumpet_amd.fused_unshift_unpartition_3d(w, B, D, H, W, C, ws, ss)

    t_part = _steady_time(part, args.warmup, args.steps, dev)
    t_unpart = _steady_time(unpart, args.warmup, args.steps, dev)
    t_step = _steady_time(step, args.warmup, args.steps, dev)

    return dict(t_part=t_part, t_unpart=t_unpart, t_step=t_step)


def bench_mask(args, dev):
    import torch

    ops = torch.ops.crumpet_ops
    out = torch.empty((2744, 343, 343), dtype=torch.float16, device=dev)

    def mk(i):
        ops.compute_attn_mask_3d(out, 98, 98, 98, 7, 7, 7, 3, 3, 3)

    return _steady_time(mk, args.warmup, args.steps, dev)


def bench_eager_references(args, dev):
    """The reference's eager constructions for configs 1 and 2 on the same
    GPU, the comparison its own speedup figures make: torch.roll + the MONAI
    view/permute window partition and window reverse + roll back
    (torch-ext/crumpet/reference.py:141-184), and the MONAI slice-assignment
    mask (benchmarks/bench_kernel.py:63-86), fp32 then cast.  Each is first
    checked equal to the kernel's output.  Timed after every fused
    measurement: the eager constructions' large temporaries left fused
    launches measured after them slower."""
    import torch

    import crumpet_amd
    from crumpet_amd import swin_unetr_compat as sw

    B, D, H, W, C, ws, ss = (C1[k] for k in ("B", "D", "H", "W", "C", "ws", "ss"))
    R = 2
    xs = [seeded((B, D, H, W, C), torch.float16, 100 + r).to(dev) for r in range(R)]
    wins = [crumpet_amd.fused_shift_partition_3d(x, ws, ss) for x in xs]
    neg = tuple(-v for v in ss)
    assert torch.equal(sw.window_partition(torch.roll(xs[0], neg, (1, 2, 3)), ws), wins[0])
    assert torch.equal(torch.roll(sw.window_reverse(wins[0], ws, (B, D, H, W)), ss, (1, 2, 3)), xs[0])

    def eager_part(i):
        sw.window_partition(torch.roll(xs[i % R], neg, (1, 2, 3)), ws)

    def eager_unpart(i):
        torch.roll(sw.window_reverse(wins[i % R], ws, (B, D, H, W)), ss, (1, 2, 3))

    res = {"t_eager_part": _steady_time(eager_part, 3, 10, dev),
           "t_eager_unpart": _steady_time(eager_unpart, 3, 10, dev)}
    del xs, wins
    torch.cuda.empty_cache()
    out = torch.empty((2744, 343, 343), dtype=torch.float16, device=dev)
    torch.ops.crumpet_ops.compute_attn_mask_3d(out, 98, 98, 98, 7, 7, 7, 3, 3, 3)
    assert torch.equal(sw.compute_mask((98, 98, 98), (7, 7, 7), (3, 3, 3), dev).to(torch.float16), out)
    del out

    def eager_mask(i):
        sw.compute_mask((98, 98, 98), (7, 7, 7), (3, 3, 3), dev).to(torch.float16)

    res["t_eager_mask"] = _steady_time(eager_mask, 1, 5, dev)
    torch.cuda.empty_cache()
    return res


def c3_inputs(dev, sets):
    import torch

    from crumpet_amd import compute_attn_mask_3d

    B, H, N, Dh = C3["B"], C3["H"], C3["N"], C3["Dh"]
    qkvs = [seeded((B, N, 3 * H * Dh), torch.float16, 300 + r).to(dev) for r in range(sets)]
    g = torch.Generator().manual_seed(310)
    table = torch.empty((2197, H))
    torch.nn.init.trunc_normal_(table, std=0.02, a=-2.0, b=2.0, generator=g)
    import numpy as np

    c = np.stack(np.meshgrid(np.arange(7), np.arange(7), np.arange(7), indexing="ij")).reshape(3, -1)
    rel = (c[:, :, None] - c[:, None, :]) + 6
    rpi = torch.from_numpy((rel[0] * 13 + rel[1]) * 13 + rel[2])
    bias = table[rpi.reshape(-1)].reshape(N, N, H).permute(2, 0, 1).contiguous().half().to(dev)
    mask = compute_attn_mask_3d(C3["D"], C3["D"], C3["D"], (7, 7, 7), (3, 3, 3), torch.float16, dev)
    nw = mask.shape[0]
    flags = (mask.view(nw, -1).abs().amax(1) > 0).to(torch.uint8)
    bnd = flags.repeat(B // nw).contiguous()
    return qkvs, bias, mask, bnd


def bench_attention(args, dev):
    import torch

    from crumpet_amd.fused_attention import fused_swin_attention_windows

    B, H, N, Dh = C3["B"], C3["H"], C3["N"], C3["Dh"]
    R = 3  # 3 x 180 MB rotating sets > 256 MB MALL
    qkvs, bias, mask, bnd = c3_inputs(dev, R)
    views = [q.reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4) for q in qkvs]
    outs = [torch.empty((B, N, H * Dh), dtype=torch.float16, device=dev) for _ in range(R)]
    ovs = [o.view(B, N, H, Dh).permute(0, 2, 1, 3) for o in outs]

    def attn(i):
        t = views[i % R]
        fused_swin_attention_windows(t[0], t[1], t[2], bias, mask, bnd, 0.25, ovs[i % R])

    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    def attn_shifted(i):
        t = views[i % R]
        fused_swin_attention_shifted(t[0], t[1], t[2], bias, (C3["D"],) * 3, (7, 7, 7), (3, 3, 3),
                                     0.25, ovs[i % R])

    # The wrapper keeps a tiled copy of a mask it sees twice (fused_attention
    # mask_tiles), so the steady state reads the tiled copy; the row-major
    # read (the op without the copy) and the copy's one-time cost are timed
    # beside it.
    import crumpet_amd
    from crumpet_amd.fused_attention import mask_tiles

    ops = crumpet_amd._native.ops()

    def attn_row_major(i):
        t = views[i % R]
        ops.fused_swin_attention(ovs[i % R], t[0], t[1], t[2], bias, mask, bnd, 0.25)

    # The first hundred or so attention launches of a process run up to 7%
    # slower than the rest (measured: whichever of these calls is timed
    # first, even after a 1 s clock settle), so an untimed pre-pass of 200
    # launches (about 30 ms) comes before the first timing.
    _events_time(attn, 200)
    t_attn = _steady_time(attn, args.warmup, args.steps, dev)
    t_shift = _steady_time(attn_shifted, args.warmup, args.steps, dev)
    res = dict(t_attn=t_attn, t_shift=t_shift)
    res["t_attn_row_major"] = _steady_time(attn_row_major, args.warmup, args.steps, dev)
    res["t_mask_tiles"] = _steady_time(lambda i: mask_tiles(mask), 2, 10, dev)

    # The layout the reference's own patch hands the kernel
    # (torch-ext/crumpet/monai_patch.py:167-191): the mask repeated over the
    # outer batch to [1372, 343, 343] and one flag per window from
    # abs().amax over its mask; window b then reads mask row block b.  Timed
    # as the kernel alone (mask and flags built once) and as the patch's
    # whole per-call sequence (repeat, flags, attention).
    from crumpet_amd.fused_attention import fused_swin_attention

    mask_rep = mask.repeat(B // mask.shape[0], 1, 1)
    bnd_rep = (mask_rep.abs().amax(dim=(1, 2)) > 0).to(torch.uint8)

    def attn_rep(i):
        t = views[i % R]
        fused_swin_attention(t[0], t[1], t[2], bias, mask_rep, bnd_rep, 0.25, out=ovs[i % R])

    def attn_rep_call(i):
        t = views[i % R]
        m = mask.repeat(B // mask.shape[0], 1, 1)
        fl = (m.abs().amax(dim=(1, 2)) > 0).to(torch.uint8)
        fused_swin_attention(t[0], t[1], t[2], bias, m, fl, 0.25, out=ovs[i % R])

    res["t_attn_rep"] = _steady_time(attn_rep, args.warmup, args.steps, dev)
    res["t_attn_rep_call"] = _steady_time(attn_rep_call, args.warmup, max(10, args.steps // 2), dev)
    attn_rep(0)
    torch.cuda.synchronize()
    rep_out = ovs[0].clone()
    attn(0)
    torch.cuda.synchronize()
    res["rep_equals_343_form"] = bool(torch.equal(rep_out, ovs[0]))
    del mask_rep, bnd_rep, rep_out
    torch.cuda.empty_cache()

    # accuracy on a sample of windows vs fp32 torch (GPU) of the same inputs
    t = views[0]
    attn(0)
    torch.cuda.synchronize()
    idx = torch.arange(0, B, 7, device=dev)
    qf, kf, vf = (t[j][idx].float() for j in range(3))
    s = (qf * 0.25) @ kf.transpose(-1, -2).contiguous() + bias.float()[None]
    mb = (mask.float()[idx % mask.shape[0]] * bnd[idx].float()[:, None, None])[:, None]
    ref = torch.softmax(s + mb, dim=-1) @ vf
    res["max_abs_err"] = float((ovs[0][idx].float() - ref).abs().max())
    attn_shifted(0)
    torch.cuda.synchronize()
    res["max_abs_err_shifted"] = float((ovs[0][idx].float() - ref).abs().max())
    del qf, kf, vf, s, mb, ref

    if not args.no_eager:
        # MONAI eager chain in fp16 on the same GPU (the "eager ROCm PyTorch" comparison)
        def eager(i):
            tt = views[i % R]
            q = tt[0] * 0.25
            a = q @ tt[1].transpose(-2, -1).contiguous()
            a = a + bias.unsqueeze(0)
            nw = mask.shape[0]
            a = a.view(B // nw, nw, H, N, N) + mask.unsqueeze(1).unsqueeze(0)
            a = torch.softmax(a.view(-1, H, N, N), dim=-1)
            return (a @ tt[2]).transpose(1, 2).reshape(B, N, H * Dh)

        with torch.no_grad():
            _events_time(eager, 2)
            res["t_eager"] = _events_time(eager, max(3, min(args.steps, 10)))
        torch.cuda.empty_cache()
    return res


def bench_attention_wide(args, dev):
    """Head dim 32 (Swin UNETR at feature size 96) at the config-3 window
    shape: 1372 windows x 3 heads, N = 343, fp16, through the tuned kernel's
    head-dim-32 form, shifted (region) and with the mask tensor, against the
    eager chain."""
    import torch

    from crumpet_amd.fused_attention import fused_swin_attention_shifted, fused_swin_attention_windows

    B, H, N, Dh = C3["B"], C3["H"], C3["N"], 32
    R = 2  # 2 x 361 MB rotating sets > 256 MB MALL
    _, bias, mask, bnd = c3_inputs(dev, 0)
    qkvs = [seeded((B, N, 3 * H * Dh), torch.float16, 320 + r).to(dev) for r in range(R)]
    views = [q.reshape(B, N, 3, H, Dh).permute(2, 0, 3, 1, 4) for q in qkvs]
    outs = [torch.empty((B, N, H * Dh), dtype=torch.float16, device=dev) for _ in range(R)]
    ovs = [o.view(B, N, H, Dh).permute(0, 2, 1, 3) for o in outs]

    def shifted(i):
        t = views[i % R]
        fused_swin_attention_shifted(t[0], t[1], t[2], bias, (C3["D"],) * 3, (7, 7, 7), (3, 3, 3), 0.25,
                                     ovs[i % R])

    def tensor(i):
        t = views[i % R]
        fused_swin_attention_windows(t[0], t[1], t[2], bias, mask, bnd, 0.25, ovs[i % R])

    steps = max(5, args.steps // 4)
    res = {"t_shift": _steady_time(shifted, 3, steps, dev)}
    res["t_tensor"] = _steady_time(tensor, 3, steps, dev)
    t = views[0]
    idx = torch.arange(0, B, 7, device=dev)
    qf, kf, vf = (t[j][idx].float() for j in range(3))
    s = (qf * 0.25) @ kf.transpose(-1, -2).contiguous() + bias.float()[None]
    mb = (mask.float()[idx % mask.shape[0]] * bnd[idx].float()[:, None, None])[:, None]
    ref = torch.softmax(s + mb, dim=-1) @ vf
    err = 0.0
    for fn in (shifted, tensor):
        fn(0)
        torch.cuda.synchronize()
        err = max(err, float((ovs[0][idx].float() - ref).abs().max()))
    res["max_abs_err"] = err
    del qf, kf, vf, s, mb, ref
    if not args.no_eager:
        def eager(i):
            tt = views[i % R]
            a = (tt[0] * 0.25) @ tt[1].transpose(-2, -1).contiguous()
            a = a + bias.unsqueeze(0)
            nw = mask.shape[0]
            a = a.view(B // nw, nw, H, N, N) + mask.unsqueeze(1).unsqueeze(0)
            a = torch.softmax(a.view(-1, H, N, N), dim=-1)
            return (a @ tt[2]).transpose(1, 2).reshape(B, N, H * Dh)

        with torch.no_grad():
            _events_time(eager, 2)
            res["t_eager"] = _events_time(eager, 5)
    torch.cuda.empty_cache()
    return res


STAGES = [  # config 4: (name, padded dim, C, heads, window, shift)
    ("s1", 28, 96, 6, (7, 7, 7), (3, 3, 3)),
    ("s2", 14, 192, 12, (7, 7, 7), (3, 3, 3)),
    ("s3", 7, 384, 24, (7, 7, 7), (0, 0, 0)),
    ("s3_monai", 6, 384, 24, (6, 6, 6), (0, 0, 0)),
]


def bench_blocks(args, dev):
    """Config 4: partition -> fused attention -> unpartition per Swin stage, B=4.

    The windows' C channels are read as H heads of 16.  q is the freshly
    partitioned tokens; k and v are the same tokens with the heads rotated
    by one and two (the workload tests/test_gpu_block_path.py checks:
    independent of q, as a qkv projection makes them), held in buffers made
    once before timing, so the timed chain is exactly the three hot-path
    kernels (the qkv/proj linears are library GEMMs outside the path).
    ``ms_qkv_equal`` times the same chain with k = v = q: every row's
    diagonal score is then 0.25 |q|^2, and in fp16 the rows whose diagonal
    passes 2^16 take the offset softmax's exact pass."""
    import torch

    import crumpet_amd
    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    res = {}
    eager_jobs = []
    B = 4
    for dtype, tag in ((torch.float16, "fp16"), (torch.bfloat16, "bf16")):
        for name, dim, C, H, ws, ss in STAGES:
            x = seeded((B, dim, dim, dim, C), dtype, 500 + dim).to(dev)
            N = ws[0] * ws[1] * ws[2]
            g = torch.Generator().manual_seed(510 + dim)
            table = torch.empty(((2 * ws[0] - 1) * (2 * ws[1] - 1) * (2 * ws[2] - 1), H))
            torch.nn.init.trunc_normal_(table, std=0.02, a=-2.0, b=2.0, generator=g)
            import numpy as np

            c = np.stack(np.meshgrid(*(np.arange(w) for w in ws), indexing="ij")).reshape(3, -1)
            rel = c[:, :, None] - c[:, None, :] + np.array(ws)[:, None, None] - 1
            rpi = torch.from_numpy((rel[0] * (2 * ws[1] - 1) + rel[1]) * (2 * ws[2] - 1) + rel[2])
            bias = table[rpi.reshape(-1)].reshape(N, N, H).permute(2, 0, 1).contiguous().to(dtype).to(dev)

            w0 = crumpet_amd.fused_shift_partition_3d(x, ws, ss)
            t0 = w0.view(w0.shape[0], N, H, 16).permute(0, 2, 1, 3)
            tk = torch.roll(t0, 1, dims=1)  # heads rotated by one and two
            tv = torch.roll(t0, 2, dims=1)
            del w0, t0

            def chain(rotated):
                def step(i):
                    w = crumpet_amd.fused_shift_partition_3d(x, ws, ss)
                    nwin = w.shape[0]
                    t = w.view(nwin, N, H, 16).permute(0, 2, 1, 3)
                    o = torch.empty_like(w)
                    fused_swin_attention_shifted(t, tk if rotated else t, tv if rotated else t, bias, (dim,) * 3,
                                                 ws, ss, 0.25, o.view(nwin, N, H, 16).permute(0, 2, 1, 3))
                    crumpet_amd.fused_unshift_unpartition_3d(o, B, dim, dim, dim, C, ws, ss)
                return step

            step = chain(True)
            ms = _steady_time(step, args.warmup, args.steps, dev)
            ms_equal = _steady_time(chain(False), args.warmup, args.steps, dev)
            # the same three launches replayed as one HIP graph (no host launch overhead)
            cap = torch.cuda.Stream()
            cap.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(cap):
                step(0)
            torch.cuda.current_stream().wait_stream(cap)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cap):
                step(0)
            ms_graph = _steady_time(lambda i: graph.replay(), args.warmup, args.steps, dev)
            del graph
            eager_jobs.append((f"{name}_{tag}", x, bias, dtype, dim, C, H, ws, ss, N))
            tokens = B * dim ** 3
            part_bytes = 2 * tokens * C * x.element_size()
            flops = 4 * N * N * 16 * H * (tokens // N)
            del tk, tv
            res[f"{name}_{tag}"] = {"ms": round(ms, 5), "ms_graph_replay": round(ms_graph, 5),
                                    "ms_qkv_equal": round(ms_equal, 5),
                                    "shape": [B, dim, dim, dim, C], "heads": H,
                                    "window": list(ws), "shift": list(ss),
                                    "partition_bytes": part_bytes, "attention_flops": flops,
                                    "effective_GB_s": round(3 * part_bytes / (ms * 1e-3) / 1e9, 1)}

    # the eager chain on the same GPU, after every fused measurement (its
    # large temporaries left eager fused launches measured after it several
    # times slower): roll + window partition, the MONAI attention chain (mask
    # from compute_mask, cached as MONAI's BasicLayer does), window reverse +
    # roll back
    from crumpet_amd import swin_unetr_compat as sw

    for key, x, bias, dtype, dim, C, H, ws, ss, N in eager_jobs:
        shifted = any(ss)
        emask = sw.compute_mask((dim,) * 3, ws, ss, dev).to(dtype) if shifted else None

        def eager_step(i):
            xr = torch.roll(x, tuple(-v for v in ss), (1, 2, 3)) if shifted else x
            w = sw.window_partition(xr, ws)
            nwin = w.shape[0]
            t = w.view(nwin, N, H, 16).permute(0, 2, 1, 3)
            a = (t * 0.25) @ t.transpose(-2, -1).contiguous() + bias.unsqueeze(0)
            if shifted:
                nw = emask.shape[0]
                a = (a.view(nwin // nw, nw, H, N, N) + emask.unsqueeze(1).unsqueeze(0)).view(-1, H, N, N)
            o = (torch.softmax(a, dim=-1) @ t).transpose(1, 2).reshape(nwin, N, C)
            back = sw.window_reverse(o, ws, (B, dim, dim, dim))
            return torch.roll(back, ss, (1, 2, 3)) if shifted else back

        with torch.no_grad():
            ms_eager = _steady_time(eager_step, 2, max(3, min(args.steps, 10)), dev)
        res[key]["eager_rocm_ms"] = round(ms_eager, 4)
        res[key]["speedup_vs_eager"] = round(ms_eager / res[key]["ms"], 2)
        res[key]["speedup_vs_eager_graph"] = round(ms_eager / res[key]["ms_graph_replay"], 2)
        del emask
    del eager_jobs
    torch.cuda.empty_cache()
    return res


FUSED_STAGES = [  # config 5 stage shapes at B=4: (name, dim, C, heads, shift)
    ("s0", 48, 48, 3, 3),
    ("s1", 24, 96, 6, 3),
    ("s2", 12, 192, 12, 3),
    ("s3", 6, 384, 24, 0),
]


def bench_fused_block(args, dev):
    """The attention half of a Swin block (forward_part1) at the config-5
    stage shapes, B=4, under fp16 autocast (fp32 block input, fp16 Linear and
    attention): the fused block kernels (window_qkv_3d -> attention ->
    window_proj_3d) against the patched unfused path (torch LayerNorm, F.pad,
    partition kernel, torch Linear, attention kernel, torch Linear,
    unpartition kernel, crop) and the unpatched eager MONAI chain.  The two
    projection kernels are also timed alone against their HBM bytes."""
    import torch

    import crumpet_amd
    from crumpet_amd import monai_patch
    from crumpet_amd import swin_unetr_compat as sw

    res = {}
    crumpet_amd.unpatch_monai_swin_unetr()
    for name, dim, C, H, shift in FUSED_STAGES:
        B = 4
        torch.manual_seed(700 + dim)
        blk = sw.SwinTransformerBlock(dim=C, num_heads=H, window_size=(7, 7, 7),
                                      shift_size=(shift,) * 3).to(dev).eval()
        x = seeded((B, dim, dim, dim, C), torch.float32, 710 + dim).to(dev)
        ws, ss = sw.get_window_size((dim,) * 3, blk.window_size, blk.shift_size)
        ws, ss = tuple(ws), tuple(ss)
        padded = tuple(-(-dim // w) * w for w in ws)
        shifted = any(v > 0 for v in ss)
        m_eager = sw.compute_mask(padded, ws, ss, dev) if shifted else None
        m_patch = None
        if shifted:
            m_patch = crumpet_amd.compute_attn_mask_3d(*padded, ws, ss, torch.float32, dev)
            setattr(m_patch, monai_patch._GEOMETRY_ATTR, (*padded, ws, ss))

        def run(fn):
            def step(i):
                with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16):
                    fn()
            return _steady_time(step, args.warmup, max(10, args.steps // 4), dev)

        t_eager = run(lambda: blk.forward_part1(x, m_eager))
        assert crumpet_amd.patch_monai_swin_unetr()
        try:
            with torch.autocast("cuda", dtype=torch.float16):
                assert monai_patch._fused_block_supported(blk, x)
            t_fused = run(lambda: monai_patch._fused_block_forward(blk, x, m_patch, sw))
            os.environ["CRUMPET_DISABLE_FUSED_BLOCK"] = "1"
            try:
                t_unfused = run(lambda: blk.forward_part1(x, m_patch))
            finally:
                os.environ.pop("CRUMPET_DISABLE_FUSED_BLOCK", None)
        finally:
            crumpet_amd.unpatch_monai_swin_unetr()

        # the two projection kernels alone
        w_qkv = blk.attn.qkv.weight.detach().half()
        b_qkv = blk.attn.qkv.bias.detach().half()
        w_p = blk.attn.proj.weight.detach().half()
        b_p = blk.attn.proj.bias.detach().half()
        nw = (padded[0] // ws[0]) * (padded[1] // ws[1]) * (padded[2] // ws[2])
        n = ws[0] * ws[1] * ws[2]
        # two rotating buffer sets, as in the profiled sequence
        xs = [x, seeded(tuple(x.shape), torch.float32, 711 + dim).to(dev)]
        qkv_outs = [torch.empty((B * nw, n, 3 * C), dtype=torch.float16, device=dev) for _ in range(2)]
        wins = [seeded((B * nw, n, C), torch.float16, 720 + dim + r).to(dev) for r in range(2)]
        ys = [torch.empty((B, dim, dim, dim, C), dtype=torch.float16, device=dev) for _ in range(2)]
        nrm = blk.norm1
        ops = torch.ops.crumpet_ops  # raw ops: no wrapper overhead between launches
        f_qkv = lambda i: ops.window_qkv_3d(qkv_outs[i % 2], xs[i % 2], nrm.weight, nrm.bias, nrm.eps, True,
                                            w_qkv, b_qkv, *ws, *ss)
        f_proj = lambda i: ops.window_proj_3d(ys[i % 2], wins[i % 2], w_p, b_p, *ws, *ss)
        # (the warm-up calls keep the first touches of the fresh buffers untimed)
        t_qkv = _steady_time(f_qkv, args.warmup, args.steps, dev)
        t_proj = _steady_time(f_proj, args.warmup, args.steps, dev)
        qkv_bytes = x.numel() * 4 + qkv_outs[0].numel() * 2
        proj_bytes = wins[0].numel() * 2 + ys[0].numel() * 2
        gq = qkv_bytes / (t_qkv * 1e-3) / 1e9
        gp = proj_bytes / (t_proj * 1e-3) / 1e9
        res[name] = {
            "shape": [B, dim, dim, dim, C], "heads": H, "window": list(ws), "shift": list(ss),
            "ms_fused": round(t_fused, 5), "ms_unfused_patched": round(t_unfused, 5),
            "ms_eager": round(t_eager, 5), "speedup_vs_unfused": round(t_unfused / t_fused, 3),
            "speedup_vs_eager": round(t_eager / t_fused, 3),
            "window_qkv": {"ms": round(t_qkv, 5), "bytes": qkv_bytes, "GB_s": round(gq, 1),
                           "frac_hbm": round(gq / HBM_PEAK_GBS, 4)},
            "window_proj": {"ms": round(t_proj, 5), "bytes": proj_bytes, "GB_s": round(gp, 1),
                            "frac_hbm": round(gp / HBM_PEAK_GBS, 4)},
        }
        del x, xs, qkv_outs, wins, ys, blk
        torch.cuda.empty_cache()
    return res


def bench_e2e(args, dev):
    """Config 5: MONAI-style Swin UNETR forward, [4,1,96,96,96] fp16 input,
    fp16 autocast, patched vs unpatched eager on the same weights."""
    import statistics

    import torch

    import crumpet_amd
    from crumpet_amd import swin_unetr_compat as sw

    crumpet_amd.unpatch_monai_swin_unetr()
    torch.manual_seed(123)
    model = sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=48, depths=(2, 2, 2, 2),
                         num_heads=(3, 6, 12, 24)).to(dev).eval()
    x = synthetic_ct((4, 1, 96, 96, 96), 77).half().to(dev)

    def timed(n):
        times = []
        y = None
        with torch.no_grad():
            for _ in range(n):
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                with torch.autocast("cuda", dtype=torch.float16):
                    y = model(x)
                e.record()
                torch.cuda.synchronize()
                times.append(s.elapsed_time(e))
        return statistics.median(times), y

    iters = max(3, min(10, args.steps // 10))
    timed(2)
    t_eager, y_eager = timed(iters)
    assert crumpet_amd.patch_monai_swin_unetr()
    try:
        timed(2)
        t_patch, y_patch = timed(iters)
    finally:
        crumpet_amd.unpatch_monai_swin_unetr()
    delta = float((y_patch.float() - y_eager.float()).abs().max())
    return {"ms_patched": round(t_patch, 3), "ms_eager": round(t_eager, 3),
            "speedup": round(t_eager / t_patch, 3), "max_abs_logit_delta": delta,
            "max_abs_logit": float(y_eager.float().abs().max()), "iters": iters,
            "workload": "config 5: SwinUNETR(1->14, feature 48, depths 2222, heads 3/6/12/24), "
                        "input [4,1,96,96,96] fp16 (uniform + Gaussian blobs), fp16 autocast, "
                        "median of iters forwards"}


def cpu_scalar_oracle():
    """The C oracle's scalar round trip (1 thread) on the full config-1 volume,
    reported beside the reference's eager CPU path."""
    import numpy as np

    from oracle import oracle

    oracle.build_oracle()
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 98, 98, 98, 48)).astype(np.float16)
    oracle.shift_partition(x, (7, 7, 7), (3, 3, 3))  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        w = oracle.shift_partition(x, (7, 7, 7), (3, 3, 3))
        oracle.unshift_unpartition(w, 1, 98, 98, 98, 48, (7, 7, 7), (3, 3, 3))
        reps += 1
        el = time.perf_counter() - t0
        if el > 10.0 or reps >= 50:
            break
    gbs = 2 * C1_BYTES * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"full config-1 round trip ([1,98^3,48] fp16) x{reps}, oracle/crumpet_oracle.c scalar, {el:.1f} s"}


def _cpu_median(fn, reps):
    import statistics

    fn()  # warm
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def _cpu_attention(q, k, v, bias, mask, scale):
    """fp32 eager chain (fused_attention.py:82-146 semantics): q*scale k^T +
    bias (+ mask) -> softmax -> @ v, on [b, H, N, 16] CPU tensors."""
    import torch

    s = (q * scale) @ k.transpose(-1, -2) + bias[None]
    if mask is not None:
        s = s + mask[:, None]
    return torch.softmax(s, dim=-1) @ v


def cpu_mask_where(D, H, W, ws, ss, dtype):
    """The vectorised eager mask of torch-ext/crumpet/reference.py:50-98, in
    torch on the CPU: per-axis region labels (0 below D - ws, 1 below D - ss,
    else 2) combined as 9 r_d + 3 r_h + r_w, window partition, pairwise
    comparison of the labels, -100 where they differ."""
    import torch

    from crumpet_amd import swin_unetr_compat as sw

    def regions(n, w, s):
        a = torch.arange(n)
        return torch.where(a < n - w, 0, torch.where(a < n - s, 1, 2))

    labels = (9 * regions(D, ws[0], ss[0])[:, None, None] + 3 * regions(H, ws[1], ss[1])[None, :, None]
              + regions(W, ws[2], ss[2])[None, None, :]).to(torch.int16)
    win = sw.window_partition(labels.view(1, D, H, W, 1), ws)[..., 0]
    differ = win[:, None, :] != win[:, :, None]
    return torch.where(differ, torch.tensor(-100.0, dtype=dtype), torch.tensor(0.0, dtype=dtype))


def cpu_eager_paths(skip_e2e=False):
    """The reference's eager paths timed on the host cores, one per config,
    each on a bounded sample stated in its entry (reported baselines only,
    never targets): torch roll + view/permute (config 1), the two eager mask
    constructions (config 2), the fp32 attention chain (configs 3 and 4) and
    the unpatched fp32 Swin UNETR forward (config 5)."""
    import torch

    from crumpet_amd import swin_unetr_compat as sw
    from oracle import oracle

    threads = torch.get_num_threads()
    res = {}

    # config 1: torch.roll + window partition and its inverse, fp16, full volume
    x = seeded((1, 98, 98, 98, 48), torch.float16, 100)

    def roundtrip():
        w = sw.window_partition(torch.roll(x, (-3, -3, -3), (1, 2, 3)), (7, 7, 7))
        torch.roll(sw.window_reverse(w, (7, 7, 7), (1, 98, 98, 98)), (3, 3, 3), (1, 2, 3))

    t = _cpu_median(roundtrip, 3)
    res["roundtrip"] = {"ms": round(t * 1e3, 2), "GB_s": round(2 * C1_BYTES / t / 1e9, 3), "threads": threads,
                        "sample": "full config 1, torch.roll + view/permute and the inverse, fp16, "
                                  "median of 3"}
    del x

    # config 2 at full size: the MONAI slice-assignment construction
    # (benchmarks/bench_kernel.py:63-86, as MONAI's compute_mask in the compat
    # model, fp32 then cast) and the vectorised where (reference.py:50-98),
    # fp16 [2744, 343, 343]; GB/s of fp16 output.  The two agree bit for bit.
    ws7, ss3 = (7, 7, 7), (3, 3, 3)
    t_monai = _cpu_median(lambda: sw.compute_mask((98, 98, 98), ws7, ss3, "cpu").to(torch.float16), 2)
    t_where = _cpu_median(lambda: cpu_mask_where(98, 98, 98, ws7, ss3, torch.float16), 2)
    same = torch.equal(sw.compute_mask((98, 98, 98), ws7, ss3, "cpu").to(torch.float16),
                       cpu_mask_where(98, 98, 98, ws7, ss3, torch.float16))
    res["mask"] = {"ms_monai_slices": round(t_monai * 1e3, 1), "ms_where": round(t_where * 1e3, 1),
                   "GB_s": round(C2_BYTES / min(t_monai, t_where) / 1e9, 3), "threads": threads,
                   "constructions_equal": same,
                   "sample": "full config 2 (98^3, [2744,343,343] fp16, 645.7 MB out), torch on the CPU, "
                             "median of 2 each"}

    # config 3: fp32 eager attention on every 14th window (98 of 1372)
    g = torch.Generator().manual_seed(300)
    qkv = torch.randn((98, 343, 144), generator=g).half().float()
    t3 = qkv.view(98, 343, 3, 3, 16).permute(2, 0, 3, 1, 4)
    bias = torch.randn((3, 343, 343), generator=g) * 0.02
    mask = torch.from_numpy(oracle.attn_mask(49, 49, 49, (7, 7, 7), (3, 3, 3), "float32"))[:98]
    t = _cpu_median(lambda: _cpu_attention(t3[0], t3[1], t3[2], bias, mask, 0.25), 3)
    fl = 4 * 343 * 343 * 16 * 3 * 98
    res["attention"] = {"ms": round(t * 1e3, 2), "TFLOP_s": round(fl / t / 1e12, 4),
                        "ms_config3_scaled": round(t * 1e3 * 1372 / 98, 1), "threads": threads,
                        "sample": "98 of the 1372 windows x 3 heads, fp32 torch on CPU, median of 3"}
    del qkv, t3

    # config 4: partition -> fp32 attention -> unpartition per stage (fp32 math on the fp16 input)
    for name, dim, C, H, ws, ss in STAGES[:3]:
        x = seeded((4, dim, dim, dim, C), torch.float16, 500 + dim).float()
        N = ws[0] * ws[1] * ws[2]
        b = torch.randn((H, N, N), generator=g) * 0.02
        m = torch.from_numpy(oracle.attn_mask(dim, dim, dim, ws, ss, "float32")) if any(ss) else None

        def chain():
            w = sw.window_partition(torch.roll(x, tuple(-s for s in ss), (1, 2, 3)), ws)
            nw = w.shape[0]
            t_ = w.view(nw, N, H, 16).permute(0, 2, 1, 3)
            mm = m.repeat(nw // m.shape[0], 1, 1) if m is not None else None
            o = _cpu_attention(t_, t_, t_, b, mm, 0.25).permute(0, 2, 1, 3).reshape(nw, N, C)
            torch.roll(sw.window_reverse(o, ws, (4, dim, dim, dim)), ss, (1, 2, 3))

        res[f"block_path_{name}"] = {"ms": round(_cpu_median(chain, 1) * 1e3, 2), "threads": threads,
                                     "sample": f"full stage [4,{dim}^3,{C}], fp32, median of 1"}

    # config 5: unpatched fp32 Swin UNETR forward, one sample of the batch of 4
    if not skip_e2e:
        torch.manual_seed(123)
        model = sw.SwinUNETR(in_channels=1, out_channels=14, feature_size=48, depths=(2, 2, 2, 2),
                             num_heads=(3, 6, 12, 24)).eval()
        xin = synthetic_ct((1, 1, 96, 96, 96), 77)
        with torch.no_grad():
            t = _cpu_median(lambda: model(xin), 1)
        res["swin_unetr_e2e"] = {"ms_per_sample": round(t * 1e3, 1), "ms_batch4_scaled": round(4 * t * 1e3, 1),
                                 "threads": threads,
                                 "sample": "[1,1,96^3] fp32 unpatched eager forward (one of the 4 "
                                           "samples), median of 1 after a warm-up"}
    return res


def profile_run(dev):
    """Fixed short sequence for rocprofv3: 2 + 20 launches of each kernel on
    rotating buffers, each kernel after 0.15 s of torch matmuls that bring
    the shader clock to its loaded rate, plus a plain 256 MiB device
    copy (read 256 MiB + write 256 MiB) for scaling the FETCH_SIZE /
    WRITE_SIZE counters.  Each kernel's
    last 20 back-to-back launches are timed with one HIP event pair; the last line
    printed holds the mean per-launch times, so a run without the profiler
    gives the undisturbed durations of the same launches."""
    import torch

    from crumpet_amd.fused_attention import fused_swin_attention_shifted

    ops = torch.ops.crumpet_ops
    n = 100
    times = {}
    def timed(name, fn):
        # the timing of bench.py's components: a clock settle, 10 untimed
        # launches (the first loads the code object), 100 timed (an
        # attention kernel's first 20 launches after the settle ran about
        # 4% faster than its 100-launch average)
        _settle_clock(dev)
        for i in range(10):
            fn(i)
        times[name] = round(_events_time(fn, n) * 1e3, 2)
    B, D, H, W, C, ws, ss = (C1[k] for k in ("B", "D", "H", "W", "C", "ws", "ss"))
    R = 4
    xs = [seeded((B, D, H, W, C), torch.float16, 100 + r).to(dev) for r in range(R)]
    wins = [torch.empty((2744, 343, C), dtype=torch.float16, device=dev) for _ in range(R)]
    backs = [torch.empty_like(xs[0]) for _ in range(R)]
    src = torch.ones((1 << 27,), dtype=torch.float16, device=dev)
    dst = torch.empty_like(src)
    timed("partition", lambda i: ops.fused_shift_partition_3d(wins[i % R], xs[i % R], *ws, *ss))
    timed("unpartition",
          lambda i: ops.fused_unshift_unpartition_3d(backs[i % R], wins[i % R], B, D, H, W, C, *ws, *ss))
    del xs, wins, backs
    outs = [torch.empty((2744, 343, 343), dtype=torch.float16, device=dev) for _ in range(2)]
    timed("mask", lambda i: ops.compute_attn_mask_3d(outs[i % 2], 98, 98, 98, 7, 7, 7, 3, 3, 3))
    for i in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    del outs

    qkvs, bias, mask, bnd = c3_inputs(dev, 3)
    Bw, Hh, N, Dh = C3["B"], C3["H"], C3["N"], C3["Dh"]
    # three rotating input and output sets, as bench_attention times them
    # (one output buffer rewritten by every launch stays partly in the MALL
    # and read about 4% faster)
    os_ = [torch.empty((Bw, N, Hh * Dh), dtype=torch.float16, device=dev) for _ in range(3)]
    ovs = [o.view(Bw, N, Hh, Dh).permute(0, 2, 1, 3) for o in os_]
    views = [q.reshape(Bw, N, 3, Hh, Dh).permute(2, 0, 3, 1, 4) for q in qkvs]
    # the tensor-mask kernel reading the mask itself, then its tiled copy
    # (what fused_swin_attention_windows does from its second call with a
    # mask; the copy is made once here, outside the timed launches)
    from crumpet_amd.fused_attention import mask_tiles

    def att(i, *extra):
        t = views[i % 3]
        return (ovs[i % 3], t[0], t[1], t[2], bias) + extra

    # untimed pre-pass: the first hundred or so attention launches of a
    # process run slower (see bench_attention); the profile summaries take
    # each kernel's last 20 launches, the timed ones
    for i in range(200):
        ops.fused_swin_attention(*att(i, mask, bnd, 0.25))
    timed("attention_tensor_mask_row_major", lambda i: ops.fused_swin_attention(*att(i, mask, bnd, 0.25)))
    tiles = mask_tiles(mask)
    timed("attention_tensor_mask", lambda i: ops.fused_swin_attention_tiled(*att(i, mask, tiles, bnd, 0.25)))
    del tiles
    vol = (C3["D"],) * 3
    timed("attention_shifted",
          lambda i: fused_swin_attention_shifted(views[i % 3][0], views[i % 3][1], views[i % 3][2], bias, vol,
                                                 (7, 7, 7), (3, 3, 3), 0.25, ovs[i % 3]))
    del qkvs, views, os_, ovs, mask
    # head dim 32 at the same window shape, shifted mode (the tuned kernel's
    # strip-group form); two rotating input and output sets
    qkvs = [seeded((Bw, N, 3 * Hh * 32), torch.float16, 320 + r).to(dev) for r in range(2)]
    views = [q.reshape(Bw, N, 3, Hh, 32).permute(2, 0, 3, 1, 4) for q in qkvs]
    os_ = [torch.empty((Bw, N, Hh * 32), dtype=torch.float16, device=dev) for _ in range(2)]
    ovs = [o.view(Bw, N, Hh, 32).permute(0, 2, 1, 3) for o in os_]
    timed("attention_hd32_shifted",
          lambda i: fused_swin_attention_shifted(views[i % 2][0], views[i % 2][1], views[i % 2][2], bias, vol,
                                                 (7, 7, 7), (3, 3, 3), 0.25, ovs[i % 2]))
    del qkvs, views, os_, ovs

    # fused block projections at the config-5 stage-0 shape: fp32 block
    # input [4,48^3,48] -> fp16 qkv [1372,343,144]; fp16 attention output
    # [1372,343,48] -> fp16 block output [4,48^3,48]; 2 rotating sets
    from crumpet_amd import fused_block

    C0 = 48
    xs = [seeded((4, 48, 48, 48, C0), torch.float32, 130 + r).to(dev) for r in range(2)]
    gw = torch.ones(C0, device=dev)
    gb = torch.zeros(C0, device=dev)
    wq = (seeded((3 * C0, C0), torch.float32, 134) / C0 ** 0.5).half().to(dev)
    bq = torch.zeros(3 * C0, dtype=torch.float16, device=dev)
    qouts = [torch.empty((1372, 343, 3 * C0), dtype=torch.float16, device=dev) for _ in range(2)]
    timed("window_qkv", lambda i: fused_block.window_qkv_3d(xs[i % 2], wq, bq, (7, 7, 7), (3, 3, 3), gw, gb, 1e-5,
                                                            True, torch.float16, qouts[i % 2]))
    del xs, qouts
    wins = [seeded((1372, 343, C0), torch.float16, 135 + r).to(dev) for r in range(2)]
    wp = (seeded((C0, C0), torch.float32, 137) / C0 ** 0.5).half().to(dev)
    ys = [torch.empty((4, 48, 48, 48, C0), dtype=torch.float16, device=dev) for _ in range(2)]
    timed("window_proj", lambda i: fused_block.window_proj_3d(wins[i % 2], wp, None, 4, 48, 48, 48, (7, 7, 7),
                                                              (3, 3, 3), ys[i % 2]))
    del wins, ys
    # window_qkv at the config-5 stage-1 and stage-2 shapes (the LDS-weight
    # streaming kernel): fp32 [4,24^3,96] -> fp16 [256,343,288] and fp32
    # [4,12^3,192] -> fp16 [32,343,576]; 2 rotating sets
    for name, dim, cs, nwin in (("window_qkv_s1", 24, 96, 256), ("window_qkv_s2", 12, 192, 32)):
        xs = [seeded((4, dim, dim, dim, cs), torch.float32, 140 + r).to(dev) for r in range(2)]
        g1 = torch.ones(cs, device=dev)
        b1 = torch.zeros(cs, device=dev)
        w1 = (seeded((3 * cs, cs), torch.float32, 144) / cs ** 0.5).half().to(dev)
        q1 = [torch.empty((nwin, 343, 3 * cs), dtype=torch.float16, device=dev) for _ in range(2)]
        timed(name, lambda i: fused_block.window_qkv_3d(xs[i % 2], w1, None, (7, 7, 7), (3, 3, 3), g1, b1, 1e-5,
                                                        True, torch.float16, q1[i % 2]))
        del xs, q1
    print("profile sequence done", flush=True)
    print("PROFILE_EVENTS_US " + json.dumps(times), flush=True)


def profiled_traffic(name):
    """HBM bytes per launch of a kernel, as measured by the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), or None."""
    path = ROOT / "profiles" / "window_gather_c1.md"
    try:
        for line in path.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "TRAFFIC" and parts[1] == name:
                return int(parts[2])
    except OSError:
        return None
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); "
              "the shifted-window path is single-GPU in this build", file=sys.stderr)
        sys.exit(2)
    import torch

    import crumpet_amd

    if not crumpet_amd._HAS_HIP_EXT:
        raise RuntimeError(f"crumpet_amd HIP extension missing: {crumpet_amd._native.load_error()}")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.profile:
        profile_run(dev)
        return

    p = bench_partition(args, dev)
    t_mask = bench_mask(args, dev)
    torch.cuda.empty_cache()
    a = {} if args.no_attention else bench_attention(args, dev)
    torch.cuda.empty_cache()
    aw = {} if args.no_attention else bench_attention_wide(args, dev)
    torch.cuda.empty_cache()
    blocks = {} if args.no_blocks else bench_blocks(args, dev)
    torch.cuda.empty_cache()
    fused = {} if args.no_fused_block else bench_fused_block(args, dev)
    torch.cuda.empty_cache()
    e2e = {} if args.no_e2e else bench_e2e(args, dev)
    torch.cuda.empty_cache()
    eager_refs = bench_eager_references(args, dev)

    gbs_step = 2 * C1_BYTES / (p["t_step"] * 1e-3) / 1e9
    gbs_part = C1_BYTES / (p["t_part"] * 1e-3) / 1e9
    gbs_unpart = C1_BYTES / (p["t_unpart"] * 1e-3) / 1e9
    gbs_mask = C2_BYTES / (t_mask * 1e-3) / 1e9
    components = {
        "partition": {"ms": round(p["t_part"], 5), "GB_s": round(gbs_part, 1),
                      "frac_hbm": round(gbs_part / HBM_PEAK_GBS, 4), "bytes": C1_BYTES,
                      "eager_rocm_ms": round(eager_refs["t_eager_part"], 4),
                      "speedup_vs_eager": round(eager_refs["t_eager_part"] / p["t_part"], 2)},
        "unpartition": {"ms": round(p["t_unpart"], 5), "GB_s": round(gbs_unpart, 1),
                        "frac_hbm": round(gbs_unpart / HBM_PEAK_GBS, 4), "bytes": C1_BYTES,
                        "eager_rocm_ms": round(eager_refs["t_eager_unpart"], 4),
                        "speedup_vs_eager": round(eager_refs["t_eager_unpart"] / p["t_unpart"], 2)},
        "mask": {"ms": round(t_mask, 5), "GB_s": round(gbs_mask, 1),
                 "frac_hbm": round(gbs_mask / HBM_PEAK_GBS, 4), "bytes": C2_BYTES,
                 "eager_rocm_ms": round(eager_refs["t_eager_mask"], 3),
                 "speedup_vs_eager": round(eager_refs["t_eager_mask"] / t_mask, 1),
                 "workload": "config 2: 98^3 fp16 ws7 ss3 -> [2744,343,343]"},
    }
    if a:
        tfl = C3_FLOPS / (a["t_attn"] * 1e-3) / 1e12
        comp = {"ms": round(a["t_attn"], 5), "TFLOP_s": round(tfl, 2),
                "frac_mfma_f16": round(tfl / MFMA_F16_PEAK_TFLOPS, 4),
                "GB_s": round(C3_BYTES / (a["t_attn"] * 1e-3) / 1e9, 1),
                "frac_hbm": round(C3_BYTES / (a["t_attn"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "flops": C3_FLOPS, "bytes": C3_BYTES, "max_abs_err_vs_fp32": a["max_abs_err"],
                "workload": "config 3: 1372 windows x 3 heads, N=343, hd16, fp16, shifted 49^3 mask"}
        if "t_eager" in a:
            comp["eager_rocm_ms"] = round(a["t_eager"], 4)
            comp["speedup_vs_eager"] = round(a["t_eager"] / a["t_attn"], 2)
        comp["mask_read"] = "tiled copy (kept by the wrapper from the second call with one mask)"
        comp["ms_row_major_mask"] = round(a["t_attn_row_major"], 5)
        comp["ms_mask_tiles_once"] = round(a["t_mask_tiles"], 5)
        comp["mask_1372_form"] = {
            "ms": round(a["t_attn_rep"], 5),
            "ms_with_repeat_and_flags": round(a["t_attn_rep_call"], 5),
            "frac_hbm": round(C3_BYTES / (a["t_attn_rep"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "same_output_as_343_form": a["rep_equals_343_form"],
            "workload": "the reference patch's layout (monai_patch.py:167-191): mask.repeat to "
                        "[1372,343,343] + abs().amax boundary flags; 'with_repeat_and_flags' times the "
                        "patch's per-call sequence"}
        components["attention"] = comp
        tfl_s = C3_FLOPS / (a["t_shift"] * 1e-3) / 1e12
        comp_s = {"ms": round(a["t_shift"], 5), "TFLOP_s": round(tfl_s, 2),
                  "frac_mfma_f16": round(tfl_s / MFMA_F16_PEAK_TFLOPS, 4),
                  "GB_s": round(C3_BYTES / (a["t_shift"] * 1e-3) / 1e9, 1),
                  "frac_hbm": round(C3_BYTES / (a["t_shift"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "max_abs_err_vs_fp32": a["max_abs_err_shifted"],
                  "workload": "config 3 through fused_swin_attention_shifted (mask from the 49^3 "
                              "geometry, never materialised)"}
        if "t_eager" in a:
            comp_s["speedup_vs_eager"] = round(a["t_eager"] / a["t_shift"], 2)
        components["attention_shifted"] = comp_s
    if aw:
        flops = 2 * C3_FLOPS  # head dim 32
        comp_w = {"workload": "head dim 32 (feature size 96) at the config-3 window shape: 1372 windows x "
                              "3 heads, N=343, fp16; the tuned kernel at head dim 32 (Q as a hi/lo pair "
                              "over two products per score tile; shifted: three strip groups of one head "
                              "per workgroup sharing double-buffered K/V; mask tensor with boundary flags: "
                              "4-wave workgroups, K/V single-buffered)",
                  "flops": flops, "max_abs_err_vs_fp32": aw["max_abs_err"]}
        for key, t in (("shifted", aw["t_shift"]), ("tensor_mask", aw["t_tensor"])):
            tfl = flops / (t * 1e-3) / 1e12
            comp_w[key] = {"ms": round(t, 5), "TFLOP_s": round(tfl, 2),
                           "frac_mfma_f16": round(tfl / MFMA_F16_PEAK_TFLOPS, 4)}
            if "t_eager" in aw:
                comp_w[key]["speedup_vs_eager"] = round(aw["t_eager"] / t, 2)
        if "t_eager" in aw:
            comp_w["eager_rocm_ms"] = round(aw["t_eager"], 4)
        components["attention_hd32"] = comp_w
    if blocks:
        components["block_path"] = blocks
    if fused:
        components["window_msa_block"] = fused
    if e2e:
        components["swin_unetr_e2e"] = e2e

    line = {
        "metric": "partition/unpartition GB/s (% HBM peak); window-attn TFLOP/s; ms per 96³ fwd",
        "value": round(gbs_step, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(p["t_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) fp16 volumes generated on the CPU",
        "config": {"workload": "config 1: shift-partition + unshift-unpartition round trip, "
                               "[1,98,98,98,48] fp16, window (7,7,7), shift (3,3,3)",
                   "bytes_per_step": 2 * C1_BYTES, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs_part, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs_part / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic("partition"),
                     "traffic_source": "profiles/window_gather_c1.md (rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                       "copy-calibrated)",
                     "kernel": "window_gather_kernel (shift-partition)",
                     "avg_launch_ms": round(p["t_part"], 5)},
        "components": components,
    }
    if not args.no_cpu:
        cpu = cpu_eager_paths(skip_e2e=args.no_e2e)
        rt = cpu["roundtrip"]
        line["cpu_baseline"] = {
            "value": rt["GB_s"], "unit": "GB/s", "cores": rt["threads"], "kind": "port",
            "sample": "the reference's eager CPU path for config 1 (torch-ext/crumpet/reference.py:141-184): "
                      "torch.roll + view/permute window partition and window reverse + roll back, fp16, "
                      f"full [1,98^3,48] volume, median of 3 round trips ({rt['ms']} ms), "
                      f"{rt['threads']} torch threads"}
        line["cpu_baseline_scalar_oracle"] = cpu_scalar_oracle()
        components["partition"]["cpu_eager_roundtrip"] = cpu["roundtrip"]
        components["mask"]["cpu_eager"] = cpu["mask"]
        if "attention" in components:
            components["attention"]["cpu_eager"] = cpu["attention"]
        if blocks:
            for name in ("s1", "s2", "s3"):
                blocks[f"cpu_eager_{name}"] = cpu[f"block_path_{name}"]
        if e2e and "swin_unetr_e2e" in cpu:
            e2e["cpu_eager"] = cpu["swin_unetr_e2e"]
    line["cpu_baseline_threads"] = {"os_cpu_count": os.cpu_count(),
                                    "torch_threads": torch.get_num_threads()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
