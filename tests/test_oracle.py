"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against something other than its own
formula: an independent numpy construction of the reference's tensor ops,
brute force, bijectivity/round trips, closed-form counts, hand-computed
entries, or a library routine (torch SDPA).  Shapes follow the reference
tests (tests/test_correctness.py:20-114, tests/test_dtype.py:13-25).
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

PART_CASES = [
    # (B, D, H, W, C, ws, ss)
    (2, 14, 14, 14, 13, (7, 7, 7), (3, 3, 3)),
    (2, 14, 14, 14, 48, (7, 7, 7), (0, 0, 0)),
    (2, 8, 8, 8, 7, (4, 4, 4), (2, 2, 2)),
    (1, 6, 4, 2, 3, (2, 2, 2), (1, 1, 1)),
    (1, 6, 8, 4, 5, (3, 4, 2), (2, 1, 1)),
    (2, 7, 7, 14, 4, (7, 7, 7), (3, 0, 5)),
]


def _rand(shape, dtype, seed=0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal(shape).astype(dtype)


def _brute_partition(x, ws, ss):
    """Element-by-element restatement straight from the roll definition
    roll(x, -s)[p] = x[(p + s) mod n] and the window index order."""
    B, D, H, W, C = x.shape
    nWd, nWh, nWw = D // ws[0], H // ws[1], W // ws[2]
    vol = ws[0] * ws[1] * ws[2]
    out = np.empty((B * nWd * nWh * nWw, vol, C), dtype=x.dtype)
    for b, wd, wh, ww in itertools.product(range(B), range(nWd), range(nWh), range(nWw)):
        win = (wd * nWh + wh) * nWw + ww
        for ld, lh, lw in itertools.product(range(ws[0]), range(ws[1]), range(ws[2])):
            loc = (ld * ws[1] + lh) * ws[2] + lw
            d = (wd * ws[0] + ld + ss[0]) % D
            h = (wh * ws[1] + lh + ss[1]) % H
            w = (ww * ws[2] + lw + ss[2]) % W
            out[b * nWd * nWh * nWw + win, loc] = x[b, d, h, w]
    return out


@pytest.mark.parametrize("case", PART_CASES)
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_partition_c_matches_numpy_roll_permute(oracle, case, dtype):
    B, D, H, W, C, ws, ss = case
    x = _rand((B, D, H, W, C), dtype)
    got = oracle.shift_partition(x, ws, ss)
    ref = oracle.np_shift_partition(x, ws, ss)
    assert got.tobytes() == ref.tobytes()


@pytest.mark.parametrize("case", PART_CASES[2:])
def test_partition_c_matches_brute_force(oracle, case):
    B, D, H, W, C, ws, ss = case
    x = _rand((B, D, H, W, C), np.float32, seed=1)
    assert np.array_equal(oracle.shift_partition(x, ws, ss), _brute_partition(x, ws, ss))


@pytest.mark.parametrize("case", PART_CASES)
def test_unpartition_c_matches_numpy_and_round_trips(oracle, case):
    B, D, H, W, C, ws, ss = case
    x = _rand((B, D, H, W, C), np.float32, seed=2)
    win = oracle.shift_partition(x, ws, ss)
    back = oracle.unshift_unpartition(win, B, D, H, W, C, ws, ss)
    assert back.tobytes() == x.tobytes()
    ref = oracle.np_unshift_unpartition(win, B, D, H, W, C, ws, ss)
    assert back.tobytes() == ref.tobytes()


def test_partition_is_a_bijection_at_14(oracle):
    # tests/test_correctness.py:100-114: every source token is used exactly once
    D = H = W = 14
    idx = np.arange(D * H * W, dtype=np.int64).reshape(1, D, H, W, 1)
    out = oracle.shift_partition(idx, (7, 7, 7), (3, 3, 3)).reshape(-1)
    assert np.array_equal(np.sort(out), np.arange(D * H * W))
    # first window token comes from (ss, ss, ss)
    assert out[0] == (3 * H + 3) * W + 3


def test_partition_byte_exact_for_every_element_size(oracle):
    for dt in (np.uint8, np.uint16, np.uint32, np.uint64):
        x = np.random.default_rng(3).integers(0, 250, (1, 8, 8, 8, 3)).astype(dt)
        assert np.array_equal(oracle.shift_partition(x, (4, 4, 4), (2, 1, 3)),
                              oracle.np_shift_partition(x, (4, 4, 4), (2, 1, 3)))


MASK_CASES = [
    ((14, 14, 14), (7, 7, 7), (3, 3, 3)),
    ((14, 14, 14), (7, 7, 7), (0, 0, 0)),
    ((8, 8, 8), (4, 4, 4), (2, 2, 2)),
    ((6, 4, 2), (2, 2, 2), (1, 1, 1)),
    ((21, 14, 7), (7, 7, 7), (3, 2, 1)),
    ((12, 8, 6), (4, 4, 3), (1, 0, 2)),
    ((49, 49, 49), (7, 7, 7), (3, 3, 3)),
]


@pytest.mark.parametrize("shape,ws,ss", MASK_CASES)
def test_mask_c_matches_both_eager_constructions(oracle, shape, ws, ss):
    got = oracle.attn_mask(*shape, ws, ss, "float32")
    where = np.where(oracle.np_mask_where(*shape, ws, ss), np.float32(-100), np.float32(0))
    assert got.tobytes() == where.tobytes()
    if any(ss):
        monai = oracle.np_mask_monai_slices(*shape, ws, ss)
        assert got.tobytes() == monai.tobytes()


@pytest.mark.parametrize("shape,ws,ss", MASK_CASES)
def test_mask_nonzero_count_closed_form(oracle, shape, ws, ss):
    """Per window, pairs with equal labels = prod over axes of sum(part^2),
    where an axis splits into parts (ws-ss, ss) only in its last window and
    only when ss > 0.  -100 count = vol^2 - that."""
    m = oracle.attn_mask(*shape, ws, ss, "float32")
    nWd, nWh, nWw = (n // w for n, w in zip(shape, ws))
    vol = ws[0] * ws[1] * ws[2]
    counts = (m != 0).reshape(m.shape[0], -1).sum(1)
    for win in range(m.shape[0]):
        wd, wh, ww = win // (nWh * nWw), (win // nWw) % nWh, win % nWw
        eq = 1
        for wi, nwi, w, s in zip((wd, wh, ww), (nWd, nWh, nWw), ws, ss):
            eq *= (w - s) ** 2 + s ** 2 if (wi == nwi - 1 and s > 0) else w * w
        assert counts[win] == vol * vol - eq


def test_mask_hand_checked_entries(oracle):
    m = oracle.attn_mask(14, 14, 14, (7, 7, 7), (3, 3, 3), "float32")
    assert m.shape == (8, 343, 343)
    assert set(np.unique(m)) <= {np.float32(0), np.float32(-100)}
    assert not m[0].any()  # window (0,0,0) is interior
    last = m[7]
    assert last[0, 342] == -100  # (0,0,0) lower on all axes vs (6,6,6) upper on all
    assert last[0, 3] == 0 and last[0, 4] == -100  # w split at ws - ss = 4
    assert last[0, 3 * 7] == 0 and last[0, 4 * 7] == -100  # h split
    assert last[0, 3 * 49] == 0 and last[0, 4 * 49] == -100  # d split
    for w in range(8):
        assert np.array_equal(m[w], m[w].T)
        assert not np.diag(m[w]).any()


def test_mask_bits_per_dtype(oracle):
    f16 = oracle.attn_mask_bits(8, 8, 8, (4, 4, 4), (2, 2, 2), "float16")
    bf16 = oracle.attn_mask_bits(8, 8, 8, (4, 4, 4), (2, 2, 2), "bfloat16")
    f32 = oracle.attn_mask_bits(8, 8, 8, (4, 4, 4), (2, 2, 2), "float32")
    assert np.float16(-100).view(np.uint16) == 0xD640
    assert np.float32(-100).view(np.uint32) >> 16 == 0xC2C8  # bf16 = high half of fp32
    assert set(np.unique(f16)) == {0, 0xD640}
    assert np.array_equal(bf16 == 0xC2C8, f32 == 0xC2C80000)
    assert np.array_equal(f16 == 0xD640, f32 == 0xC2C80000)


def test_relative_position_index(oracle):
    a = oracle.relative_position_index((7, 7, 7))
    b = oracle.relative_position_index_swin((7, 7, 7))
    assert np.array_equal(a, b)
    assert a.shape == (343, 343)
    assert np.all(np.diag(a) == 6 * 169 + 6 * 13 + 6)
    assert a[0, 342] == 0 and a[342, 0] == 13 ** 3 - 1
    assert a.min() == 0 and a.max() == 2196
    c = oracle.relative_position_index((3, 4, 2))
    assert np.array_equal(c, oracle.relative_position_index_swin((3, 4, 2)))


def test_get_window_size_rule(oracle):
    assert oracle.get_window_size((6, 6, 6), (7, 7, 7), (3, 3, 3)) == ((6, 6, 6), (0, 0, 0))
    assert oracle.get_window_size((49, 49, 49), (7, 7, 7), (3, 3, 3)) == ((7, 7, 7), (3, 3, 3))
    assert oracle.get_window_size((7, 14, 7), (7, 7, 7), (3, 3, 3)) == ((7, 7, 7), (0, 3, 0))


def _attn_inputs(B=6, H=3, N=27, D=16, M=None, seed=0):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, N, D)).astype(np.float32)
    k = rng.standard_normal((B, H, N, D)).astype(np.float32)
    v = rng.standard_normal((B, H, N, D)).astype(np.float32)
    bias = (0.02 * rng.standard_normal((H, N, N))).astype(np.float32)
    mask = None
    if M:
        mask = np.where(rng.random((M, N, N)) < 0.3, -100.0, 0.0).astype(np.float32)
    return q, k, v, bias, mask


def test_attention_matches_torch_sdpa(oracle):
    torch = pytest.importorskip("torch")
    q, k, v, bias, mask = _attn_inputs(M=3)
    bnd = np.array([1, 0, 1, 1, 0, 1], dtype=np.uint8)
    got = oracle.attention(q, k, v, bias, mask, bnd, scale=0.25, dtype=np.float64)
    madd = mask[np.arange(6) % 3] * bnd[:, None, None]
    am = torch.from_numpy(bias[None].astype(np.float64) + madd[:, None].astype(np.float64))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double(), torch.from_numpy(k).double(), torch.from_numpy(v).double(),
        attn_mask=am, scale=0.25,
    ).numpy()
    assert np.abs(got - ref).max() < 1e-12
    got32 = oracle.attention(q, k, v, bias, mask, bnd, scale=0.25)
    assert np.abs(got32 - ref).max() < 2e-6


def test_attention_invariants(oracle):
    q, k, v, bias, mask = _attn_inputs(M=6, seed=4)
    base = oracle.attention(q, k, v, bias, None, None, dtype=np.float64)
    # default scale is head_dim^-0.5
    assert np.allclose(base, oracle.attention(q, k, v, bias, None, None, scale=0.25, dtype=np.float64))
    # uniform shift of the bias leaves softmax unchanged
    assert np.allclose(base, oracle.attention(q, k, v, bias.astype(np.float64) + 3.5, None, None, dtype=np.float64), atol=1e-12)
    # a zero mask equals no mask; all-zero boundary flags skip the mask
    zero = np.zeros_like(mask)
    assert np.allclose(base, oracle.attention(q, k, v, bias, zero, None, dtype=np.float64), atol=1e-14)
    assert np.allclose(base, oracle.attention(q, k, v, bias, mask, np.zeros(6, np.uint8), dtype=np.float64), atol=1e-14)
    # constant values are reproduced exactly: rows of P sum to one
    ones = np.ones_like(v)
    assert np.allclose(oracle.attention(q, k, ones, bias, mask, None, dtype=np.float64), 1.0, atol=1e-12)
    # a dominant bias on one key selects that key's value
    sel = np.full_like(bias, -1e4)
    sel[:, :, 5] = 0.0
    out = oracle.attention(np.zeros_like(q), k, v, sel, None, None, dtype=np.float64)
    assert np.allclose(out, v[:, :, 5:6, :].repeat(q.shape[2], axis=2), atol=1e-12)


def test_gather_bias_layout(oracle):
    rng = np.random.default_rng(0)
    table = rng.standard_normal((13 ** 3, 3)).astype(np.float32)
    bias = oracle.gather_bias(table, (7, 7, 7))
    rpi = oracle.relative_position_index((7, 7, 7))
    assert bias.shape == (3, 343, 343)
    assert bias[2, 10, 200] == table[rpi[10, 200], 2]
    assert np.all(bias[1].diagonal() == table[1098, 1])


def test_reference_numerics_restatement(oracle):
    """attention_reference_numerics (the reference kernel's rounding steps):
    with fp32 inputs nothing rounds and the online recurrence is exact, so it
    equals the two-pass formula for any chunk size; one key gives v itself;
    and a two-key case fixes the rounding order by hand: the numerator uses P
    rounded to the input type, the row sum the unrounded P."""
    import torch

    g = torch.Generator().manual_seed(41)
    B, H, N, D = 3, 2, 37, 16
    q, k, v = (torch.randn((B, H, N, D), generator=g) for _ in range(3))
    bias = torch.randn((H, N, N), generator=g) * 0.1
    mask = torch.where(torch.rand((B, N, N), generator=g) > 0.8, -100.0, 0.0)
    want = oracle.attention(q.numpy(), k.numpy(), v.numpy(), bias.numpy(), mask.numpy(), None, scale=0.3,
                            dtype=np.float64)
    for block in (1, 5, 32, N):
        got = oracle.attention_reference_numerics(q, k, v, bias, mask, scale=0.3, block_n=block)
        assert np.abs(got.numpy() - want).max() < 2e-6

    for dt in (torch.float16, torch.bfloat16):
        one = torch.randn((1, 1, 1, 8), generator=g).to(dt)
        got = oracle.attention_reference_numerics(one, one, one, torch.zeros((1, 1, 1)), None, scale=1.0)
        assert torch.equal(got, one)

        # two keys with scores s0 = -1.1 and 0 (both queries alike): the row max
        # is 0, P = [exp(s0), 1]; exp(s0) is not representable in the input
        # type, and v = identity makes the output [round(exp(s0)), 1] / (exp(s0) + 1)
        s0 = -1.1
        qq = torch.tensor([[[[1.0, 0.0], [1.0, 0.0]]]]).to(dt)
        kk = torch.tensor([[[[s0, 0.0], [0.0, 0.0]]]]).to(dt)
        vv = torch.tensor([[[[1.0, 0.0], [0.0, 1.0]]]]).to(dt)
        got = oracle.attention_reference_numerics(qq, kk, vv, torch.zeros((1, 2, 2)), None, scale=1.0)
        s0r = float(torch.tensor(s0).to(dt))  # k is stored in dt
        p0 = np.exp(np.float32(s0r))  # row max is the score 0 of key 1
        num = float(torch.tensor(p0).to(dt))
        exp0 = torch.tensor(num / (p0 + 1.0), dtype=torch.float32).to(dt)
        exp1 = torch.tensor(1.0 / (p0 + 1.0), dtype=torch.float32).to(dt)
        assert torch.equal(got[0, 0, 0], torch.stack([exp0, exp1]))
        assert torch.equal(got[0, 0, 1], got[0, 0, 0])
        # rounding P only in the row sum as well would give a different first element
        alt = torch.tensor(num / (num + 1.0), dtype=torch.float32).to(dt)
        assert float(torch.tensor(p0).to(dt)) != p0 and (alt != exp0 or dt == torch.bfloat16)
