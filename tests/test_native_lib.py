"""CPU checks of the native boundary: the C-ABI library loads and exports
every symbol include/crumpet_hip.h declares, the torch binding registers the
crumpet_ops schemas, and the host-side argument checks of the C ABI return
their error codes without touching a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import torch

from helpers import c_abi

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "crumpet_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(crumpet_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    from crumpet_amd import _native

    declared = _declared_symbols()
    assert len(declared) >= 10
    lib = ctypes.CDLL(str(_native.HIP_LIB))
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.C_ABI_SYMBOLS)


def test_library_exports_only_the_c_abi():
    """Internal C++ symbols and kernel stubs are hidden, so another library in
    the process can neither interpose on them nor be interposed."""
    import subprocess

    from crumpet_amd import _native

    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.HIP_LIB)],
                         capture_output=True, text=True, check=True).stdout
    names = {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    ours = {n for n in names if not n.startswith(("_", "hip", "__"))}
    assert ours == set(_declared_symbols())
    assert not any("crumpet" in n for n in names - ours)


def test_version_and_status_strings():
    lib = c_abi()
    assert lib.crumpet_version() == b"0.1.0"
    assert lib.crumpet_status_string(0) == b"CRUMPET_OK"
    assert lib.crumpet_status_string(1) == b"CRUMPET_ERR_INVALID_ARGUMENT"
    assert lib.crumpet_status_string(2) == b"CRUMPET_ERR_UNSUPPORTED"
    assert lib.crumpet_status_string(3) == b"CRUMPET_ERR_HIP"


def test_host_argument_checks_need_no_gpu():
    """Invalid arguments are rejected before any HIP call."""
    lib = c_abi()
    fake = ctypes.c_void_p(16)
    st = lib.crumpet_shift_partition_3d(fake, fake, 1, 15, 14, 14, 4, 2, 7, 7, 7, 3, 3, 3, None)
    assert st == 1 and b"divisible" in lib.crumpet_last_error()
    st = lib.crumpet_unshift_unpartition_3d(fake, fake, 1, 14, 14, 14, 4, 2, 7, 7, 7, 7, 0, 0, None)
    assert st == 1 and b"shift" in lib.crumpet_last_error()
    st = lib.crumpet_shift_partition_3d(fake, fake, 1, 14, 14, 14, 4, 3, 7, 7, 7, 3, 3, 3, None)
    assert st == 1 and b"elem_size" in lib.crumpet_last_error()
    st = lib.crumpet_compute_attn_mask_3d(fake, 1, 11, 11, 11, 11, 11, 11, 5, 5, 5, None)
    assert st == 2 and b"1024" in lib.crumpet_last_error()
    st = lib.crumpet_compute_attn_mask_3d(fake, 7, 14, 14, 14, 7, 7, 7, 3, 3, 3, None)
    assert st == 1
    # zero-size work is a successful no-op
    assert lib.crumpet_shift_partition_3d(None, None, 0, 14, 14, 14, 4, 2, 7, 7, 7, 3, 3, 3, None) == 0


def test_attention_argument_checks_need_no_gpu():
    lib = c_abi()
    s4 = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    s3 = (ctypes.c_int64 * 3)(1, 1, 1)
    fake = ctypes.c_void_p(256)

    def call(dtype=1, B=2, H=3, N=343, Dh=16, mask=None, mb=1):
        rows = (ctypes.c_int64 * 3)(N * N, N, 1)
        return lib.crumpet_fused_swin_attention(
            fake, s4, fake, s4, fake, s4, fake, s4, dtype, B, H, N, Dh, fake, 1, rows,
            mask, 1, mb, rows, None, ctypes.c_float(0.25), None)

    assert call(Dh=8) == 2
    assert call(Dh=24) == 2 and b"head_dim 24" in lib.crumpet_last_error()
    assert call(dtype=5) == 1
    assert call(mask=fake, mb=3) == 1  # mask batch must divide B
    assert call(B=0) == 0
    # bias and mask rows are read with multi-element loads: overlapping rows
    # (row stride below N) are rejected; the torch op makes them contiguous
    s3_rows = (ctypes.c_int64 * 3)(343 * 343, 343, 1)
    st = lib.crumpet_fused_swin_attention(fake, s4, fake, s4, fake, s4, fake, s4, 1, 2, 3, 343, 16, fake, 1,
                                          s3, None, 1, 1, s3, None, ctypes.c_float(0.25), None)
    assert st == 1 and b"bias rows must not overlap" in lib.crumpet_last_error()
    st = lib.crumpet_fused_swin_attention(fake, s4, fake, s4, fake, s4, fake, s4, 1, 2, 3, 343, 16, fake, 1,
                                          s3_rows, fake, 1, 1, s3, None, ctypes.c_float(0.25), None)
    assert st == 1 and b"mask rows must not overlap" in lib.crumpet_last_error()

    def shifted(B=8, N=343, D=14, ws=7, ss=3):
        bias_s = (ctypes.c_int64 * 3)(N * N, N, 1)
        return lib.crumpet_fused_swin_attention_shifted(
            fake, s4, fake, s4, fake, s4, fake, s4, 1, B, 3, N, 16, fake, 1, bias_s,
            D, D, D, ws, ws, ws, ss, ss, ss, ctypes.c_float(0.25), None)

    assert shifted(D=15) == 1 and b"divisible" in lib.crumpet_last_error()
    assert shifted(ss=7) == 1 and b"shift" in lib.crumpet_last_error()
    assert shifted(N=216) == 1 and b"window volume" in lib.crumpet_last_error()
    assert shifted(B=6) == 1 and b"multiple" in lib.crumpet_last_error()
    # the general kernel's region mode holds one class byte per token in LDS
    assert shifted(N=13 ** 3, D=26, ws=13) == 2 and b"exceed" in lib.crumpet_last_error()


def test_window_projection_argument_checks_need_no_gpu():
    lib = c_abi()
    fake = ctypes.c_void_p(256)
    eps = ctypes.c_float(1e-5)

    def qkv(C=48, n_out=144, ws=7, ss=3, x_dtype=0, dtype=1, ln=None, ln_dtype=0, out=fake, B=1):
        return lib.crumpet_window_qkv_3d(out, dtype, fake, x_dtype, B, 12, 12, 12, C, 1, ln, ln, ln_dtype, eps,
                                         fake, None, n_out, ws, ws, ws, ss, ss, ss, None)

    assert qkv(C=24) == 2 and b"multiple of 16" in lib.crumpet_last_error()
    assert qkv(n_out=40) == 2 and b"output features" in lib.crumpet_last_error()
    assert qkv(C=400) == 2
    assert qkv(ss=7) == 1 and b"shift_size" in lib.crumpet_last_error()
    assert qkv(dtype=9) == 1
    assert qkv(x_dtype=9) == 1
    assert qkv(ln=fake, ln_dtype=2, x_dtype=1) == 1 and b"LayerNorm" in lib.crumpet_last_error()
    assert qkv(out=ctypes.c_void_p(8)) == 2 and b"aligned" in lib.crumpet_last_error()
    assert qkv(dtype=0, C=384, n_out=384) == 2 and b"staging tile" in lib.crumpet_last_error()
    assert qkv(B=0) == 0  # no tokens: a successful no-op

    def proj(C=48, n_out=48, ws=7, ss=3):
        return lib.crumpet_window_proj_3d(fake, fake, 1, 1, 12, 12, 12, C, fake, None, n_out,
                                          ws, ws, ws, ss, ss, ss, None)

    assert proj(C=40) == 2
    assert proj(n_out=8) == 2
    assert proj(ws=0) == 1 and b"window_size" in lib.crumpet_last_error()


def test_fused_block_support_check_matches_the_tile_plan():
    """monai_patch only routes a block to the fused projections when their
    LDS tile plan accepts its width: the Python check agrees with the C ABI
    for every C, in both directions (B = 0 plans the tile and launches
    nothing)."""
    from crumpet_amd.monai_patch import _fits_staging_tile

    lib = c_abi()
    fake = ctypes.c_void_p(256)
    for dtype, esize in ((0, 4), (1, 2), (2, 2)):
        for C in range(16, 385, 16):
            rc_q = lib.crumpet_window_qkv_3d(fake, dtype, fake, dtype, 0, 12, 12, 12, C, 1, None, None, 0,
                                             ctypes.c_float(1e-5), fake, None, 3 * C, 7, 7, 7, 3, 3, 3, None)
            rc_p = lib.crumpet_window_proj_3d(fake, fake, dtype, 0, 12, 12, 12, C, fake, None, C,
                                              7, 7, 7, 3, 3, 3, None)
            assert (rc_q == 0) == _fits_staging_tile(C, esize) == (rc_p == 0), (dtype, C, rc_q, rc_p)


def test_dispatcher_schemas_match_reference():
    import crumpet_amd  # noqa: F401  (loads the binding)

    ops = torch.ops.crumpet_ops
    expect = {
        "compute_attn_mask_3d": "(Tensor(a0!) output, int D, int H, int W, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        "fused_shift_partition_3d": "(Tensor(a0!) output, Tensor x, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        "fused_shift_partition_3d_backward": "(Tensor(a0!) grad_x, Tensor grad_windows, int B, int D, int H, int W, int C, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        "fused_unshift_unpartition_3d": "(Tensor(a0!) output, Tensor windows, int B, int D, int H, int W, int C, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
        "fused_unshift_unpartition_3d_backward": "(Tensor(a0!) grad_windows, Tensor grad_x, int ws_d, int ws_h, int ws_w, int ss_d, int ss_h, int ss_w) -> ()",
    }
    for name, sig in expect.items():
        schema = str(getattr(ops, name).default._schema)
        norm = re.sub(r"\(\$?a?\d+! -> \)", "(a0!)", schema)
        norm = re.sub(r"Tensor\([^)]*!\)", "Tensor(a0!)", norm)
        assert norm == f"crumpet_ops::{name}{sig}", schema
        assert torch.Tag.pt2_compliant_tag in getattr(ops, name).default.tags
        assert torch.Tag.needs_fixed_stride_order in getattr(ops, name).default.tags


def test_mask_tiles_element_count():
    """crumpet_attn_mask_tiles_elements: M x ceil(N / 16) strips x the tuned
    kernel's tile count (made even: the layout is in tile pairs) x 256 (64
    lanes x 4 keys), -1 outside 1 <= N <= 512 (host arithmetic only)."""
    from crumpet_amd import _native

    f = ctypes.CDLL(str(_native.HIP_LIB)).crumpet_attn_mask_tiles_elements
    f.restype = ctypes.c_int64
    f.argtypes = [ctypes.c_int64, ctypes.c_int64]
    for N, strips, tiles in ((1, 1, 2), (16, 1, 2), (17, 2, 2), (129, 9, 14), (224, 14, 14), (225, 15, 22),
                             (343, 22, 22), (352, 22, 22), (353, 23, 32), (512, 32, 32)):
        assert f(3, N) == 3 * strips * tiles * 256, N
    assert f(0, 343) == 0
    assert f(1, 0) == -1 and f(1, 513) == -1 and f(-1, 343) == -1
