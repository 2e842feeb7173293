"""In-tree build of the native libraries.

* ``libcrumpet_hip.so``: the gfx950 HIP kernels and their C ABI
  (include/crumpet_hip.h), compiled by hipcc, one object per source.
* ``_crumpet_ops.so``: the torch dispatcher binding (csrc/torch_binding.cpp),
  compiled by g++ against the torch headers and linked to libcrumpet_hip.so
  through an ``$ORIGIN`` rpath.

Both land next to this file so that they travel with the source tree.  The
HIP library records NEEDED ``libamdhip64.so.7``; once torch is imported the
dynamic loader binds that to torch's already-loaded HIP runtime (same
soname), so the process keeps a single HIP runtime.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = PKG / "_build"
HIP_LIB = PKG / "libcrumpet_hip.so"
OPS_LIB = PKG / "_crumpet_ops.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

HIP_SOURCES = [
    "api.hip", "partition.hip", "attn_mask.hip", "mask_tile.hip", "attention.hip",
    "attention_f16.hip", "attention_bf16.hip", "attention_f32.hip", "attention_d32.hip", "attention_wide.hip",
    "window_linear.hip",
]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # packed fp32 VALU ops stay disabled on these boxes
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    # dma16() (attention_kernel.h) sets m0 in inline asm on purpose
    "-Wno-inline-asm",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = proc.stdout
    # hipcc's host pass does not know the packed-fp32 feature; that warning is harmless
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + "\n".join(lines))
    if verbose and lines:
        print("\n".join(lines), flush=True)


def _torch_paths():
    import torch

    tdir = Path(torch.__file__).resolve().parent
    return tdir / "include", tdir / "lib"


def build_hip(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    flags = HIPCC_FLAGS + list(extra_flags or [])
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (src.rsplit(".", 1)[0] + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *flags, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 4)) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run(
        [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
         f"-Wl,-rpath,{ROCM / 'lib'}"],
        verbose,
    )
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_binding(verbose: bool = False) -> Path:
    tinc, tlib = _torch_paths()
    tmp = OPS_LIB.with_suffix(".so.tmp")
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM",
        f"-I{tinc}", f"-I{tinc / 'torch' / 'csrc' / 'api' / 'include'}",
        f"-I{ROCM / 'include'}", f"-I{INCLUDE}",
        str(CSRC / "torch_binding.cpp"),
        "-o", str(tmp),
        f"-L{PKG}", "-lcrumpet_hip",
        f"-L{tlib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}",
    ]
    _run(cmd, verbose)
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


def build(verbose: bool = False) -> None:
    """Compile both native libraries (always recompiles)."""
    build_hip(verbose)
    build_binding(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {HIP_LIB.name} and {OPS_LIB.name}")
