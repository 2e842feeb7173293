"""``__graft_entry__.build()`` on a checkout with no built libraries.

The build must compile everything and then load what it just compiled, in a
single call (the reference's loader likewise builds on first import,
torch-ext/crumpet/_jit_ops.py:27-43).  The sources are copied to a scratch
tree without any ``.so`` files and ``build()`` runs there in a child
process, so the libraries already mapped by this test session play no part.
"""

from __future__ import annotations

import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

_SKIP = shutil.ignore_patterns("*.so", "*.so.tmp", "_build", "__pycache__", "*.o")


def test_build_from_a_clean_tree(tmp_path):
    for sub in ("crumpet_amd", "include", "oracle"):
        shutil.copytree(ROOT / sub, tmp_path / sub, ignore=_SKIP)
    shutil.copy2(ROOT / "__graft_entry__.py", tmp_path / "__graft_entry__.py")
    assert not list(tmp_path.rglob("*.so"))

    proc = subprocess.run(
        [sys.executable, "-c", "import __graft_entry__ as g; g.build(); print('BUILD-OK')"],
        cwd=str(tmp_path), stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
        timeout=900,
    )
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert "BUILD-OK" in proc.stdout
    for lib in ("crumpet_amd/libcrumpet_hip.so", "crumpet_amd/_crumpet_ops.so", "oracle/liboracle.so"):
        assert (tmp_path / lib).is_file(), lib

    # the libraries a fresh process maps are the scratch tree's own
    probe = (
        "import crumpet_amd, crumpet_amd._native as n; "
        "print(n.HIP_LIB); assert crumpet_amd._HAS_HIP_EXT"
    )
    proc = subprocess.run([sys.executable, "-c", probe], cwd=str(tmp_path),
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert str(tmp_path) in proc.stdout
