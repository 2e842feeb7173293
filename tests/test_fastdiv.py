"""The kernels' magic-number divider (crumpet_amd/csrc/crumpet_common.h,
Granlund & Montgomery 1994) compiled for the host with g++ and checked
against hardware division over edge cases and random numerators."""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

PROGRAM = r"""
#include <cstdio>
#include <cstdint>
#include <random>
#include "crumpet_common.h"
int main() {
    std::mt19937_64 rng(12345);
    const uint32_t divisors[] = {1u, 2u, 3u, 5u, 6u, 7u, 13u, 14u, 49u, 98u, 343u, 2744u, 117649u,
                                 941192u, 1000003u, (1u << 20) + 1u, (1u << 30) - 1u, 1u << 30,
                                 (1u << 30) + 1u, 0x7fffffffu};
    long checked = 0;
    for (uint32_t d : divisors) {
        crumpet::FastDiv f(d);
        uint32_t edge[] = {0u, 1u, d - 1u, d, d + 1u, 2u * d - 1u, 0x7fffffffu, 0x7ffffffeu,
                           0x7fffffffu / d * d, 0x7fffffffu / d * d - 1u};
        for (uint32_t n : edge) {
            if (n > 0x7fffffffu) continue;
            uint32_t q, r; f.divmod(n, q, r);
            if (q != n / d || r != n % d) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
            ++checked;
        }
        for (int i = 0; i < 200000; ++i) {
            uint32_t n = static_cast<uint32_t>(rng() & 0x7fffffffu);
            if (f.div(n) != n / d) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
            ++checked;
        }
    }
    for (uint32_t d = 1; d < 5000; ++d) {  // every small divisor, every numerator below 20000
        crumpet::FastDiv f(d);
        for (uint32_t n = 0; n < 20000; ++n)
            if (f.div(n) != n / d) { printf("FAIL d=%u n=%u\n", d, n); return 1; }
        checked += 20000;
    }
    printf("OK %ld\n", checked);
    return 0;
}
"""


def test_fastdiv_matches_division(tmp_path):
    src = tmp_path / "fastdiv.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "fastdiv"
    subprocess.check_call(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'crumpet_amd' / 'csrc'}",
                           str(src), "-o", str(exe)])
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout
    assert out.stdout.startswith("OK")
