"""Floating-point identities the HIP kernels rely on, checked on the host.

- Markstein division: the RMSNorm paths (GEMV prologue, QK-norm) compute x / rms as
  q = RN(x*y), r = fma(-q, rms, x), RN(q + r*y) with y = RN(1/rms). This must equal IEEE
  x / rms for every finite fp16 x; it is checked here in C (fmaf is correctly rounded)
  over all finite fp16 numerators and a spread of divisors, including significands of
  all ones and powers of two. Signed zeros may differ; the kernels add +0.0 afterwards.
- Nibble magics of the W4G dequant: half(0x6400 | n) - 1032 and half(0x5400 | n << 4)
  - 72 are both n - 8 exactly for every nibble n.
"""
from __future__ import annotations

import shutil
import subprocess

import numpy as np
import pytest

_C = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float h2f(uint16_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023; float v;
    if (e == 0) v = ldexpf((float)m, -24); else v = ldexpf((float)(m | 1024), (int)e - 25);
    return s ? -v : v;
}
static uint32_t st = 12345u;
static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 17; st ^= st << 5; return st; }
int main(void) {
    long bad = 0, tot = 0;
    for (int t = 0; t < 1500; ++t) {
        float b;
        if (t < 500) { uint32_t bits = ((rnd() % 154u + 100u) << 23) | (rnd() & 0x7FFFFFu); memcpy(&b, &bits, 4); }
        else if (t < 800) { uint32_t bits = ((uint32_t)(118 + t % 20) << 23) | 0x7FFFFFu; memcpy(&b, &bits, 4); }
        else if (t < 1000) b = ldexpf(1.0f, t % 40 - 20);
        else b = sqrtf(ldexpf((float)(rnd() % 100000u + 1u), -(int)(rnd() % 30u)));
        const float y = 1.0f / b;
        for (uint32_t h = 0; h < 65536u; ++h) {
            if (((h >> 10) & 31u) == 31u) continue;
            const float a = h2f((uint16_t)h), ref = a / b;
            const float q = a * y;
            const float r = fmaf(-q, b, a);
            const float q1 = fmaf(r, y, q);
            ++tot;
            if (memcmp(&q1, &ref, 4) != 0 && !(q1 == 0.0f && ref == 0.0f)) ++bad;
        }
    }
    printf("%ld %ld\n", tot, bad);
    return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_division_matches_ieee(tmp_path):
    src = tmp_path / "mk.c"
    exe = tmp_path / "mk"
    src.write_text(_C)
    # -ffp-contract=off: the a * y and a / b above must be the plain rounded operations
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(src), "-o", str(exe), "-lm"], check=True)
    tot, bad = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    assert tot == 1500 * 63488
    assert bad == 0


def test_nibble_magics_are_exact():
    n = np.arange(16, dtype=np.uint16)
    lo = (np.uint16(0x6400) | n).view(np.float16)
    hi = (np.uint16(0x5400) | (n << 4)).view(np.float16)
    assert np.array_equal((lo - np.float16(1032)).astype(np.int32), n.astype(np.int32) - 8)
    assert np.array_equal((hi - np.float16(72)).astype(np.int32), n.astype(np.int32) - 8)
    # pair placement: bits 0-3 and 4-7 of each 16-bit half land in the right element
    w = np.array([0x76543210], dtype=np.uint32)
    lo_pair = ((w & 0x000F000F) | 0x64006400).view(np.float16) - np.float16(1032)
    hi_pair = ((w & 0x00F000F0) | 0x54005400).view(np.float16) - np.float16(72)
    assert lo_pair.tolist() == [0 - 8, 4 - 8] and hi_pair.tolist() == [1 - 8, 5 - 8]
