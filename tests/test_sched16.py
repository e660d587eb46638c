"""The code-pair schedules of the f16 prefill GEMM (jangq_amd/csrc/jq_sched16.h), checked on
the CPU against what the kernel does with them: every pair of a 32-code unit cut from one
32-bit window by one and-or lands both codes where the mask says; the 16 pairs cover the
unit's 32 codes once; each half reads 1024 + q 2^p as an f16 and the two fused multiply-adds
of the kernel (constants 2^-p and -1024 2^-p, then s' and b') give f16(s' q + b') with a
single rounding, emulated here with numpy's float16 on exact float64 products."""
import re
from pathlib import Path

import numpy as np
import pytest

HDR = Path(__file__).resolve().parents[1] / "jangq_amd" / "csrc" / "jq_sched16.h"


def _tables():
    text = HDR.read_text()
    out = {}
    for bits, body in re.findall(r"kSched16_(\d) = \{(.*?)\};", text, re.S):
        rows = [list(map(int, r.split(","))) for r in re.findall(r"\{([\d,\s]+)\}", body)]
        assert len(rows) == 5 and all(len(r) == 16 for r in rows)
        out[int(bits)] = rows
    return out


def _f16_of_bits(h):
    return np.array([h], dtype=np.uint16).view(np.float16)[0]


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6])
def test_schedule_extracts_every_code(bits):
    s, a, b, pa, pb = _tables()[bits]
    assert sorted(a + b) == list(range(32))
    rng = np.random.default_rng(bits)
    m = (1 << bits) - 1
    for _ in range(50):
        codes = rng.integers(0, 1 << bits, 32)
        unit = 0
        for i, c in enumerate(codes):
            unit |= int(c) << (bits * i)
        for p in range(16):
            assert 0 <= pa[p] and pa[p] + bits <= 10 and 0 <= pb[p] and pb[p] + bits <= 10
            assert 0 <= s[p] < 32 * bits
            win = (unit >> s[p]) & 0xFFFFFFFF
            mask = (m << pa[p]) | (m << (16 + pb[p]))
            v = (win & mask) | 0x64006400
            lo, hi = v & 0xFFFF, v >> 16
            assert _f16_of_bits(lo) == 1024 + int(codes[a[p]]) * 2 ** pa[p]
            assert _f16_of_bits(hi) == 1024 + int(codes[b[p]]) * 2 ** pb[p]


def test_dequant_arithmetic_single_rounding():
    """(1024 + q 2^p) 2^-p - 1024 2^-p = q exactly, then fma(s', q, b') rounded once to f16."""
    rng = np.random.default_rng(7)
    for _ in range(2000):
        p = int(rng.integers(0, 7))
        q = int(rng.integers(0, 1 << (10 - p)))
        v = np.float16(1024 + q * 2 ** p)
        qn = float(v) * 2.0 ** -p - 1024 * 2.0 ** -p  # exact in float64: the fma's exact result
        assert np.float16(qn) == q
        s = np.float16(rng.uniform(-4, 4))
        bb = np.float16(rng.uniform(-64, 64))
        w = np.float16(float(s) * q + float(bb))  # one rounding of the exact value
        assert abs(float(w) - (float(s) * q + float(bb))) <= abs(float(w)) * 2 ** -11 + 2 ** -25
