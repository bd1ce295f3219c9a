"""Pins for the oracle's MXFP8 E4M3 activation functions (the reference has
no FP8 activation format; these define the extension, hb_oracle.c):

  * the decode of all 256 codes against the OCP E4M3 formula in exact
    rationals;
  * the element encoder against brute force over the E4M3 grid (nearest,
    ties to the even mantissa, saturation at 448), on random values and on
    every midpoint between neighbouring codes;
  * the block encoder's exponent rule (floor(log2 max) - 8, clamped);
  * the block value against exact rational arithmetic rounded to 24 bits at
    its own binade (below the normal range -> +0, overflow -> inf);
  * a layer whose FP8 and MXINT8 operands hold the same exact values gives
    the same bits through both folds (the MXINT8 fold is pinned against the
    compiled reference), and a small layer against a Python fold.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import helpers
import oracle


def e4m3_value(code: int) -> Fraction:
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    v = Fraction(m, 8) * Fraction(1, 64) if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
    return -v if s else v


FINITE = [c for c in range(0x7F)]  # 0x00 .. 0x7E: every finite magnitude, 0 to 448


def test_decode_all_codes():
    for c in range(256):
        assert Fraction(oracle.fp8_int(c), 512) == e4m3_value(c), hex(c)


def brute_encode(v: Fraction) -> int:
    mag = abs(v)
    if mag >= 448:
        best = 0x7E
    else:
        best = min(FINITE, key=lambda c: (abs(e4m3_value(c) - mag), c & 1))
    if best == 0:
        return 0
    return best | (0x80 if v < 0 else 0)


def f32_fraction(bits: int) -> Fraction:
    x = np.array([bits], np.uint32).view(np.float32)[0]
    return Fraction(float(x))


def test_element_encoder_random():
    rng = np.random.default_rng(81)
    for _ in range(3000):
        x = int(rng.integers(-140, 140))
        v = np.float32(np.ldexp(rng.standard_normal(), int(rng.integers(-12, 12)) + x))
        if not np.isfinite(v) or v == 0:
            continue
        bits = int(np.array([v], np.float32).view(np.uint32)[0])
        want = brute_encode(f32_fraction(bits) / Fraction(2) ** x)
        assert oracle.quantize_fp8(bits, x) == want, (float(v), x)


def test_element_encoder_midpoints_and_edges():
    vals = sorted({e4m3_value(c) for c in FINITE})
    cases = []
    for lo, hi in zip(vals, vals[1:]):
        cases += [lo, hi, (lo + hi) / 2]
    cases += [Fraction(464), Fraction(470), Fraction(1000), Fraction(1, 1024), Fraction(3, 2048)]
    for v in cases:
        for sign in (1, -1):
            y = float(sign * v)
            bits = int(np.array([y], np.float32).view(np.uint32)[0])
            assert Fraction(float(np.float32(y))) == sign * v  # exact in fp32
            assert oracle.quantize_fp8(bits, 0) == brute_encode(sign * v), float(sign * v)


def test_block_exponent_rule():
    rng = np.random.default_rng(82)
    x = (rng.standard_normal((6, 64)) * 2.0 ** rng.integers(-20, 20, (6, 1))).astype(np.float32)
    x[1, :32] = 0.0
    x[2, :32] = np.float32(1e-42)  # subnormal: clamped to -127
    q, e = oracle.encode_mxfp8(x.view(np.uint32))
    for r in range(6):
        for b in range(2):
            blk = x[r, 32 * b:32 * b + 32]
            amax = float(np.abs(blk).max())
            if amax == 0:
                want = 0
            else:
                field = int(np.array([np.float32(amax)]).view(np.uint32)[0] >> 23) & 0xFF
                want = max(-127, min(127, field - 127 - 8))
            assert e[r, b] == want
            for k in range(32):
                bits = int(blk[k:k + 1].view(np.uint32)[0])
                assert q[r, 32 * b + k] == oracle.quantize_fp8(bits, want)


def round24(v: Fraction) -> int:
    """Fraction -> fp32 bits: 24 significant bits at the value's own binade,
    ties to even, below 2^-126 -> +0, 2^128 and above -> inf."""
    if v == 0:
        return 0
    sign = 1 if v < 0 else 0
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = Fraction(2) ** (e - 23)
    n, rem = divmod(a / q, 1)
    n = int(n)
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n & 1):
        n += 1
    r = n * q
    if r < Fraction(2) ** -126:
        return 0
    if r >= Fraction(2) ** 128:
        return (sign << 31) | 0x7F800000
    bits = int(np.array([np.float32(float(r))]).view(np.uint32)[0])
    return (sign << 31) | bits


def test_block_value_against_exact_rationals():
    rng = np.random.default_rng(83)
    cases = [(1, 127, 127), (-1, 127, 127), ((1 << 24) + 1, 130, 120), ((1 << 25) + 3, 100, 90),
             ((1 << 27) - 1, 200, 200), (88080384, 254, 254), (-88080384, 0, 0), (3, 1, 1),
             ((1 << 24) - 1, 68, 69), (12345677, 70, 70)]
    for _ in range(4000):
        s = int(rng.integers(-88080384, 88080385))
        cases.append((s, int(rng.integers(0, 255)), int(rng.integers(0, 255))))
    for s, ea, ew in cases:
        want = 0 if s == 0 else round24(Fraction(s) * Fraction(2) ** (ea + ew - 264))
        assert oracle.block_value_fp8(s, ea, ew) == want, (s, ea, ew)


def test_fp8_and_mxint8_folds_agree_on_shared_values():
    """A in [-16, 16] (integers, exact in both formats): MXINT8 q at scale
    byte s, FP8 code of q at scale byte s - 6; every block value is exact in
    both, so the two folds give the same bits."""
    rng = np.random.default_rng(84)
    m, n, kb = 8, 16, 5
    q = rng.integers(-16, 17, (m, kb * 32)).astype(np.int8)
    s8 = rng.integers(118, 130, (m, kb)).astype(np.int32) - 127
    a8 = oracle.pack_abuf(q, s8)
    codes = np.zeros((m, kb * 32), np.uint8)
    for v in range(-16, 17):
        bits = int(np.array([np.float32(v)]).view(np.uint32)[0])
        codes[q == v] = oracle.quantize_fp8(bits, 0)
    af = oracle.pack_abuf(codes.view(np.int8), s8 - 6)
    code, e = helpers.mxfp4_weights(rng, n, kb * 32)
    w = oracle.pack_wbuf(code, e)
    c8, _ = oracle.linear(m, n, kb, a8, [w], [0])
    cf, _ = oracle.linear(m, n, kb, af, [w], [0], a_fp8=True)
    assert np.array_equal(c8, cf)


def test_small_layer_against_python_fold():
    rng = np.random.default_rng(85)
    m, n, kb = 4, 8, 3
    x = (rng.standard_normal((m, kb * 32)) * 4).astype(np.float32)
    codes, e = oracle.encode_mxfp8(x.view(np.uint32))
    a = oracle.pack_abuf(codes.view(np.int8), e)
    wc, we = helpers.mxfp4_weights(rng, n, kb * 32)
    w = oracle.pack_wbuf(wc, we)
    got, _ = oracle.linear(m, n, kb, a, [w], [0], a_fp8=True)
    mag = [0, 1, 2, 3, 4, 6, 8, 12]
    for r in range(m):
        for col in range(n):
            acc = 0
            for b in range(kb):
                s = 0
                for k in range(32):
                    c = int(wc[col, 32 * b + k])
                    wv = (-1 if c & 8 else 1) * mag[c & 7]
                    s += oracle.fp8_int(int(codes[r, 32 * b + k])) * wv
                bv = round24(Fraction(s) * Fraction(2) ** (int(e[r, b]) + 127 + int(we[col, b]) + 127 - 264)) if s else 0
                acc = int(oracle.fp32_add_n(np.array([acc], np.uint32),
                                            np.array([bv], np.uint32))[0])
            assert got[r, col] == acc, (r, col)


def test_rejects_infinity():
    x = np.zeros((1, 32), np.float32)
    x[0, 3] = np.inf
    with pytest.raises(ValueError, match="infinite"):
        oracle.encode_mxfp8(x.view(np.uint32))
