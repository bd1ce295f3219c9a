"""The oracle's operand formats (formats.cpp, tensors.cpp, weights.cpp), VEC
lane arithmetic (lane.cpp) and VEC passes (vec_engine.cpp, vec_rom.cpp)
against the reference tests' known answers and closed forms."""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np
import pytest

import helpers
import oracle
from test_oracle_fp32 import round_binary32, value

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def known():
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        return json.load(f)


def test_encode_mxint8_known_answers(olib):
    k = known()["encode_mxint8"]
    x = np.zeros((k["rows"], k["cols"]), np.uint32)
    for idx, bits in k["inputs"]:
        x.flat[idx] = int(bits, 16)
    q, e = oracle.encode_mxint8(x)
    assert q.shape == (2, k["kpad"])
    for idx, want in k["q"]:
        assert q.flat[idx] == want, idx
    for idx, want in k["e"]:
        assert e.flat[idx] == want, idx


def quantize_int8_exact(bits, e):
    v = value(bits) if (bits >> 23) & 0xFF else (
        Fraction(bits & 0x7FFFFF, 1 << 149) * (-1 if bits >> 31 else 1))
    y = v * Fraction(2) ** (6 - e)
    fl = y.numerator // y.denominator
    r = y - fl
    q = fl + (1 if r > Fraction(1, 2) or (r == Fraction(1, 2) and fl % 2) else 0)
    return max(-128, min(127, q))


def test_quantize_int8_closed_form(olib):
    rng = np.random.default_rng(5)
    for _ in range(5000):
        bits = int(rng.integers(0, 1 << 32)) & ~(0xFF << 23) | (int(rng.integers(0, 255)) << 23)
        e = int(rng.integers(-130, 130))
        assert olib.hbo_quantize_int8(bits, e) == quantize_int8_exact(bits, e)


def test_pack_abuf_layout(olib):
    k = known()["abuf_pack"]
    q = (np.arange(256) % 200 - 100).astype(np.int8).reshape(4, 64)
    e = np.array(k["e"], np.int32).reshape(4, 2)
    words = oracle.pack_abuf(q, e)
    assert words.shape == (2, 144)
    for kb in range(2):
        for j in range(4):
            assert np.array_equal(words[kb, j * 32:(j + 1) * 32].view(np.int8), q[j, kb * 32:(kb + 1) * 32])
            assert words[kb, 128 + j] == e[j, kb] + 127
        assert not words[kb, 132:].any()


def test_fbuf_pack_roundtrip(olib):
    x = (0x40000000 + 3 * np.arange(128)).astype(np.uint32).reshape(8, 16)
    words = np.zeros(128, np.uint32)
    assert olib.hbo_pack_fbuf(oracle._ptr(x, oracle.u32p), 8, 16, oracle._ptr(words, oracle.u32p)) == 0
    for r in range(8):
        for c in range(16):
            w, el = (r // 4) * 2 + c // 8, (r % 4) * 8 + c % 8
            assert words[w * 32 + el] == x[r, c]
    back = np.zeros_like(x)
    assert olib.hbo_unpack_fbuf(oracle._ptr(words, oracle.u32p), 8, 16, oracle._ptr(back, oracle.u32p)) == 0
    assert np.array_equal(back, x)


def test_pack_wbuf_and_split_w8(olib):
    rng = np.random.default_rng(6)
    w_int = rng.integers(-127, 128, (16, 64)).astype(np.float32)
    q, e = oracle.encode_mxint8(oracle.f32_bits(w_int))
    # lossless: q * 2^(e-6) reproduces the integers
    assert np.array_equal(q.astype(np.float64) * np.exp2(np.repeat(e, 32, axis=1) - 6), w_int)
    hi, lo = oracle.split_w8(q)
    assert np.array_equal(((hi.astype(np.int32) ^ 8) - 8) * 16 + lo, q.astype(np.int32))
    words = oracle.pack_wbuf(hi, e)
    for g in range(2):
        for kb in range(2):
            wd = words[g * 2 + kb]
            for c in range(8):
                nib = np.empty(32, np.uint8)
                nib[0::2] = wd[c * 16:(c + 1) * 16] & 15
                nib[1::2] = wd[c * 16:(c + 1) * 16] >> 4
                assert np.array_equal(nib, hi[g * 8 + c, kb * 32:(kb + 1) * 32])
                assert wd[128 + c] == e[g * 8 + c, kb] + 127


def test_canonical_mxfp4_preserves_values(olib):
    rng = np.random.default_rng(8)
    code = rng.integers(0, 16, (8, 64), dtype=np.uint8)
    code[0, :32] &= 0b1011  # a block whose top magnitude is below 4
    e = rng.integers(-10, -1, (8, 2)).astype(np.int32)
    oc, oe = oracle.canonical_mxfp4(code, e)
    mag = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6])

    def vals(c, ee):
        v = np.where(c & 8, -mag[c & 7], mag[c & 7])
        return v * np.exp2(np.repeat(ee, 32, axis=1).astype(np.float64))
    assert np.array_equal(vals(oc, oe), vals(code, e))
    tops = np.maximum.reduceat(oc & 7, [0, 32], axis=1)
    assert ((tops == 0) | (tops >= 6)).all()


def test_quantize_element_closed_form(olib):
    rng = np.random.default_rng(9)
    for _ in range(5000):
        emax = int(rng.integers(1, 255))
        e = int(rng.integers(max(0, emax - 30), emax + 1))
        bits = (int(rng.integers(0, 2)) << 31) | (e << 23) | int(rng.integers(0, 1 << 23))
        got = olib.hbo_quantize_element(bits, emax)
        v = value(bits) * Fraction(2) ** (6 - (emax - 127))
        mag = abs(v)
        fl = mag.numerator // mag.denominator
        r = mag - fl
        m = fl + (1 if r > Fraction(1, 2) or (r == Fraction(1, 2) and fl % 2) else 0)
        want = (0x80 if m >= 128 else (256 - m) & 0xFF) if bits >> 31 else (0x7F if m >= 128 else m)
        assert got == want


def test_activation_index_and_interpolation(olib):
    tbuf = helpers.activation_table("silu")
    rng = np.random.default_rng(10)
    tb = np.ascontiguousarray(tbuf)
    for _ in range(3000):
        e = int(rng.integers(100, 135))
        bits = (int(rng.integers(0, 2)) << 31) | (e << 23) | int(rng.integers(0, 1 << 23))
        got = olib.hbo_activation(bits, oracle._ptr(tb, oracle.u64p))
        x = abs(value(bits))
        if x >= 16:
            assert got == 0x3F800000
            continue
        fixed = int(x * (1 << 21))  # UQ4.21, truncated
        idx, frac = fixed >> 16, fixed & 0xFFFF
        entry = int(tbuf[512 + idx])
        s, v = entry >> 32, entry & 0xFFFFFFFF
        prod = round_binary32(value(s) * Fraction(frac, 1 << 16))
        assert got == round_binary32(value(v) + value(prod))


# ---- VEC passes ----

def vec_cmd(**kw):
    c = oracle.VecCmd()
    for k, v in kw.items():
        setattr(c, k, int(v))
    return c


def element(words, base, n8, row, col):
    return int(words[(base + (row // 4) * n8 + col // 8) % 4096, (row % 4) * 8 + col % 8])


@pytest.mark.parametrize("entry", [0, 1, 2, 3, 4, 5, 6, 7])
def test_elementwise_entries(olib, entry):
    """vec_engine_test.cpp:188-250 recipe: quads 3, n8 5, src 100, src2 300,
    dst 500, p_base 20; expected = the reference formulas per op."""
    rng = np.random.default_rng(100 + entry)
    mem = oracle.Memories()
    mem.fbuf[100:115] = helpers.random_fp32_words(rng, (15, 32))
    mem.fbuf[300:315] = helpers.random_fp32_words(rng, (15, 32))
    mem.pbuf[20:22] = helpers.random_fp32_words(rng, (2, 32))
    imm = int(helpers.random_fp32_words(rng, (1,), 120, 130)[0])
    before = mem.fbuf.copy()
    assert oracle.vec_exec(vec_cmd(entry=entry, src=100, src2=300, dst=500, rows_q=3, n8=5,
                                   p_base=20, imm=imm), mem) == 0
    add, mul = olib.hbo_fp32_add, olib.hbo_fp32_mul
    for row in range(12):
        for col in range(40):
            x, x2 = element(before, 100, 5, row, col), element(before, 300, 5, row, col)
            p = int(mem.pbuf[20 + col // 32, col % 32])
            want = {0: add(x, x2), 1: mul(x, x2), 3: add(x, p), 4: mul(x, p), 5: mul(x, imm),
                    6: x, 7: 0 if x >> 31 else x,
                    2: x if (x2 >> 31 and not x >> 31) or (x >> 31 == x2 >> 31 and
                       ((x & 0x7FFFFFFF) >= (x2 & 0x7FFFFFFF)) != bool(x >> 31)) or x == x2 else x2}[entry]
            assert element(mem.fbuf, 500, 5, row, col) == want, (entry, row, col)


@pytest.mark.parametrize("entry", [8, 9])
def test_activation_entries(olib, entry):
    """vec_engine_test.cpp:430-472: ACT = x * T(|x|) with the sign fix,
    ACT_MUL also times up."""
    rng = np.random.default_rng(200 + entry)
    mem = oracle.Memories()
    mem.tbuf[...] = helpers.activation_table("gelu")
    mem.fbuf[0:6] = helpers.random_fp32_words(rng, (6, 32), 110, 132)
    mem.fbuf[20:26] = helpers.random_fp32_words(rng, (6, 32), 120, 130)
    mem.fbuf[0, 0:3] = [0x41800000, 0xC1800001, 0x417FFFFF]
    before = mem.fbuf.copy()
    assert oracle.vec_exec(vec_cmd(entry=entry, src=0, src2=20, dst=40, rows_q=2, n8=3, imm=40), mem) == 0
    tb = np.ascontiguousarray(mem.tbuf)
    add, mul = olib.hbo_fp32_add, olib.hbo_fp32_mul
    for row in range(8):
        for col in range(24):
            x = element(before, 0, 3, row, col)
            t = olib.hbo_activation(x, oracle._ptr(tb, oracle.u64p))
            prod = mul(x, t)
            want = add(prod ^ 0x80000000, x) if x >> 31 else prod
            if entry == 9:
                want = mul(want, element(before, 20, 3, row, col))
            assert element(mem.fbuf, 40, 3, row, col) == want


def test_quantize_to_abuf(olib):
    """vec_engine_test.cpp:252-283: COPY with q, zero words and a subnormal."""
    rng = np.random.default_rng(300)
    mem = oracle.Memories()
    mem.fbuf[40:56] = helpers.random_fp32_words(rng, (16, 32), 100, 140)
    mem.fbuf[52:56] = 0
    mem.fbuf[45] = 0
    mem.fbuf[46, 3] = 1
    before = mem.fbuf.copy()
    assert oracle.vec_exec(vec_cmd(entry=6, quantize=1, src=40, dst=7000, rows_q=2, n8=8, imm=3000), mem) == 0
    for quad in range(2):
        for blk in range(2):
            words = np.stack([before[40 + quad * 8 + blk * 4 + qw] for qw in range(4)])
            want = np.zeros(132, np.uint8)
            assert olib.hbo_quantize_block(oracle._ptr(np.ascontiguousarray(words), oracle.u32p),
                                           oracle._ptr(want, oracle.u8p)) == 0
            assert np.array_equal(mem.abuf[7000 + quad * 2 + blk], want)


@pytest.mark.parametrize("cmd,text", [
    (dict(entry=6, src=10, dst=12, rows_q=1, n8=5), "after writing it"),
    (dict(entry=6, src=0, dst=0, rows_q=0, n8=5), "0 quads"),
    (dict(entry=6, quantize=1, src=0, dst=0, rows_q=2, n8=6), "out of order"),
    (dict(entry=6, quantize=1, src=0, dst=0, rows_q=1, n8=6), "ends inside a block"),
    (dict(entry=10, src=0, dst=0, rows_q=1, n8=4), "not an epilogue program"),
])
def test_vec_failures(olib, cmd, text):
    mem = oracle.Memories()
    assert oracle.vec_exec(vec_cmd(**cmd), mem) != 0
    assert text in oracle.last_error()
