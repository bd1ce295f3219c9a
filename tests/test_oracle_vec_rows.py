"""The oracle's row programs (SOFTMAX 12, LAYERNORM 22, RMSNORM 34;
tools/compiler/vec_rom.cpp:72-212, 239-272 run by tools/iss/vec_engine.cpp)
and their building blocks, pinned by:

- the reference's own lane and scalar-unit code (tools/iss/lane.cpp,
  scalar.cpp) compiled into oracle/_ref/libref_vec.so: Reciprocal,
  ReciprocalSqrt, CountReciprocal, SumTree, MaxTree, Fp32Max, Exp2,
  LaneOutput for every pass configuration the programs use, ApplyRowScalar;
- closed forms of the reference's program tests
  (tools/iss/vec_engine_test.cpp:283-420), restated here from the already
  pinned FP32 add / multiply and the pinned scalar functions: the row sum as
  8 accumulators over the words' 8-lane trees, then a tree; and of a
  program whose quads share words, run in the engine's pass order;
- mathematics: 1/x and 1/sqrt(x) within a few ulps, softmax rows summing to
  one, normalized rows of mean 0 / mean square 1;
- the reference's failure texts."""
from __future__ import annotations

import numpy as np
import pytest

import helpers
import oracle

u32 = np.uint32


def L():
    return oracle.lib()


def R():
    r = oracle.ref_vec()
    if r is None:
        pytest.skip("oracle/_ref/libref_vec.so is not built (no reference tree)")
    return r


def rand_bits(rng, shape, lo, hi):
    e = rng.integers(lo, hi + 1, shape, dtype=np.uint32)
    f = rng.integers(0, 1 << 23, shape, dtype=np.uint32)
    s = rng.integers(0, 2, shape, dtype=np.uint32)
    return (s << u32(31)) | (e << u32(23)) | f


def edge_bits():
    return np.array([0, 0x80000000, 1, 0x807FFFFF, 0x00800000, 0x3F800000, 0xBF800000,
                     0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000, 0x7FFFFFFF, 0xFFFFFFFF,
                     0x40000000, 0x3F000000, 0x00FFFFFF, 0x7E800000], np.uint32)


def ptr32(a):
    return a.ctypes.data_as(oracle.u32p)


def ptr64(a):
    return a.ctypes.data_as(oracle.u64p)


# ---- the scalar unit and trees against the reference's compiled code ----

def test_scalar_functions_match_the_reference():
    rng = np.random.default_rng(1)
    xs = np.concatenate([edge_bits(), rand_bits(rng, 20000, 0, 255)])
    for x in xs.tolist():
        assert L().hbo_reciprocal(x) == R().ref_reciprocal(x), hex(x)
        assert L().hbo_rsqrt(x) == R().ref_rsqrt(x), hex(x)
    for n in list(range(0, 2100)) + [0x3FFF, 0x4000, 0x7FF, 12345, 0xFFFFFFFF]:
        assert L().hbo_count_reciprocal(n) == R().ref_count_reciprocal(n), n


def test_scalar_functions_are_close_to_the_mathematics():
    """Independent of the reference build: after 4 Newton steps the results
    are within 4 ulps of 1/x and 1/sqrt(x) over normal inputs of moderate
    range (a wrong seed constant or step formula fails this)."""
    rng = np.random.default_rng(2)
    xs = rand_bits(rng, 5000, 100, 150) & u32(0x7FFFFFFF)
    for x in xs.tolist():
        v = float(np.array([x], np.uint32).view(np.float32)[0])
        for got, want in ((L().hbo_reciprocal(x), 1.0 / v), (L().hbo_rsqrt(x), v ** -0.5)):
            g = float(np.array([got], np.uint32).view(np.float32)[0])
            ulp = np.spacing(np.float32(want))
            assert abs(g - want) <= 4 * ulp, (hex(x), g, want)
    for n in (1, 3, 29, 64, 256, 960, 1024):
        g = float(np.array([L().hbo_count_reciprocal(n)], np.uint32).view(np.float32)[0])
        assert abs(g - 1.0 / n) <= 2 * np.spacing(np.float32(1.0 / n))


def test_trees_and_max_match_the_reference():
    rng = np.random.default_rng(3)
    for _ in range(3000):
        v = rand_bits(rng, 8, 90, 160)
        if rng.integers(0, 4) == 0:
            v[rng.integers(0, 8, 3)] = edge_bits()[rng.integers(0, len(edge_bits()), 3)]
        assert L().hbo_sum_tree(ptr32(v)) == R().ref_sum_tree(ptr32(v))
        assert L().hbo_max_tree(ptr32(v)) == R().ref_max_tree(ptr32(v))
        a, b = int(v[0]), int(v[1])
        assert L().hbo_fp32_max(a, b) == R().ref_fp32_max(a, b)


def test_exp2_matches_the_reference():
    rng = np.random.default_rng(4)
    tb = helpers.activation_table("silu")
    xs = np.concatenate([edge_bits(), rand_bits(rng, 40000, 90, 140),
                         rand_bits(rng, 2000, 0, 255)])
    for x in xs.tolist():
        assert L().hbo_exp2(x, ptr64(tb)) == R().ref_exp2(x, ptr64(tb)), hex(x)


# the pass configurations of the three programs: (c0, b, nl, cmp, sel)
PASSES = {
    "layernorm sum": (0, 0, 0, 0, 0), "layernorm squares": (1, 1, 0, 0, 0),
    "layernorm normalize": (1, 2, 0, 0, 0), "gamma": (0, 3, 0, 0, 0), "beta": (2, 0, 0, 0, 0),
    "rmsnorm squares": (0, 1, 0, 0, 0), "rmsnorm normalize": (0, 2, 0, 0, 0),
    "softmax max": (0, 0, 0, 1, 2), "softmax exp": (1, 4, 1, 1, 1), "softmax normalize": (0, 2, 0, 0, 0),
}


@pytest.mark.parametrize("name", sorted(PASSES))
def test_lane_output_matches_the_reference(name):
    c0, b, nl, cmp, sel = PASSES[name]
    rng = np.random.default_rng(sum(name.encode()))
    tb = helpers.activation_table("silu")
    for _ in range(4000):
        x, pb, rs0, rs1 = (int(v) for v in rand_bits(rng, 4, 100, 150))
        if rng.integers(0, 8) == 0:
            x = int(edge_bits()[rng.integers(0, len(edge_bits()))])
        t, l, w = int(rng.integers(0, 4)), int(rng.integers(0, 8)), int(rng.integers(0, 40))
        imm = 0x3FB8AA3B if b == 4 else int(rand_bits(rng, 1, 110, 130)[0])
        imm2 = int(rng.integers(0, 330))
        args = (c0, b, nl, cmp, sel, x, pb, t, l, w, imm, imm2, rs0, rs1, ptr64(tb))
        assert L().hbo_row_lane(*args) == R().ref_lane_output(*args), (name, args[5:14])


@pytest.mark.parametrize("red,sf,st,srn,seps", [(1, 1, 1, 1, 0), (1, 3, 0, 1, 1), (2, 1, 1, 0, 0),
                                                (1, 2, 0, 0, 0), (2, 4, 0, 0, 0)])
def test_apply_row_scalar_matches_the_reference(red, sf, st, srn, seps):
    rng = np.random.default_rng(red * 100 + sf * 10 + st)
    for _ in range(500):
        sums = rand_bits(rng, 32, 110, 140)
        if sf == 3:
            sums &= u32(0x7FFFFFFF)
        mx = rand_bits(rng, 4, 110, 140)
        eps, rn = 0x3727C5AC, int(L().hbo_count_reciprocal(int(rng.integers(1, 2000))))
        a, b = np.zeros(4, np.uint32), np.zeros(4, np.uint32)
        L().hbo_apply_row_scalar(red, sf, st, srn, seps, ptr32(sums), ptr32(mx), eps, rn, ptr32(a))
        R().ref_apply_row_scalar(red, sf, st, srn, seps, ptr32(sums), ptr32(mx), eps, rn, ptr32(b))
        assert np.array_equal(a, b)


# ---- whole programs against the reference tests' closed forms ----

EPS = 0x3727C5AC  # vec_engine_test.cpp:21
LOG2E = 0x3FB8AA3B


def add(a, b):
    return L().hbo_fp32_add(int(a), int(b))


def mul(a, b):
    return L().hbo_fp32_mul(int(a), int(b))


def neg(b):
    return 0 if (b & 0x7FFFFFFF) == 0 else b ^ 0x80000000


def tree(v):
    return add(add(add(v[0], v[1]), add(v[2], v[3])), add(add(v[4], v[5]), add(v[6], v[7])))


def row_sum(values):
    """RowSum (the reference test helper): 8 accumulators over the groups of
    8, accumulator j % 8, each adding its group's tree; then a tree."""
    acc = [0] * 8
    for j in range(len(values) // 8):
        acc[j % 8] = add(acc[j % 8], tree(values[8 * j: 8 * j + 8]))
    return tree(acc)


def row_max(values):
    best = 0xFF800000
    for v in values:
        best = L().hbo_fp32_max(best, int(v))  # ties keep the earlier value
    return best


def element(fbuf, base, n8, row, col):
    return int(fbuf[(base + (row // 4) * n8 + col // 8) % 4096][(row % 4) * 8 + col % 8])


def run(cmd_kw, mem):
    c = oracle.VecCmd()
    for k, v in cmd_kw.items():
        setattr(c, k, v)
    return oracle.vec_exec(c, mem)


def fill(mem, rng, first, count, lo, hi, what="fbuf"):
    img = getattr(mem, what)
    for w in range(first, first + count):
        img[w % img.shape[0]] = rand_bits(rng, 32, lo, hi)


@pytest.mark.parametrize("quantize", [False, True])
def test_layernorm_program(quantize):
    """vec_engine_test.cpp:286-340: 2 quads of 8 words, gamma / beta in PBUF."""
    rng = np.random.default_rng(5 + quantize)
    mem = oracle.Memories()
    quads, n8, src, scratch, pbase = 2, 8, 64, 900, 30
    dst = 5000 if quantize else 640
    fill(mem, rng, src, quads * n8, 120, 132)
    fill(mem, rng, pbase, 4, 124, 128, "pbuf")
    before = mem.fbuf.copy()
    assert run(dict(entry=22, quantize=int(quantize), src=src, src2=scratch if quantize else dst,
                    dst=dst, rows_q=quads, n8=n8, p_base=pbase, aux=n8 * 8, imm=EPS), mem) == 0
    n = n8 * 8
    rn = L().hbo_reciprocal(0x42800000)  # FromInt(64)
    gamma = lambda c: int(mem.pbuf[pbase + c // 32][c % 32])
    beta = lambda c: int(mem.pbuf[pbase + n8 // 4 + c // 32][c % 32])
    rows = []
    for row in range(quads * 4):
        x = [element(before, src, n8, row, c) for c in range(n)]
        negative_mean = neg(mul(row_sum(x), rn))
        d = [add(v, negative_mean) for v in x]
        rstd = L().hbo_rsqrt(add(mul(row_sum([mul(v, v) for v in d]), rn), EPS))
        out = [add(mul(mul(d[c], rstd), gamma(c)), beta(c)) for c in range(n)]
        rows.append(out)
        if not quantize:
            got = [element(mem.fbuf, dst, n8, row, c) for c in range(n)]
            assert got == out, row
        # mathematics: the normalized row has mean ~0 and mean square ~1
        z = np.array([mul(d[c], rstd) for c in range(n)], np.uint32).view(np.float32).astype(float)
        assert abs(z.mean()) < 1e-5 and abs((z * z).mean() - 1) < 1e-3
    if quantize:
        for q in range(quads):
            for b in range(n8 // 4):
                words = np.zeros((4, 32), np.uint32)
                for qw in range(4):
                    for t in range(4):
                        for l in range(8):
                            words[qw][t * 8 + l] = rows[q * 4 + t][b * 32 + qw * 8 + l]
                want = np.zeros(132, np.uint8)
                L().hbo_quantize_block(ptr32(words), want.ctypes.data_as(oracle.u8p))
                assert np.array_equal(mem.abuf[dst + q * (n8 // 4) + b], want), (q, b)


def test_rmsnorm_program():
    """vec_engine_test.cpp:344-380: 3 quads of 4 words, count 29 (not n8 * 8),
    the scratch region is the destination."""
    rng = np.random.default_rng(7)
    mem = oracle.Memories()
    quads, n8, src, dst, pbase, count = 3, 4, 10, 60, 3, 29
    fill(mem, rng, src, quads * n8, 118, 134)
    fill(mem, rng, pbase, 1, 124, 128, "pbuf")
    before = mem.fbuf.copy()
    assert run(dict(entry=34, quantize=0, src=src, src2=dst, dst=dst, rows_q=quads, n8=n8,
                    p_base=pbase, aux=count, imm=EPS), mem) == 0
    rn = L().hbo_reciprocal(0x41E80000)  # FromInt(29)
    assert rn == L().hbo_count_reciprocal(count)
    for row in range(quads * 4):
        x = [element(before, src, n8, row, c) for c in range(n8 * 8)]
        rstd = L().hbo_rsqrt(add(mul(row_sum([mul(v, v) for v in x]), rn), EPS))
        want = [mul(mul(x[c], rstd), int(mem.pbuf[pbase + c // 32][c % 32])) for c in range(n8 * 8)]
        assert [element(mem.fbuf, dst, n8, row, c) for c in range(n8 * 8)] == want, row


def test_rmsnorm_quads_sharing_words():
    """Quads that read what other quads write run in the engine's order:
    pairs of quads pass by pass, each in its own row context, and a last
    odd quad alone (Grouped, tools/compiler/vec_rom.cpp:84-131, with
    kContexts = 2, tools/iss/vec_engine.hpp:14).  RMSNorm over 3 quads of 4
    words, quad q's source at 100 + 4q, its scratch and destination at
    104 + 4q: quad 1 computes its rstd from its own source, then normalizes
    quad 0's scratch, which quad 0's second pass wrote there in between;
    quad 2 then reads quad 1's result."""
    rng = np.random.default_rng(11)
    mem = oracle.Memories()
    n8, pbase, count = 4, 3, 32
    fill(mem, rng, 100, 3 * n8, 118, 134)
    fill(mem, rng, pbase, 1, 124, 128, "pbuf")
    before = mem.fbuf.copy()
    assert run(dict(entry=34, quantize=0, src=100, src2=104, dst=104, rows_q=3, n8=n8,
                    p_base=pbase, aux=count, imm=EPS), mem) == 0
    rn = L().hbo_count_reciprocal(count)
    gamma = [int(mem.pbuf[pbase + c // 32][c % 32]) for c in range(32)]

    def quad(img, base):
        return [[element(img, base, n8, t, c) for c in range(32)] for t in range(4)]

    def rstd(m):
        return [L().hbo_rsqrt(add(mul(row_sum([mul(v, v) for v in row]), rn), EPS)) for row in m]

    def scale(m, r):
        return [[mul(v, r[t]) for v in m[t]] for t in range(4)]

    def times_gamma(m):
        return [[mul(v, gamma[c]) for c, v in enumerate(row)] for row in m]

    x0, x1 = quad(before, 100), quad(before, 104)
    r0, r1 = rstd(x0), rstd(x1)  # pass 1 of quads 0 and 1
    n0 = scale(x0, r0)  # quad 0's pass 2 -> 104..107
    q0 = times_gamma(n0)  # quad 0's pass 3 -> 104..107
    q1 = times_gamma(scale(n0, r1))  # quad 1's passes 2, 3 over quad 0's scratch -> 108..111
    q2 = times_gamma(scale(q1, rstd(q1)))  # quad 2 alone, source = quad 1's result
    assert quad(mem.fbuf, 100) == quad(before, 100)
    assert quad(mem.fbuf, 104) == q0
    assert quad(mem.fbuf, 108) == q1
    assert quad(mem.fbuf, 112) == q2
    # the order matters here: quad 1 run on its own source gives other words
    assert q1 != times_gamma(scale(x1, r1))


@pytest.mark.parametrize("valid", [50, 64, 1])
def test_softmax_program(valid):
    """vec_engine_test.cpp:384-420: 2 quads of 8 words, the first `valid`
    columns, the 2^f table; rows sum to one over the valid columns."""
    rng = np.random.default_rng(9 + valid)
    mem = oracle.Memories()
    quads, n8, src, dst = 2, 8, 200, 400
    fill(mem, rng, src, quads * n8, 120, 131)
    mem.tbuf[:] = helpers.activation_table("silu")
    before = mem.fbuf.copy()
    assert run(dict(entry=12, quantize=0, src=src, src2=0, dst=dst, rows_q=quads, n8=n8,
                    p_base=0, aux=valid, imm=dst), mem) == 0
    tb = mem.tbuf
    for row in range(quads * 4):
        x = [element(before, src, n8, row, c) for c in range(valid)]
        negative_max = neg(row_max(x))
        e = [L().hbo_exp2(mul(add(v, negative_max), LOG2E), ptr64(tb)) for v in x]
        e += [0] * (n8 * 8 - valid)
        inverse = L().hbo_reciprocal(row_sum(e))
        want = [mul(e[c], inverse) if c < valid else 0 for c in range(n8 * 8)]
        got = [element(mem.fbuf, dst, n8, row, c) for c in range(n8 * 8)]
        assert got == want, row
        p = np.array(got, np.uint32).view(np.float32).astype(float)
        assert abs(p.sum() - 1) < 1e-4
        xs = np.array(x, np.uint32).view(np.float32).astype(float)
        ref = np.exp(xs - xs.max())
        assert np.abs(p[:valid] - ref / ref.sum()).max() < 2e-3


def test_row_program_failures_carry_the_reference_texts():
    mem = oracle.Memories()
    kw = dict(entry=34, quantize=0, src=10, src2=200, dst=200, rows_q=1, n8=0, p_base=0,
              aux=8, imm=EPS)
    assert run(kw, mem) != 0 and oracle.last_error() == "a PASS has 1 quads and 0 words"
    kw.update(n8=6, quantize=1)
    assert run(kw, mem) != 0
    assert oracle.last_error() == "a PASS ends inside a block of 4 quantized words"
    kw.update(n8=4, quantize=0, entry=22, src2=11)  # scratch one word past src
    assert run(kw, mem) != 0
    assert oracle.last_error() == "a PASS reads FBUF word 11 after writing it"
    kw.update(rows_q=0)  # no quads: no PASS runs, no failure
    assert run(kw, mem) == 0
