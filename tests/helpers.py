"""Shared generators for the parity tests (seeded, numpy only)."""
from __future__ import annotations

import numpy as np

import oracle

MASK20 = (1 << 20) - 1


def random_memories(seed: int, scale_lo=118, scale_hi=136, fbuf_lo=0x3F000000) -> oracle.Memories:
    """Fill(seed) recipe of tools/iss/gemm_array_test.cpp:45-70: random bytes,
    scale bytes in [118, 136], FBUF = 0x3F000000 + (byte << 16)."""
    rng = np.random.default_rng(seed)
    m = oracle.Memories()
    m.abuf[:, :128] = rng.integers(0, 256, (8192, 128), dtype=np.uint8)
    m.abuf[:, 128:132] = rng.integers(scale_lo, scale_hi + 1, (8192, 4), dtype=np.uint8)
    m.wbuf[:, :128] = rng.integers(0, 256, (2048, 128), dtype=np.uint8)
    m.wbuf[:, 128:136] = rng.integers(scale_lo, scale_hi + 1, (2048, 8), dtype=np.uint8)
    m.fbuf[...] = fbuf_lo + (rng.integers(0, 256, (4096, 32), dtype=np.uint32) << 16)
    m.pbuf[...] = 0x3F000000 + (rng.integers(0, 256, (512, 32), dtype=np.uint32) << 16)
    return m


def gemm_cmd(**kw) -> oracle.GemmCmd:
    c = oracle.GemmCmd()
    for k, v in kw.items():
        setattr(c, k, int(v))
    return c


def cmd_dict(c) -> dict:
    return {f: getattr(c, f) for f, _ in c._fields_}


def random_fp32_words(rng, shape, lo=110, hi=140):
    """FP32 bits with exponent field in [lo, hi] and random sign/fraction."""
    e = rng.integers(lo, hi + 1, shape, dtype=np.uint32)
    s = rng.integers(0, 2, shape, dtype=np.uint32)
    f = rng.integers(0, 1 << 23, shape, dtype=np.uint32)
    return ((s << 31) | (e << 23) | f).astype(np.uint32)


def activation_table(kind: str = "silu") -> np.ndarray:
    """A 1024-entry TBUF: [0,512) 2^f, [512,1024) sigma or Phi-tilde, entries
    {slope = fp32(v[i+1] - v[i]), value = fp32(F(i h))} as tools/compiler/
    tensors.cpp:28-62 lays them out.  Values here are float64-rounded; the
    table is an input of the kernels, so its exact bits are test data."""
    seg = 512
    i = np.arange(seg + 1, dtype=np.float64)
    e2 = np.exp2(i / seg)
    x = i / 32.0
    if kind == "silu":
        act = 1.0 / (1.0 + np.exp(-x))
    else:
        act = 0.5 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
    out = np.zeros(1024, np.uint64)
    for base, v in ((0, e2), (512, act)):
        vb = v.astype(np.float32)
        slope = (vb[1:].astype(np.float64) - vb[:-1].astype(np.float64)).astype(np.float32)
        out[base:base + seg] = (slope.view(np.uint32).astype(np.uint64) << np.uint64(32)) | \
            vb[:-1].view(np.uint32).astype(np.uint64)
    return out


# ------------------------------------------------------------ linear data --

def mxfp4_weights(rng, n: int, k: int, exp_lo=-10, exp_hi=-2):
    """MXFP4 weights W[n][k]: codes uniform over 16, E8M0 exponent uniform
    in [exp_lo, exp_hi] per 32-block."""
    code = rng.integers(0, 16, (n, k), dtype=np.uint8)
    e = rng.integers(exp_lo, exp_hi + 1, (n, k // 32)).astype(np.int32)
    return code, e


def w8_planes_from_int8(w_int: np.ndarray):
    """int8-valued weights [n][k] -> MXINT8 (lossless) -> SplitW8 planes."""
    q, e = oracle.encode_mxint8(oracle.f32_bits(w_int.astype(np.float32)))
    hi, lo = oracle.split_w8(q)
    return oracle.pack_wbuf(hi, e), oracle.pack_wbuf(lo, e)


def activations_fp8(rng, m: int, k: int, scale=1.0):
    """fp32 [m][k] ~ N(0, scale^2) -> MXFP8 E4M3 DDR words over ceil(m/4)
    quads (the oracle's OCP MX encoder)."""
    x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
    mp = (m + 3) // 4 * 4
    xp = np.zeros((mp, k), np.float32)
    xp[:m] = x
    q, e = oracle.encode_mxfp8(oracle.f32_bits(xp))
    return x, oracle.pack_abuf(q.view(np.int8), e)


def activations(rng, m: int, k: int):
    """fp32 [m][k] ~ N(0,1) -> MXINT8 DDR words over ceil(m/4) quads."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    mp = (m + 3) // 4 * 4
    xp = np.zeros((mp, k), np.float32)
    xp[:m] = x
    q, e = oracle.encode_mxint8(oracle.f32_bits(xp))
    return x, oracle.pack_abuf(q, e)


# ------------------------------------------------- oracle over threads --

def oracle_threads() -> int:
    """Host threads for the oracle: the cores, at most 16 (one GPU's share of
    a GPU box's cores)."""
    import os
    return max(1, min(16, os.cpu_count() or 1))


def oracle_linear_mt(m, n, kb, a, planes, modes, ops=(), pieces=None, onto=None, tbuf=None,
                     quantize=False, threads=None, a_fp8=False):
    """oracle.linear over column slices on several host threads: column
    groups are independent in the reference's loop nest
    (tools/iss/gemm_array.cpp:123-147), and every epilogue op and the
    requantize are per column or per 32-column block.  m is padded to whole
    quads as the oracle needs; returns (c bits [m][n], q words or None).
    a_fp8: A holds MXFP8 E4M3 words (one MXFP4 plane)."""
    from concurrent.futures import ThreadPoolExecutor
    mp = (m + 3) // 4 * 4
    unit = 32 if quantize else 8
    parts = max(1, min(threads or oracle_threads(), n // unit))
    bounds = [(n // unit) * i // parts * unit for i in range(parts + 1)]
    wplanes = [np.asarray(p).reshape(n // 8, kb, 144) for p in planes]

    def pad_rows(x):
        out = np.zeros((mp, n), np.uint32)
        out[:m] = x
        return out

    c0 = pad_rows(onto) if onto is not None else None
    full_ops = [(k, pad_rows(v) if k in (EP_ACT_MUL, EP_ADD) else v) for k, v in ops]

    def part(i):
        lo, hi = bounds[i], bounds[i + 1]
        if lo == hi:
            return None
        sub_planes = [np.ascontiguousarray(w[lo // 8: hi // 8]).reshape(-1, 144) for w in wplanes]
        sub_ops = []
        for kind, arg in full_ops:
            if kind in (EP_ACT_MUL, EP_ADD):
                sub_ops.append((kind, np.ascontiguousarray(arg[:, lo:hi])))
            elif kind in (EP_ADDP, EP_MULP):
                sub_ops.append((kind, np.ascontiguousarray(arg[lo:hi])))
            else:
                sub_ops.append((kind, arg))
        c = np.ascontiguousarray(c0[:, lo:hi]) if c0 is not None else None
        return oracle.linear(mp, hi - lo, kb, a, sub_planes, modes, pieces=pieces, c=c,
                             onto=onto is not None, ops=sub_ops, tbuf=tbuf, quantize=quantize,
                             a_fp8=a_fp8)

    with ThreadPoolExecutor(parts) as pool:
        results = list(pool.map(part, range(parts)))
    c = np.zeros((mp, n), np.uint32)
    q = np.zeros((mp // 4, n // 32, 144), np.uint8) if quantize else None
    for i, r in enumerate(results):
        if r is None:
            continue
        lo, hi = bounds[i], bounds[i + 1]
        c[:, lo:hi] = r[0]
        if quantize:
            q[:, lo // 32: hi // 32] = r[1].reshape(mp // 4, (hi - lo) // 32, 144)
    return c[:m], (q.reshape(-1, 144) if quantize else None)


EP_ADDP, EP_MULP, EP_SCALE, EP_COPY, EP_RELU, EP_ACT, EP_ACT_MUL, EP_ADD = 3, 4, 5, 6, 7, 8, 9, 0x100


def block_abs_sums(m, n, kb, a, planes, modes, pieces=None):
    """sum over the folded blocks of |block value| per output: the scale of
    the fast mode's accumulation-order error (each FP32 addition rounds by at
    most 2^-24 of its running sum, which is at most this sum).  Float64
    matrix products per block are exact (|block sum| < 2^17)."""
    qa = np.asarray(a).reshape(-1, kb, 144)
    rows = qa.shape[0] * 4
    aq = qa[:, :, :128].view(np.int8).reshape(-1, kb, 4, 32).transpose(0, 2, 1, 3) \
        .reshape(rows, kb, 32).astype(np.float64)
    ea = qa[:, :, 128:132].astype(np.int64).transpose(0, 2, 1).reshape(rows, kb)
    blocks = range(kb) if pieces is None else [o + i for o, k in pieces for i in range(k)]
    mag = np.array([0, 1, 2, 3, 4, 6, 8, 12])
    tot = np.zeros((rows, n))
    for plane, mode in zip(planes, modes):
        w = np.asarray(plane).reshape(n // 8, kb, 144)
        nib = np.empty((n // 8, kb, 8, 32), np.int64)
        nib[..., 0::2] = (w[:, :, :128] & 15).reshape(n // 8, kb, 8, 16)
        nib[..., 1::2] = (w[:, :, :128] >> 4).reshape(n // 8, kb, 8, 16)
        if mode == 0:
            v = np.where(nib & 8, -mag[nib & 7], mag[nib & 7])
        elif mode == 1:
            v = np.where(nib & 8, nib - 16, nib)
        else:
            v = nib
        v = v.transpose(0, 2, 1, 3).reshape(n, kb, 32).astype(np.float64)
        ew = w[:, :, 128:136].astype(np.int64).transpose(0, 2, 1).reshape(n, kb)
        bias = {0: -7, 1: -8, 2: -12}[mode]
        for b in blocks:
            s = np.abs(aq[:, b, :] @ v[:, b, :].T)
            tot += s * np.exp2((ea[:, b:b + 1] - 127) + (ew[:, b][None, :] - 127) + bias)
    return tot[:m]


def check_fast(got, want, gq=None, wq=None, bound=None):
    """Fast-mode tolerance: per output row, max |gpu - ref| <= 1e-5 max |ref|
    (normwise); with `bound` (sum |block value| per output) also per element
    |gpu - ref| <= 2^-17 bound (plus one rounding of the result).  The
    per-element factor is an envelope measured on the matrix cores, not a
    proof: their internal summation of a 64-deep product is not documented,
    and operands whose int8 codes cover all 256 values reached 1.9e-6
    (2^-19.0) at K = 384, where one FP32 rounding per instruction would give
    3.5e-7.  Requantized bytes may differ by 1 where the values straddle a
    step."""
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    err = np.abs(g - w)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (err <= 1e-5 * row_scale).all(), float((err / np.maximum(row_scale, 1e-300)).max())
    if bound is not None:
        assert (err <= 2.0 ** -17 * bound + 2.0 ** -23 * np.abs(w) + 1e-30).all(), \
            float((err / (bound + 1e-30)).max())
    if gq is not None:
        check_requantized(gq, wq)


def check_requantized(gq, wq):
    """Requantized MXINT8 words of a fast-mode C against the exact ones.  A
    row's block takes the scale of its largest element, so where that
    element sits within the fast-mode error of a power of two the two scale
    bytes differ by one and the block's codes are on steps twice as large:
    per element the values agree within one step of the coarser scale.
    Where the scale bytes agree the codes differ by at most 1; scale bytes
    differ in fewer than 1% of the blocks and codes in fewer than 1%.
    (Rounding on each side and the saturation of a block's largest code
    at 127 add up to at most one and a half steps of the coarser scale.)"""
    g = gq.reshape(-1, 144)
    w = wq.reshape(-1, 144)
    gqb = g[:, :128].view(np.int8).astype(np.int64).reshape(-1, 4, 32)
    wqb = w[:, :128].view(np.int8).astype(np.int64).reshape(-1, 4, 32)
    gs, ws = g[:, 128:132].astype(np.int64), w[:, 128:132].astype(np.int64)
    assert (g[:, 132:] == 0).all()
    same = gs == ws
    assert np.abs(gs - ws).max() <= 1 and (~same).mean() < 0.01
    assert (np.abs(gqb - wqb)[same] <= 1).all() and (gqb != wqb).mean() < 0.01
    lo = np.minimum(gs, ws)[..., None]
    vg = gqb * np.exp2(gs[..., None] - lo)
    vw = wqb * np.exp2(ws[..., None] - lo)
    assert (np.abs(vg - vw) <= 1.5 * np.exp2(np.maximum(gs, ws)[..., None] - lo)).all()


def random_a_words(rng, m, kb, lo=118, hi=132):
    """MXINT8 DDR words over ceil(m/4) quads whose codes are uniform over all
    256 int8 values (so -128, which the VEC requantize emits on saturation,
    appears), with scale bytes in [lo, hi]; rows past m are zero."""
    quads = (m + 3) // 4
    a = np.zeros((quads, kb, 144), np.uint8)
    a[:, :, :128] = rng.integers(0, 256, (quads, kb, 128), dtype=np.uint8)
    a[:, :, 128:132] = rng.integers(lo, hi + 1, (quads, kb, 4), dtype=np.uint8)
    if m % 4:
        for t in range(m % 4, 4):
            a[-1, :, 32 * t: 32 * t + 32] = 0
    return a.reshape(-1, 144)
