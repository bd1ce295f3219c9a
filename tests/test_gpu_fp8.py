"""MXFP8 E4M3 activations (HB_LINEAR_A_FP8, no counterpart in the
reference) on an MI355X against the oracle's definition (hb_oracle.c,
pinned in test_oracle_fp8.py):

  * hb_encode_mxfp8 byte for byte against the oracle's OCP MX encoder
    (zero, subnormal and saturating blocks, ragged rows and K, Inf
    rejected);
  * exact mode bitwise: ops with requantize, pieces, `onto`, weight panels,
    a batch of layers;
  * fast mode (FP8 x FP4 matrix cores, each block's codes in two
    exponent planes) within the fast-mode bound of the MXINT8 path
    (check_fp8_fast) at config 1's sweep M in {1, 16, 128, 1024} (K = 2560,
    N = 960) one layer per launch and batched (the streaming kernel, more
    tiles than CUs, from C, a partial panel, a mid-stream exact recompute;
    the skinny kernel for up to 16 rows: ragged rows, partial panels, DDR
    words, pieces, an out-of-window scale),
    and M = 141, with ops and requantize, and with scale bytes outside the
    fast window (those tiles are computed exactly, bitwise);
  * the descriptor rule (one MXFP4 plane).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
import oracle
from test_gpu_bench_routes import DEV, dev, host, mxfp4_planes, say, to_panels

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [(4, 32), (13, 50), (128, 2560), (1001, 96)])
def test_encode_mxfp8(gpu, rows, cols):
    rng = np.random.default_rng(700 + rows)
    x = (rng.standard_normal((rows, cols)) * 2.0 ** rng.integers(-30, 30, (rows, 1))).astype(np.float32)
    x[0, :min(32, cols)] = 0.0
    if rows > 2:
        x[1, :min(32, cols)] = np.float32(1e-41)           # subnormal block
        x[2, 0] = np.float32(1.9 * 2.0 ** 20)              # scaled past 448: saturates
    quads, blocks = (rows + 3) // 4, (cols + 31) // 32
    out = torch.full((quads * blocks, 144), 0xA5, dtype=torch.uint8, device=DEV)
    say("encode_mxfp8", dict(rows=rows, cols=cols))
    hb.encode_mxfp8(dev(x), rows, cols, out, ctx=gpu)
    xp = np.zeros((quads * 4, cols), np.float32)
    xp[:rows] = x
    q, e = oracle.encode_mxfp8(oracle.f32_bits(xp))
    assert np.array_equal(host(out), oracle.pack_abuf(q.view(np.int8), e))


def test_encode_mxfp8_rejects_inf(gpu):
    x = np.ones((4, 32), np.float32)
    x[2, 5] = np.inf
    out = torch.zeros((32, 144), dtype=torch.uint8, device=DEV)
    with pytest.raises(hb.HbError) as err:
        hb.encode_mxfp8(dev(x), 4, 32, out, ctx=gpu)
    assert err.value.code == hb.HB_EINVAL and "MXFP8" in err.value.message


def fp8_layer(gpu, m, n, kb, mode, ops_fn=None, quantize=False, tbuf=None, seed=0,
              pieces=None, onto=False, panels=False, w_lo=-10, w_hi=-2, a_scale=1.0):
    rng = np.random.default_rng(seed)
    a = helpers.activations_fp8(rng, m, kb * 32, a_scale)[1]
    code, e = helpers.mxfp4_weights(rng, n, kb * 32, w_lo, w_hi)
    planes = [oracle.pack_wbuf(code, e)]
    w_dev = [dev(planes[0])]
    if panels:
        w_dev = [to_panels(gpu, w_dev[0], n, kb)]
    ops = ops_fn(rng, m, n) if ops_fn else []
    dev_ops = [(k, dev(v.view(np.float32)) if isinstance(v, np.ndarray) else v) for k, v in ops]
    c0 = helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else np.zeros((m, n), np.uint32)
    c_d = dev(c0.view(np.float32))
    q_d = torch.zeros(((m + 3) // 4 * (n // 32), 144), dtype=torch.uint8, device=DEV) \
        if quantize else None
    tb_d = dev(tbuf.view(np.int64)) if tbuf is not None else None
    say("fp8 layer", dict(m=m, n=n, kb=kb, mode=mode, ops=[o[0] for o in ops], quantize=quantize,
                          pieces=pieces, onto=onto, panels=panels))
    hb.linear(gpu, a=dev(a), planes=w_dev, modes=[0], c=c_d, m=m, n=n, kb_total=kb, ops=dev_ops,
              tbuf=tb_d, q_out=q_d, mode=mode, pieces=pieces, onto=onto, panels=panels,
              a_fp8=True)
    got = host(c_d).view(np.uint32)
    gq = host(q_d) if quantize else None
    want, wq = helpers.oracle_linear_mt(m, n, kb, a, planes, [0], ops=ops, tbuf=tbuf,
                                        quantize=quantize, pieces=pieces,
                                        onto=c0 if onto else None, a_fp8=True)
    fp8_layer.abs_sums = (lambda: fp8_abs_sums(m, n, kb, a, planes[0]))
    return got, gq, want, wq


FP8_INT = np.array([oracle.fp8_int(c) for c in range(256)], np.float64)
E2M1_INT = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float64)


def fp8_abs_sums(m, n, kb, a_words, w_words):
    """sum over blocks of |block value| per output (the scale of the fast
    path's accumulation error), from the DDR words."""
    aw = np.asarray(a_words).reshape(-1, kb, 144)
    ww = np.asarray(w_words).reshape(n // 8, kb, 144)
    tot = np.zeros((m, n))
    for b in range(kb):
        codes = aw[:, b, :128].reshape(-1, 4, 32).reshape(-1, 32)[:m]
        ea = aw[:, b, 128:132].reshape(-1)[:m].astype(np.int64)
        ai = FP8_INT[codes]
        nib = ww[:, b, :128].reshape(n // 8, 8, 16)
        wc = np.stack([nib & 15, nib >> 4], -1).reshape(n, 32)
        ew = ww[:, b, 128:136].reshape(-1).astype(np.int64)
        s = np.abs(ai @ E2M1_INT[wc].T)
        tot += s * np.exp2((ea[:, None] + ew[None, :] - 264).astype(np.float64))
    return tot


def check_fp8_fast(got, want, abs_sums, gq=None, wq=None):
    """The fast-mode bound of the MXINT8 path, an envelope measured on the
    matrix cores (not a proof): per output row max |gpu - ref| <= 1e-5 max
    |ref|, per element |gpu - ref| <= 2^-17 sum |block value| (+ one
    rounding of the result).  The matrix cores sum an instruction's FP8 x
    FP4 products exactly only while they span few binades, so each block's
    codes go through two MFMAs split by exponent (measured worst 3.3e-7 per
    row and 2^-21.6 per element; one MFMA over the whole E4M3 range gave
    1.7e-5 and 2^-14.3).  (Exact mode is bitwise.)"""
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    err = np.abs(g - w)
    row = np.abs(w).max(axis=1, keepdims=True)
    r1 = float((err / np.maximum(row, 1e-300)).max())
    r2 = float((err / np.maximum(abs_sums, 1e-300)).max())
    say("fp8 fast error", dict(normwise=r1, per_element_log2=float(np.log2(max(r2, 1e-300)))))
    assert r1 <= 1e-5, r1
    assert (err <= 2.0 ** -17 * abs_sums + 2.0 ** -23 * np.abs(w) + 1e-30).all(), r2
    if gq is not None:
        helpers.check_requantized(gq, wq)


def per_channel(r, m, n):
    return [(hb.EP_MULP, np.asarray(r.uniform(0.5, 2.0, n), np.float32).view(np.uint32)),
            (hb.EP_ADDP, np.asarray(r.normal(0, 0.1, n), np.float32).view(np.uint32))]


@pytest.mark.parametrize("m,n,kb,kw", [
    (50, 256, 23, dict(ops_fn=lambda r, m, n: per_channel(r, m, n) + [(hb.EP_ACT, None)],
                       quantize=True, tbuf=helpers.activation_table("silu"))),
    (141, 320, 30, dict(pieces=[(0, 12), (12, 18)], onto=True)),
    (64, 512, 16, dict(panels=True, quantize=True)),
    (200, 96, 7, dict(ops_fn=lambda r, m, n: [(hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))]))])
def test_exact_bitwise(gpu, m, n, kb, kw):
    got, gq, want, wq = fp8_layer(gpu, m, n, kb, hb.EXACT, seed=710 + m, **kw)
    assert np.array_equal(got, want)
    if gq is not None:
        assert np.array_equal(gq, wq)


def test_exact_batched(gpu):
    rng = np.random.default_rng(720)
    m, n, kb, layers = 36, 128, 6, 3
    a = [helpers.activations_fp8(rng, m, kb * 32)[1] for _ in range(layers)]
    w = [mxfp4_planes(rng, n, kb)[0][0] for _ in range(layers)]
    a_d, w_d = dev(np.concatenate(a)), dev(np.concatenate(w))
    c = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_d[i * len(a[0]):(i + 1) * len(a[0])],
                            [w_d[i * len(w[0]):(i + 1) * len(w[0])]], [0], c[i], mode=hb.EXACT,
                            a_fp8=True) for i in range(layers)]
    say("fp8 exact batched", dict(layers=layers))
    hb.linear_batched(descs, gpu)
    got = host(c).view(np.uint32)
    for i in range(layers):
        want, _ = oracle.linear(m, n, kb, a[i], [w[i]], [0], a_fp8=True)
        assert np.array_equal(got[i], want)


@pytest.mark.parametrize("m", [1, 16, 128, 1024])
def test_fast_config1_sweep(gpu, m):
    got, _, want, _ = fp8_layer(gpu, m, 960, 80, hb.FAST, seed=730 + m)
    check_fp8_fast(got, want, fp8_layer.abs_sums())


def test_fast_plain_141(gpu):
    got, _, want, _ = fp8_layer(gpu, 141, 960, 30, hb.FAST, seed=741)
    check_fp8_fast(got, want, fp8_layer.abs_sums())


def test_fast_ops_requantize(gpu):
    got, gq, want, wq = fp8_layer(gpu, 141, 960, 30, hb.FAST, per_channel, quantize=True,
                                  seed=740)
    helpers.check_fast(got, want, gq, wq)


def test_fast_out_of_window_scales_exact(gpu):
    """W scale bytes 40..60 (below the fast window): every tile is folded
    exactly, so the result is the exact one, bit for bit."""
    got, _, want, _ = fp8_layer(gpu, 50, 256, 12, hb.FAST, seed=750, w_lo=-87, w_hi=-67)
    assert np.array_equal(got, want)


def test_fp8_needs_one_mxfp4_plane(gpu):
    a = torch.zeros((16, 144), dtype=torch.uint8, device=DEV)
    w = torch.zeros((8 * 1, 144), dtype=torch.uint8, device=DEV)
    c = torch.zeros((4, 64), dtype=torch.float32, device=DEV)
    with pytest.raises(hb.HbError) as err:
        hb.linear(gpu, a=a, planes=[w, w], modes=[1, 2], c=c, m=4, n=64, kb_total=1, a_fp8=True)
    assert err.value.code == hb.HB_EINVAL and "MXFP8" in err.value.message


# ---- batches over weight panels: the streaming kernel ----

def fp8_batch(gpu, m, n, kb, layers, sets, onto=False, bad=None, seed=0, panels=True,
              pieces=None, tile_cols=320):
    """`layers` MXFP8 x MXFP4 layers (weights in panels, or DDR words) in
    one fast batched launch; layer i holds data set i % sets.  The oracle
    computes each set once and every layer holding it must equal it bit for
    bit.  bad = (layer, word): that layer's weights get one scale byte
    outside the fast window in DDR word `word` (the tile_cols-wide column
    tile holding it is recomputed by the exact fold, bitwise, in the middle
    of the workgroup's stream)."""
    rng = np.random.default_rng(seed)
    a_sets, w_sets, c_sets = [], [], []
    for _ in range(sets):
        a_sets.append(helpers.activations_fp8(rng, m, kb * 32)[1])
        w_sets.append(mxfp4_planes(rng, n, kb)[0][0])
        c_sets.append(helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None)
    set_of = [i % sets for i in range(layers)]
    w_bad = None
    if bad is not None:
        w_bad = w_sets[set_of[bad[0]]].copy()
        w_bad.reshape(-1, 144)[bad[1], 128 + 2] = 200
    pb = hb.panel_bytes(n, kb)
    a_d = torch.empty((layers,) + a_sets[0].shape, dtype=torch.uint8, device=DEV)
    w_p = torch.empty((layers, pb), dtype=torch.uint8, device=DEV)
    c_d = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    w_dev = [dev(w) for w in w_sets]
    if not panels:
        w_p = torch.empty((layers,) + w_sets[0].shape, dtype=torch.uint8, device=DEV)
    for i in range(layers):
        a_d[i].copy_(dev(a_sets[set_of[i]]))
        src = dev(w_bad) if bad is not None and i == bad[0] else w_dev[set_of[i]]
        if panels:
            hb.pack_weights(src, n, kb, w_p[i], ctx=gpu)
        else:
            w_p[i].copy_(src)
        if onto:
            c_d[i].copy_(dev(c_sets[set_of[i]].view(np.float32)))
    descs = [hb.linear_desc(m, n, kb, a_d[i], [w_p[i]], [0], c_d[i], mode=hb.FAST, panels=panels,
                            onto=onto, a_fp8=True, pieces=pieces) for i in range(layers)]
    torch.cuda.synchronize()
    say("fp8 batch", dict(m=m, n=n, kb=kb, layers=layers, sets=sets, onto=onto, bad=bad,
                          panels=panels, pieces=pieces))
    hb.linear_batched(descs, gpu)
    got = host(c_d).view(np.uint32)
    rep = {}
    for i in range(layers):
        if bad is not None and i == bad[0]:
            continue
        if set_of[i] in rep:
            assert np.array_equal(got[i], got[rep[set_of[i]]]), i
        else:
            rep[set_of[i]] = i
    for s in range(sets):
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_sets[s], [w_sets[s]], [0], onto=c_sets[s],
                                           a_fp8=True, pieces=pieces)
        if onto:
            g, w = got[rep[s]].view(np.float32).astype(np.float64), want.view(np.float32)
            row = np.abs(w.astype(np.float64)).max(axis=1, keepdims=True)
            assert (np.abs(g - w) <= 1e-5 * row).all()
        else:
            check_fp8_fast(got[rep[s]], want, fp8_abs_sums(m, n, kb, a_sets[s], w_sets[s]))
    if bad is not None:
        layer, word = bad
        s = set_of[layer]
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_sets[s], [w_bad], [0], onto=c_sets[s],
                                           a_fp8=True, pieces=pieces)
        c0 = (word // kb) * 8 // tile_cols * tile_cols
        cols = slice(c0, min(c0 + tile_cols, n))
        assert np.array_equal(got[layer][:, cols], want[:, cols])
        others = np.setdiff1d(np.arange(n), np.arange(n)[cols])
        assert np.array_equal(got[layer][:, others], got[rep[s]][:, others])


@pytest.mark.parametrize("m,layers,sets", [(1, 256, 5), (16, 256, 5), (128, 256, 7),
                                           (1024, 64, 3)])
def test_fast_batched_config1(gpu, m, layers, sets):
    """Config 1's sweep batched as bench.py times it: K = 2560, N = 960,
    768 tiles (1,536 at M = 1024) over 256 workgroups."""
    fp8_batch(gpu, m, 960, 80, layers, sets, seed=800 + m)


def test_fast_batched_onto_partial_panel(gpu):
    """From C, N = 200 (a partial last panel), odd block count, 300 tiles."""
    fp8_batch(gpu, 1000, 200, 7, 40, 3, onto=True, seed=810)


def test_fast_batched_exact_recompute_mid_stream(gpu):
    """One weight scale byte outside the window in layer 150's middle column
    tile: that tile is folded exactly, the rest of the stream is fast."""
    fp8_batch(gpu, 128, 960, 80, 256, 11, bad=(150, 50 * 80 + 41), seed=811)


# ---- batches of layers of up to 16 rows: the skinny kernel ----

@pytest.mark.parametrize("m,n,kb,panels,onto", [(5, 200, 7, True, True), (16, 256, 13, False, False),
                                                (1, 64, 1, True, False), (11, 960, 80, False, True)])
def test_skinny_batched(gpu, m, n, kb, panels, onto):
    """Ragged rows, a partial last panel, odd and single block counts (a
    K chunk's blocks past the end), over panels and DDR words, from C."""
    fp8_batch(gpu, m, n, kb, 24, 3, onto=onto, panels=panels, seed=820 + m)


@pytest.mark.parametrize("panels", [True, False])
def test_skinny_pieces(gpu, panels):
    """Two pieces, W blocks [9, 23) then [0, 9), over panels and DDR words."""
    fp8_batch(gpu, 16, 320, 23, 12, 2, panels=panels, pieces=[(9, 14), (0, 9)], seed=830)


def test_skinny_out_of_window_scale(gpu):
    """One weight scale byte outside the window: that workgroup's 64 columns
    are folded exactly (bitwise), every other one is fast."""
    fp8_batch(gpu, 16, 960, 80, 64, 5, bad=(40, 7 * 80 + 33), seed=831, tile_cols=64)
