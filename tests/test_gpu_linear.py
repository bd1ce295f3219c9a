"""hb_linear (the linear layer over DDR words, fused epilogue, requantize)
and hb_encode_mxint8 on an MI355X against the oracle.

Exact mode: bitwise.  Fast mode: the block products are exact and only the
FP32 accumulation order differs; tolerance per output row r:
    max_n |gpu[r][n] - ref[r][n]| <= 1e-5 * max_n |ref[r][n]|   (normwise)
and, per element, |gpu - ref| <= 2^-20 * sum_b |block value b|."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
import oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def make_layer(rng, m, n, k, w8, exp_lo=-10, exp_hi=-2):
    kb = (k + 31) // 32
    x, a = helpers.activations(rng, m, kb * 32)
    if w8:
        planes = list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32))))
        modes = [1, 2]
    else:
        code, e = helpers.mxfp4_weights(rng, n, kb * 32, exp_lo, exp_hi)
        planes, modes = [oracle.pack_wbuf(code, e)], [0]
    return kb, a, planes, modes


def run_linear(gpu, m, n, kb, a, planes, modes, ops=(), pieces=None, onto=None, tbuf=None,
               quantize=False, mode=hb.EXACT):
    say("linear", dict(m=m, n=n, kb=kb, planes=len(planes), ops=[o[0] for o in ops], pieces=pieces,
                       onto=onto is not None, quantize=quantize, mode=mode))
    a_d = dev(a)
    w_d = [dev(p) for p in planes]
    c_d = dev(onto.view(np.float32)) if onto is not None else torch.zeros((m, n), dtype=torch.float32, device=DEV)
    dev_ops = []
    for kind, arg in ops:
        if kind in (hb.EP_ADDP, hb.EP_MULP):
            dev_ops.append((kind, dev(arg.view(np.float32))))
        elif kind in (hb.EP_ACT_MUL, hb.EP_ADD):
            dev_ops.append((kind, dev(arg.view(np.float32))))
        else:
            dev_ops.append((kind, arg))
    tb = dev(tbuf.view(np.int64)) if tbuf is not None else None
    q_d = torch.zeros((((m + 3) // 4) * (n // 32), 144), dtype=torch.uint8, device=DEV) if quantize else None
    torch.cuda.synchronize()
    hb.linear(gpu, a=a_d, planes=w_d, modes=modes, c=c_d, m=m, n=n, kb_total=kb, pieces=pieces,
              onto=onto is not None, ops=dev_ops, tbuf=tb, q_out=q_d, mode=mode)
    return host(c_d).view(np.uint32), (host(q_d) if quantize else None)


def oracle_linear(m, n, kb, a, planes, modes, ops=(), pieces=None, onto=None, tbuf=None,
                  quantize=False):
    mp = (m + 3) // 4 * 4
    c0 = None
    if onto is not None:
        c0 = np.zeros((mp, n), np.uint32)
        c0[:m] = onto
    oops = []
    for kind, arg in ops:
        if kind in (hb.EP_ACT_MUL, hb.EP_ADD):
            pad = np.zeros((mp, n), np.uint32)
            pad[:m] = arg
            oops.append((kind, pad))
        else:
            oops.append((kind, arg))
    c, q = oracle.linear(mp, n, kb, a, planes, modes, pieces=pieces, c=c0, onto=onto is not None,
                         ops=oops, tbuf=tbuf, quantize=quantize)
    return c[:m], q


def assert_bits(got, want):
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{len(bad)} differ; first {bad[0]}: {got[tuple(bad[0])]:#x} vs {want[tuple(bad[0])]:#x}"


# ---- the workloads: W8 M=64 K=960 N=2560 + MULP + ADDP; MXFP4 K=2560 N=960 ----

def test_w8_layer_with_scale_and_bias(gpu):
    rng = np.random.default_rng(1)
    m, n, k = 64, 2560, 960
    kb, a, planes, modes = make_layer(rng, m, n, k, True)
    scale = np.asarray(rng.uniform(0.001, 0.02, n), np.float32).view(np.uint32)
    bias = np.asarray(rng.normal(0, 0.1, n), np.float32).view(np.uint32)
    ops = [(hb.EP_MULP, scale), (hb.EP_ADDP, bias)]
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, ops)
    want, _ = oracle_linear(m, n, kb, a, planes, modes, ops)
    assert_bits(got, want)


@pytest.mark.parametrize("m", [1, 16, 128])
def test_mxfp4_layer(gpu, m):
    rng = np.random.default_rng(2 + m)
    n, k = 960, 2560
    kb, a, planes, modes = make_layer(rng, m, n, k, False)
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    assert_bits(got, want)


def block_abs_sums(m, n, kb, a, planes, modes):
    """sum_b |block value| per output (the fast-mode error scale)."""
    qa = a.reshape(-1, kb, 144)
    tot = np.zeros((qa.shape[0] * 4, n))
    for plane, mode in zip(planes, modes):
        w = plane.reshape(n // 8, kb, 144)
        nib = np.empty((n // 8, kb, 8, 32), np.int64)
        nib[..., 0::2] = (w[:, :, :128] & 15).reshape(n // 8, kb, 8, 16)
        nib[..., 1::2] = (w[:, :, :128] >> 4).reshape(n // 8, kb, 8, 16)
        mag = np.array([0, 1, 2, 3, 4, 6, 8, 12])
        if mode == 0:
            v = np.where(nib & 8, -mag[nib & 7], mag[nib & 7])
        elif mode == 1:
            v = np.where(nib & 8, nib - 16, nib)
        else:
            v = nib
        bias = {0: -7, 1: -8, 2: -12}[mode]
        aq = qa[:, :, :128].view(np.int8).reshape(-1, kb, 4, 32).astype(np.int64)
        ea = qa[:, :, 128:132].astype(np.int64)
        ew = w[:, :, 128:136].astype(np.int64)
        for b in range(kb):
            s = np.einsum("qtk,gck->qtgc", aq[:, b], v[:, b]).reshape(-1, n)
            sc = (ea[:, b, :].reshape(-1, 1) - 127) + (ew[:, b, :].reshape(1, -1) - 127) + bias
            tot += np.abs(s) * np.exp2(sc.astype(np.float64))
    return tot[:m]


@pytest.mark.parametrize("m,w8,n,k", [(128, False, 960, 2560), (1024, False, 960, 2560),
                                      (64, True, 768, 768), (2048, True, 768, 768),
                                      (64, True, 2560, 960), (200, True, 2304, 768)])
def test_fast_mode_tolerance(gpu, m, w8, n, k):
    """MXFP4 at the K=2560 N=960 workload, W8 at the W8 workload (M=64 K=960
    N=2560) and at SigLIP-style shapes."""
    rng = np.random.default_rng(10 + m + n)
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, mode=hb.FAST)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    err = np.abs(g - w)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (err <= 1e-5 * row_scale).all(), float((err / row_scale).max())
    if m <= 128:
        assert (err <= 2.0 ** -20 * block_abs_sums(m, n, kb, a, planes, modes) + 1e-30).all()


@pytest.mark.parametrize("m,w8", [(1, False), (50, False), (128, False), (1, True), (50, True),
                                  (128, True)])
def test_fast_split_layer_with_epilogue(gpu, m, w8):
    """A single small fast-mode layer takes the K-split path with the
    element-parallel epilogue: pieces, onto, MULP and ADDP, requantize."""
    rng = np.random.default_rng(70 + m + 1000 * w8)
    n, k = 320, 1280
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    onto = helpers.random_fp32_words(rng, (m, n), 120, 130)
    scale = helpers.random_fp32_words(rng, (n,), 117, 122)
    bias = helpers.random_fp32_words(rng, (n,), 118, 124)
    ops = [(hb.EP_MULP, scale), (hb.EP_ADDP, bias)]
    pieces = [(24, 16), (0, 17), (17, 7)]
    got, gq = run_linear(gpu, m, n, kb, a, planes, modes, ops, pieces=pieces, onto=onto,
                         quantize=True, mode=hb.FAST)
    want, wq = oracle_linear(m, n, kb, a, planes, modes, ops, pieces=pieces, onto=onto,
                             quantize=True)
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())
    # requantized bytes: equal except where the fp32 values straddle a rounding step
    gqb = gq.reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
    wqb = wq.reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
    assert np.abs(gqb - wqb).max() <= 1 and (gqb != wqb).mean() < 0.01
    assert np.array_equal(gq.reshape(-1, 144)[:, 128:], wq.reshape(-1, 144)[:, 128:]) or \
        (gq.reshape(-1, 144)[:, 128:132] != wq.reshape(-1, 144)[:, 128:132]).mean() < 0.01


@pytest.mark.parametrize("mode", [hb.EXACT, hb.FAST])
def test_narrow_layer_many_rows(gpu, mode):
    """The SparseDrive-S stage-1 3x3 im2col shape (K=576, N=64: one partly
    used column tile) on 1000 rows, a slice of its 67,584."""
    rng = np.random.default_rng(80)
    m, n, k = 1000, 64, 576
    kb, a, planes, modes = make_layer(rng, m, n, k, False)
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, mode=mode)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    if mode == hb.EXACT:
        assert_bits(got, want)
    else:
        g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
        row_scale = np.abs(w).max(axis=1, keepdims=True)
        assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())


@pytest.mark.parametrize("w8", [False, True])
def test_pieces_and_onto(gpu, w8):
    rng = np.random.default_rng(20 + w8)
    m, n, k = 96, 256, 640
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    onto = helpers.random_fp32_words(rng, (m, n), 120, 130)
    pieces = [(12, 8), (0, 5), (5, 7)]
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, pieces=pieces, onto=onto)
    want, _ = oracle_linear(m, n, kb, a, planes, modes, pieces=pieces, onto=onto)
    assert_bits(got, want)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_epilogue_ops_and_requantize(gpu, act):
    rng = np.random.default_rng(30)
    m, n, k = 64, 512, 256
    kb, a, planes, modes = make_layer(rng, m, n, k, False, -6, 0)
    tbuf = helpers.activation_table(act)
    up = helpers.random_fp32_words(rng, (m, n), 120, 130)
    res = helpers.random_fp32_words(rng, (m, n), 118, 128)
    vec = helpers.random_fp32_words(rng, (n,), 120, 128)
    imm = int(helpers.random_fp32_words(rng, (1,), 124, 128)[0])
    for ops in ([(hb.EP_ACT, None)], [(hb.EP_ACT_MUL, up)], [(hb.EP_RELU, None), (hb.EP_SCALE, imm)],
                [(hb.EP_MULP, vec), (hb.EP_ADD, res), (hb.EP_COPY, None)],
                [(hb.EP_ADDP, vec), (hb.EP_ACT, None), (hb.EP_MULP, vec)]):
        for quantize in (False, True):
            got, gq = run_linear(gpu, m, n, kb, a, planes, modes, ops, tbuf=tbuf, quantize=quantize)
            want, wq = oracle_linear(m, n, kb, a, planes, modes, ops, tbuf=tbuf, quantize=quantize)
            assert_bits(got, want)
            if quantize:
                assert np.array_equal(gq, wq)


@pytest.mark.parametrize("m", [1, 3, 5, 30, 37])
def test_rows_not_a_multiple_of_four(gpu, m):
    rng = np.random.default_rng(40 + m)
    n, k = 320, 384
    kb, a, planes, modes = make_layer(rng, m, n, k, m % 2 == 0)
    res = helpers.random_fp32_words(rng, (m, n), 118, 128)
    ops = [(hb.EP_ADD, res)]
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, ops)
    want, _ = oracle_linear(m, n, kb, a, planes, modes, ops)
    assert_bits(got, want)


def test_extreme_scales_exact(gpu):
    rng = np.random.default_rng(50)
    m, n, k = 64, 128, 256
    kb, a, planes, modes = make_layer(rng, m, n, k, False, -127, 127)
    a = a.copy()
    a.reshape(-1, 144)[::7, 128] = 1      # tiny activation scales in some words
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    assert_bits(got, want)


def test_batched_layers(gpu):
    rng = np.random.default_rng(60)
    layers, m, n, k = 5, 128, 192, 512
    kb = k // 32
    data = [make_layer(rng, m, n, k, False) for _ in range(layers)]
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = dev(np.stack([d[2][0] for d in data]))
    c_all = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], [0], c_all[i]) for i in range(layers)]
    torch.cuda.synchronize()
    say("batched", layers)
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    for i, d in enumerate(data):
        want, _ = oracle_linear(m, n, kb, d[1], d[2], d[3])
        assert_bits(got[i], want)


@pytest.mark.parametrize("w8,mode,quantize", [(True, hb.EXACT, False), (False, hb.EXACT, True),
                                              (False, hb.FAST, False), (True, hb.FAST, True)])
def test_batched_layers_with_epilogue(gpu, w8, mode, quantize):
    """Per-layer MULP scale and ADDP bias vectors at a uniform stride, as in
    the W8 workload (per-channel scale and bias), batched into one launch."""
    rng = np.random.default_rng(61 + w8)
    layers, m, n, k = 4, 64, 256, 320
    data = [make_layer(rng, m, n, k, w8) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    scale = np.stack([helpers.random_fp32_words(rng, (n,), 117, 122) for _ in range(layers)])
    bias = np.stack([helpers.random_fp32_words(rng, (n,), 118, 124) for _ in range(layers)])
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = [dev(np.stack([d[2][p] for d in data])) for p in range(len(modes))]
    s_all, b_all = dev(scale.view(np.float32)), dev(bias.view(np.float32))
    c_all = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    nb = n // 32
    q_all = (torch.zeros((layers, m // 4 * nb, 144), dtype=torch.uint8, device=DEV)
             if quantize else None)
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w[i] for w in w_all], modes, c_all[i],
                            ops=[(hb.EP_MULP, s_all[i]), (hb.EP_ADDP, b_all[i])],
                            q_out=q_all[i] if quantize else None, mode=mode)
             for i in range(layers)]
    torch.cuda.synchronize()
    say("batched with epilogue", dict(layers=layers, w8=w8, mode=mode, quantize=quantize))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    gq = host(q_all) if quantize else None
    for i, d in enumerate(data):
        ops = [(hb.EP_MULP, scale[i]), (hb.EP_ADDP, bias[i])]
        want, wq = oracle_linear(m, n, kb, d[1], d[2], d[3], ops, quantize=quantize)
        if mode == hb.EXACT:
            assert_bits(got[i], want)
            if quantize:
                assert np.array_equal(gq[i], wq)
        else:
            g = got[i].view(np.float32).astype(np.float64)
            w = want.view(np.float32).astype(np.float64)
            row_scale = np.abs(w).max(axis=1, keepdims=True)
            assert (np.abs(g - w) <= 1e-5 * row_scale).all()
            if quantize:
                gqb = gq[i].reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
                wqb = wq.reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
                assert np.abs(gqb - wqb).max() <= 1 and (gqb != wqb).mean() < 0.01


@pytest.mark.parametrize("w8", [False, True])
def test_fast_batched_pieces_and_onto(gpu, w8):
    """Fast mode over a piece list (the multi-piece kernel), starting from C,
    with rows and columns that leave partial tiles, batched.  Step 3 pairs
    block 19 with block 0 (a step's blocks out of memory order)."""
    rng = np.random.default_rng(63 + w8)
    layers, m, n, k = 3, 160, 320, 640
    data = [make_layer(rng, m, n, k, w8) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    pieces = [(13, 7), (0, 5), (5, 8)]
    onto = np.stack([helpers.random_fp32_words(rng, (m, n), 120, 130) for _ in range(layers)])
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = [dev(np.stack([d[2][p] for d in data])) for p in range(len(modes))]
    c_all = dev(onto.view(np.float32))
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w[i] for w in w_all], modes, c_all[i],
                            pieces=pieces, onto=True, mode=hb.FAST) for i in range(layers)]
    torch.cuda.synchronize()
    say("fast batched pieces onto", dict(layers=layers, w8=w8))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    for i, d in enumerate(data):
        want, _ = oracle_linear(m, n, kb, d[1], d[2], d[3], pieces=pieces, onto=onto[i])
        g = got[i].view(np.float32).astype(np.float64)
        w = want.view(np.float32).astype(np.float64)
        row_scale = np.abs(w).max(axis=1, keepdims=True)
        assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())


@pytest.mark.parametrize("m,k,pieces", [(130, 416, None), (257, 640, [(11, 3), (0, 6)])])
def test_fast_batched_odd_blocks_partial_tiles(gpu, m, k, pieces):
    """MXFP4 layers of more than 64 rows (128-row tiles) with an odd number
    of K blocks (the last step's second block is padding), rows not a
    multiple of 4 and a partly used last column tile, batched.  With the
    piece list, step 1 pairs block 13 with block 0."""
    rng = np.random.default_rng(66 + m)
    layers, n = 3, 296
    data = [make_layer(rng, m, n, k, False) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = dev(np.stack([d[2][0] for d in data]))
    c_all = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], modes, c_all[i], pieces=pieces,
                            mode=hb.FAST) for i in range(layers)]
    torch.cuda.synchronize()
    say("fast batched odd blocks", dict(m=m, k=k, pieces=pieces))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    for i, d in enumerate(data):
        want, _ = oracle_linear(m, n, kb, d[1], d[2], d[3], pieces=pieces)
        g = got[i].view(np.float32).astype(np.float64)
        w = want.view(np.float32).astype(np.float64)
        row_scale = np.abs(w).max(axis=1, keepdims=True)
        assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())


def test_fast_many_tiles_per_workgroup(gpu):
    """More 128-row MXFP4 tiles than CUs (300 tiles over 25 layers): each
    workgroup runs several tiles back to back.  Starting from C, an odd
    number of K blocks, a partly used last column tile, and one row tile of
    one layer with an out-of-window scale byte (that tile exact, bit for
    bit; its neighbours within tolerance)."""
    rng = np.random.default_rng(67)
    layers, m, n, k = 25, 260, 1000, 160
    data = [make_layer(rng, m, n, k, False) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    bad_layer = 12
    a_bad = data[bad_layer][1].copy()
    a_bad.reshape(-1, kb, 144)[5, 2, 128] = 60  # row 20 (row tile 0), block 2
    data[bad_layer] = (kb, a_bad, data[bad_layer][2], modes)
    onto = np.stack([helpers.random_fp32_words(rng, (m, n), 120, 130) for _ in range(layers)])
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = dev(np.stack([d[2][0] for d in data]))
    c_all = dev(onto.view(np.float32))
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], modes, c_all[i], onto=True,
                            mode=hb.FAST) for i in range(layers)]
    torch.cuda.synchronize()
    say("fast many tiles", dict(layers=layers, m=m, n=n, k=k))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    for i, d in enumerate(data):
        want, _ = oracle_linear(m, n, kb, d[1], d[2], d[3], onto=onto[i])
        if i == bad_layer:
            assert_bits(got[i][:128], want[:128])
        g = got[i].view(np.float32).astype(np.float64)
        w = want.view(np.float32).astype(np.float64)
        row_scale = np.abs(w).max(axis=1, keepdims=True)
        assert (np.abs(g - w) <= 1e-5 * row_scale).all(), (i, float((np.abs(g - w) / row_scale).max()))


@pytest.mark.parametrize("w8", [False, True])
def test_fast_out_of_window_scales_recompute_exactly(gpu, w8):
    """Row tiles whose scale bytes leave the fast path's window recompute
    with the NPU's ordered fold, bit for bit; the other tiles stay within
    the fast-mode tolerance."""
    rng = np.random.default_rng(64 + w8)
    m, n, k = 256, 512, 384
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    a = a.copy()
    a.reshape(m // 4, kb, 144)[:32, 3, 128] = 60   # rows 0..127: an out-of-window scale byte
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, mode=hb.FAST)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    assert_bits(got[:128], want[:128])
    g, w = got[128:].view(np.float32).astype(np.float64), want[128:].view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all()


@pytest.mark.parametrize("w8", [False, True])
def test_fast_k_split_64_row_tiles_out_of_window(gpu, w8):
    """1100 x 512 x 512: more than 1,024 rows on 36 tiles of 64 rows, so K
    splits whose partial sums and window flags go to the epilogue kernel.
    Rows 64..127 (the second row tile) carry an out-of-window scale byte:
    that row tile recomputes exactly, bit for bit; the rest stays within
    the fast-mode tolerance."""
    rng = np.random.default_rng(66 + w8)
    m, n, k = 1100, 512, 512
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    a = a.copy()
    a.reshape(-1, kb, 144)[16:32, 3, 128] = 60   # rows 64..127
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, mode=hb.FAST)
    want, _ = oracle_linear(m, n, kb, a, planes, modes)
    assert_bits(got[64:128], want[64:128])
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all()


def test_fast_96_row_tiles_out_of_window(gpu):
    """4512 x 960 x 960 MXFP4: 188 tiles of 96 rows (128-row tiles would
    leave CUs idle, 64-row tiles take two rounds).  Rows 96..191 (the second
    row tile) carry an out-of-window scale byte: that row tile recomputes
    exactly, bit for bit; the rest stays within the fast-mode tolerance."""
    rng = np.random.default_rng(67)
    m, n, k = 4512, 960, 960
    kb, a, planes, modes = make_layer(rng, m, n, k, False)
    a = a.copy()
    a.reshape(-1, kb, 144)[24:48, 5, 128] = 60   # rows 96..191
    got, _ = run_linear(gpu, m, n, kb, a, planes, modes, mode=hb.FAST)
    want, _ = helpers.oracle_linear_mt(m, n, kb, a, planes, modes)
    assert_bits(got[96:192], want[96:192])
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all()


@pytest.mark.parametrize("w8", [False, True])
def test_fast_skinny_out_of_window_and_onto(gpu, w8):
    """A layer of at most 64 rows (one workgroup holds all rows): a weight
    scale byte out of the window makes that workgroup's columns exact, bit
    for bit; the rest, started from C with MULP and requantize, stays within
    tolerance."""
    rng = np.random.default_rng(65 + w8)
    m, n, k = 40, 512, 736
    kb, a, planes, modes = make_layer(rng, m, n, k, w8)
    planes = [p.copy() for p in planes]
    for p in planes:
        p.reshape(n // 8, kb, 144)[0, 5, 128] = 200    # column 0, block 5: out of the window
    onto = helpers.random_fp32_words(rng, (m, n), 120, 130)
    scale = helpers.random_fp32_words(rng, (n,), 117, 122)
    ops = [(hb.EP_MULP, scale)]
    got, gq = run_linear(gpu, m, n, kb, a, planes, modes, ops, onto=onto, quantize=True,
                         mode=hb.FAST)
    want, wq = oracle_linear(m, n, kb, a, planes, modes, ops, onto=onto, quantize=True)
    assert_bits(got[:, :32], want[:, :32])  # within the exact workgroup's columns
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())


def test_batched_rejects_mismatched_layers(gpu):
    rng = np.random.default_rng(62)
    m, n, k = 32, 64, 64
    kb, a, planes, modes = make_layer(rng, m, n, k, False)
    a_all = dev(np.stack([a] * 3))
    w_all = dev(np.stack([planes[0]] * 3))
    c_all = torch.zeros((3, m, n), dtype=torch.float32, device=DEV)
    vec = torch.zeros((3, n), dtype=torch.float32, device=DEV)
    good = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], modes, c_all[i],
                           ops=[(hb.EP_MULP, vec[i])]) for i in range(3)]
    cases = {
        "op vector stride": [good[0], good[1],
                             hb.linear_desc(m, n, kb, a_all[2], [w_all[2]], modes, c_all[2],
                                            ops=[(hb.EP_MULP, vec[0])])],
        "op kind": [good[0], good[1],
                    hb.linear_desc(m, n, kb, a_all[2], [w_all[2]], modes, c_all[2],
                                   ops=[(hb.EP_ADDP, vec[2])])],
        "pieces": [good[0], good[1],
                   hb.linear_desc(m, n, kb, a_all[2], [w_all[2]], modes, c_all[2],
                                  pieces=[(1, 1)], ops=[(hb.EP_MULP, vec[2])])],
    }
    for name, descs in cases.items():
        say("batched mismatch", name)
        with pytest.raises(hb.HbError):
            hb.linear_batched(descs, gpu)
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows,cols", [(1, 32), (4, 960), (7, 100), (64, 2560)])
def test_encode_mxint8(gpu, rows, cols):
    rng = np.random.default_rng(rows * cols)
    x = (rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-20, 20, (rows, cols)))).astype(np.float32)
    x[0, :5] = [0.0, -0.0, 1e-40, -1e-39, 3.0]
    say("encode", rows, cols)
    x_d = dev(x)
    quads, blocks = (rows + 3) // 4, (cols + 31) // 32
    out = torch.full((quads * blocks, 144), 0xAB, dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()
    hb.encode_mxint8(x_d, rows, cols, out, gpu)
    got = host(out)
    xp = np.zeros((quads * 4, cols), np.float32)
    xp[:rows] = x
    q, e = oracle.encode_mxint8(oracle.f32_bits(xp))
    assert np.array_equal(got, oracle.pack_abuf(q, e))


def test_encode_rejects_non_finite(gpu):
    x_d = dev(np.array([[1.0, np.inf, 2.0]], np.float32))
    out = torch.zeros((1, 144), dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()
    with pytest.raises(hb.HbError):
        hb.encode_mxint8(x_d, 1, 3, out, gpu)


# ---- A pieces with their own place and stride (LinearPiece.a / a_stride) ----

def a_words_view(a, quads, words):
    return a.reshape(quads, words, 144)


@pytest.mark.parametrize("mode", [hb.EXACT, hb.FAST])
@pytest.mark.parametrize("m,w8", [(50, True), (150, True), (128, False), (8, False)])
def test_a_stride_selects_a_head(gpu, mode, m, w8):
    """One piece whose A words are head h's 2 blocks inside a projection
    output of 30 words per quad (kernels.cpp:155-170: Q per head, a_stride =
    the row's words).  Expected: the oracle on the head's words copied out."""
    rng = np.random.default_rng(200 + m + 7 * w8 + mode)
    n, kb, row_words, head = 256, 2, 30, 11
    quads = (m + 3) // 4
    _, q_all = helpers.activations(rng, m, row_words * 32)
    if w8:
        planes, modes = list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32)))), [1, 2]
    else:
        code, e = helpers.mxfp4_weights(rng, n, kb * 32)
        planes, modes = [oracle.pack_wbuf(code, e)], [0]
    a_head = np.ascontiguousarray(a_words_view(q_all, quads, row_words)[:, 2 * head: 2 * head + 2])
    want, _ = oracle_linear(m, n, kb, a_head.reshape(-1, 144), planes, modes)
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    say("a_stride head", dict(m=m, w8=w8, mode=mode))
    hb.linear(gpu, a=dev(q_all), planes=[dev(p) for p in planes], modes=modes, c=c_d, m=m, n=n,
              kb_total=kb, pieces=[(0, kb, 2 * head)], a_stride=row_words, mode=mode)
    got = host(c_d).view(np.uint32)
    if mode == hb.EXACT:
        assert_bits(got, want)
    else:
        g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
        row_scale = np.abs(w).max(axis=1, keepdims=True)
        assert (np.abs(g - w) <= 1e-5 * row_scale).all()


@pytest.mark.parametrize("mode", [hb.EXACT, hb.FAST])
def test_a_pieces_at_different_places_chain(gpu, mode):
    """The output projection over head-major MXINT8 attention outputs
    ([head][quad][2 words]): 15 pieces, piece h = W blocks [2h, 2h+2) and A
    words from head h's own array (a_stride 2, a_word h * quads * 2), with
    MULP, ADDP and requantize, batched over 2 layers.  The pieces sit at
    different offsets, so the layer runs as a chain of launches; expected:
    the oracle on the words gathered into [quad][30]."""
    rng = np.random.default_rng(300 + mode)
    layers, m, n, heads = 2, 50, 960, 15
    quads, kb = (m + 3) // 4, 2 * heads
    data = []
    for _ in range(layers):
        per_head = [helpers.activations(rng, m, 64)[1].reshape(quads, 2, 144) for _ in range(heads)]
        a_std = np.concatenate(per_head, axis=1).reshape(-1, 144)
        a_hm = np.stack(per_head).reshape(-1, 144)
        planes = list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32))))
        data.append((a_std, a_hm, planes))
    scale = helpers.random_fp32_words(rng, (n,), 117, 122)
    bias = helpers.random_fp32_words(rng, (n,), 118, 124)
    a_d = dev(np.stack([d[1] for d in data]))
    w_d = [dev(np.stack([d[2][p] for d in data])) for p in range(2)]
    c_d = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    q_d = torch.zeros((layers, quads * n // 32, 144), dtype=torch.uint8, device=DEV)
    ops = [(hb.EP_MULP, dev(scale.view(np.float32))), (hb.EP_ADDP, dev(bias.view(np.float32)))]
    pieces = [(2 * h, 2, h * quads * 2) for h in range(heads)]
    descs = [hb.linear_desc(m, n, kb, a_d[i], [w[i] for w in w_d], [1, 2], c_d[i], pieces=pieces,
                            ops=ops, q_out=q_d[i], mode=mode, a_stride=2) for i in range(layers)]
    torch.cuda.synchronize()
    say("a pieces chain", dict(mode=mode))
    hb.linear_batched(descs, gpu)
    got, gq = host(c_d).view(np.uint32), host(q_d)
    for i, (a_std, _, planes) in enumerate(data):
        want, wq = oracle_linear(m, n, kb, a_std, planes, [1, 2], ops=[(hb.EP_MULP, scale),
                                 (hb.EP_ADDP, bias)], quantize=True)
        if mode == hb.EXACT:
            assert_bits(got[i], want)
            assert np.array_equal(gq[i], wq.reshape(-1, 144)[: quads * n // 32])
        else:
            g, w = got[i].view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
            row_scale = np.abs(w).max(axis=1, keepdims=True)
            assert (np.abs(g - w) <= 1e-5 * row_scale).all()


def test_a_stride_rejects_offsets_past_4gib(gpu):
    a = torch.zeros((16, 144), dtype=torch.uint8, device=DEV)
    w = torch.zeros((1, 144), dtype=torch.uint8, device=DEV)
    c = torch.zeros((8, 8), dtype=torch.float32, device=DEV)
    with pytest.raises(hb.HbError) as e:
        hb.linear(gpu, a=a, planes=[w], modes=[0], c=c, m=8, n=8, kb_total=1,
                  pieces=[(0, 1, 1 << 25)], a_stride=1)
    assert e.value.code == hb.HB_EINVAL
