"""Weight panels on an MI355X: hb_pack_weights against the oracle's
restatement of the layout byte for byte, hb_unpack_weights back to the DDR
words (tools/compiler/tensors.cpp:66-90) bit for bit, and linear layers over
panels against the oracle's layer over the same weights as DDR words
(tools/iss/gemm_array.cpp:112-149 folded as tools/compiler/kernels.cpp:
343-395): exact mode bitwise, fast mode within the fast-mode tolerance, on
every kernel route that reads panels (the panel streaming kernel batched and
persistent, a partial last panel and odd block counts, from C, out-of-window
scale bytes; the skinny kernel for batches of up to 16 rows; the single-launch
split kernel for one layer of up to 160 rows, with ops, requantize and W8
planes; the 128-row tile kernel and its K-split path; the exact tile
kernel)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
import oracle
from test_gpu_bench_routes import (DEV, batched_layers, dev, host, per_channel, say, single_layer,
                                    to_panels)

pytestmark = pytest.mark.gpu


def ddr_words(rng, n, kb):
    w = rng.integers(0, 256, (n // 8, kb, 144), dtype=np.uint8)
    w[:, :, 136:] = 0
    return w.reshape(-1, 144)


@pytest.mark.parametrize("n,kb", [(8, 1), (72, 3), (960, 80), (2048, 23), (2560, 30)])
def test_pack_and_unpack(gpu, n, kb):
    rng = np.random.default_rng(n + kb)
    w = ddr_words(rng, n, kb)
    say("pack", dict(n=n, kb=kb))
    w_d = dev(w)
    p_d = torch.full((hb.panel_bytes(n, kb),), 0xA5, dtype=torch.uint8, device=DEV)
    hb.pack_weights(w_d, n, kb, p_d, ctx=gpu)
    assert np.array_equal(host(p_d), oracle.pack_panels(w, n, kb))
    back = torch.full_like(w_d, 0x5A)
    hb.unpack_weights(p_d, n, kb, back, ctx=gpu)
    assert np.array_equal(host(back), w)


def test_pack_rejects_bad_arguments(gpu):
    buf = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    for args in ((buf, 12, 3, buf), (buf, 8, 0, buf), (buf[1:], 8, 1, buf)):
        with pytest.raises(hb.HbError) as err:
            hb.pack_weights(*args, ctx=gpu)
        assert err.value.code == hb.HB_EINVAL


# ---- the panel streaming kernel (fast, plain MXFP4, more than 64 rows) ----

@pytest.mark.parametrize("layers,check", [(2, (0, 1)), (80, (0, 1, 37, 79))])
def test_headline_shape(gpu, layers, check):
    batched_layers(gpu, 128, 960, 80, layers, check, hb.FAST, seed=layers + 500, panels=True)


def test_m1024_batched(gpu):
    batched_layers(gpu, 1024, 960, 80, 10, (0, 9), hb.FAST, seed=501, panels=True)


@pytest.mark.parametrize("m,n,kb", [(128, 72, 3), (200, 320, 23), (131, 200, 5)])
def test_partial_panels_odd_blocks(gpu, m, n, kb):
    """n not a multiple of 64 (a partial last panel; with n = 72 three of a
    tile's four waves have no columns), odd block counts (the last step's
    second block is padding), rows past a 128-row tile, many tiles."""
    batched_layers(gpu, m, n, kb, 40, (0, 17, 39), hb.FAST, seed=m + n + kb, panels=True)


def test_onto_and_all_codes(gpu):
    batched_layers(gpu, 128, 256, 12, 3, range(3), hb.FAST, all_codes=True, seed=502,
                   panels=True, onto=True)


def test_out_of_window_scales_take_the_exact_fold(gpu):
    batched_layers(gpu, 128, 320, 10, 4, range(4), hb.FAST, seed=503, panels=True,
                   bad_scales=True)


def test_single_layer_many_tiles(gpu):
    single_layer(gpu, 16384, 64, 18, False, hb.FAST, seed=504, bound=True, panels=True)


# ---- the panel streaming kernel's persistent schedule: more tiles than CUs ----
#
# With more tiles than the grid's 256 workgroups every workgroup runs several
# tiles in sequence from one load ring: the next tile's first steps are in
# flight while the current tile's last steps compute, and its accumulators
# are stored (or recomputed exactly) between them.  These launches use the
# bench's shapes.  Layer i holds data set i % sets (sets coprime to the
# schedule's strides), so every tile of the launch is checked: the oracle
# computes each data set once, and every other layer holding the same data set
# must equal that layer bit for bit (the kernel is deterministic per tile).

def replicated_layers(gpu, m, n, kb, layers, sets, check, onto=False, bad=None, seed=0):
    """`layers` MXFP4 layers over panels in one batched fast launch; layer i
    holds data set i % sets.  `check`: the data sets the oracle computes (the
    rest are compared bitwise with their representative only when checked).
    bad = (layer, word, byte): that layer gets a data set of its own, equal to
    its set's but with one weight scale byte set outside the fast window (its
    tile is recomputed by the exact fold in the middle of the workgroup's
    stream)."""
    rng = np.random.default_rng(seed)
    a_sets, w_sets, c_sets = [], [], []
    for _ in range(sets):
        a_sets.append(helpers.activations(rng, m, kb * 32)[1])
        w_sets.append(mxfp4_w(rng, n, kb))
        c_sets.append(helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None)
    set_of = [i % sets for i in range(layers)]
    w_bad = None
    if bad is not None:
        layer, word, byte = bad
        w_bad = w_sets[set_of[layer]].copy()
        w_bad.reshape(-1, 144)[word, 128 + byte] = 200
    pb = hb.panel_bytes(n, kb)
    a_d = torch.empty((layers,) + a_sets[0].shape, dtype=torch.uint8, device=DEV)
    w_p = torch.empty((layers, pb), dtype=torch.uint8, device=DEV)
    c_d = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    w_dev = [dev(w) for w in w_sets]
    wb_dev = dev(w_bad) if w_bad is not None else None
    for i in range(layers):
        a_d[i].copy_(dev(a_sets[set_of[i]]))
        src = wb_dev if bad is not None and i == bad[0] else w_dev[set_of[i]]
        hb.pack_weights(src, n, kb, w_p[i], ctx=gpu)
        if onto:
            c_d[i].copy_(dev(c_sets[set_of[i]].view(np.float32)))
    descs = [hb.linear_desc(m, n, kb, a_d[i], [w_p[i]], [0], c_d[i], mode=hb.FAST, panels=True,
                            onto=onto) for i in range(layers)]
    torch.cuda.synchronize()
    tiles = layers * ((m + 127) // 128) * ((n + 319) // 320)
    say("stream schedule", dict(m=m, n=n, kb=kb, layers=layers, sets=sets, tiles=tiles,
                                onto=onto, bad=bad))
    hb.linear_batched(descs, gpu)
    got = host(c_d).view(np.uint32)
    rep = {}
    for i in range(layers):
        if bad is not None and i == bad[0]:
            continue
        s = set_of[i]
        if s in rep:
            assert np.array_equal(got[i], got[rep[s]]), (i, rep[s])
        else:
            rep[s] = i
    for s in check:
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_sets[s], [w_sets[s]], [0], onto=c_sets[s])
        helpers.check_fast(got[rep[s]], want,
                           bound=None if onto else
                           helpers.block_abs_sums(m, n, kb, a_sets[s], [w_sets[s]], [0]))
    if bad is not None:
        layer = bad[0]
        s = set_of[layer]
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_sets[s], [w_bad], [0], onto=c_sets[s])
        helpers.check_fast(got[layer], want)
        # the tile holding the bad byte is recomputed bitwise; the layer's
        # other tiles are the plain fast result
        if not onto:
            exact_cols = _tile_cols_of_word(n, kb, bad[1])
            ex, _ = helpers.oracle_linear_mt(m, n, kb, a_sets[s], [w_bad], [0])
            assert np.array_equal(got[layer][:, exact_cols], ex[:, exact_cols])
            other = np.setdiff1d(np.arange(n), np.arange(n)[exact_cols])
            assert np.array_equal(got[layer][:, other], got[rep[s]][:, other])
    return got


def mxfp4_w(rng, n, kb):
    code, e = helpers.mxfp4_weights(rng, n, kb * 32)
    return oracle.pack_wbuf(code, e)


def _tile_cols_of_word(n, kb, word):
    """The 320-column tile holding DDR weight word `word` (group word // kb)."""
    c0 = (word // kb) * 8 // 320 * 320
    return slice(c0, min(c0 + 320, n))


def test_stream_headline_launch(gpu):
    """The bench's launch: M=128 K=2560 N=960, 256 layers, 768 tiles (3 per
    workgroup); 17 data sets, every layer checked."""
    replicated_layers(gpu, 128, 960, 80, 256, 17, range(17), seed=600)


def test_stream_m1024_launch(gpu):
    """The M=1024 sweep's launch: 64 layers, 1,536 tiles (6 per workgroup)."""
    replicated_layers(gpu, 1024, 960, 80, 64, 5, range(5), seed=601)


def test_stream_many_tiles_onto(gpu):
    """From C, 300 tiles: each tile's accumulators start from its C words
    while the previous tile's last steps are still in the ring."""
    replicated_layers(gpu, 128, 960, 80, 100, 7, range(7), onto=True, seed=602)


def test_stream_many_tiles_exact_recompute_mid_stream(gpu):
    """One weight scale byte outside the window in the middle column tile of
    layer 150 of 256 (tile 451 of 768): that tile is recomputed by the exact
    fold while the ring streams on, and the workgroup's next tile follows."""
    kb = 80
    word = 50 * kb + 40  # column group 50 (column tile 1), block 40
    replicated_layers(gpu, 128, 960, kb, 256, 13, range(3), bad=(150, word, 3), seed=603)


def test_stream_many_tiles_partial_panel(gpu):
    """N=200 (a partial last panel, three of a tile's five panels past the
    layer) at M=1024 over 40 layers: 320 tiles."""
    replicated_layers(gpu, 1024, 200, 5, 40, 3, range(3), seed=604)


# ---- the other kernels over panels ----

@pytest.mark.parametrize("m", [1, 16])
def test_skinny_batched(gpu, m):
    batched_layers(gpu, m, 960, 80, 6, range(6), hb.FAST, seed=505 + m, panels=True)


@pytest.mark.parametrize("m,w8", [(50, False), (16, True)])
def test_skinny_single(gpu, m, w8):
    single_layer(gpu, m, 720, 23, w8, hb.FAST, seed=507 + m, bound=True, panels=True)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_w8_ops_requantize(gpu, mode):
    """W8 planes as panels with MULP, ADDP, GELU and the requantize: the
    128-row tile kernel (fast) and the exact tile kernel."""
    single_layer(gpu, 512, 3072, 24, True, mode, lambda r, m, n: per_channel(r, n, True),
                 quantize=True, tbuf=helpers.activation_table("gelu"), seed=509, panels=True)


@pytest.mark.parametrize("m", [141, 200])
@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_small_layer_split_with_ops(gpu, mode, m):
    """One small layer with the residual ADD: at 141 rows the single-launch
    split kernel (fast), at 200 rows the 128-row tile kernel's K splits and
    the epilogue kernel (fast); the deferred exact epilogue in exact mode."""
    single_layer(gpu, m, 320, 30, False, mode,
                 lambda r, m, n: [(hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))],
                 seed=510 + m, panels=True)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_pieces_over_panels(gpu, mode):
    """A piece list (fold order pieces, then blocks) over panels."""
    single_layer(gpu, 96, 256, 20, False, mode, seed=511, panels=True,
                 pieces=[(12, 8), (0, 5), (5, 7)])


@pytest.mark.parametrize("m,w8", [(128, False), (1000, True), (64, False)])
def test_exact_over_panels(gpu, m, w8):
    single_layer(gpu, m, 320, 13, w8, hb.EXACT, seed=512 + m, panels=True)


# ---- the streaming kernel's epilogue: ops, C and the requantize ----

def all_ops(rng, m, n):
    """Every fast epilogue op kind: MULP, ADDP, SCALE, ADD, ACT (the table's
    activation), ACT_MUL, RELU, COPY."""
    vec = lambda lo, hi: np.asarray(rng.uniform(lo, hi, n), np.float32).view(np.uint32)
    return [(hb.EP_MULP, vec(0.5, 2.0)), (hb.EP_ADDP, vec(-0.1, 0.1)),
            (hb.EP_SCALE, int(np.float32(0.75).view(np.uint32))),
            (hb.EP_ADD, helpers.random_fp32_words(rng, (m, n), 118, 126)),
            (hb.EP_ACT, None),
            (hb.EP_ACT_MUL, helpers.random_fp32_words(rng, (m, n), 124, 128)),
            (hb.EP_RELU, None), (hb.EP_COPY, None)]


def stream_ops(gpu, m, n, kb, ops_fn, seed, keep_c=True, onto=False, bad=False, fp8=False):
    """One layer over panels with ops and the requantize, tiles enough to
    take the streaming kernel (at least one per CU); bad: a few weight
    scale bytes outside the fast window (their tiles are folded exactly,
    then the same ops)."""
    rng = np.random.default_rng(seed)
    a = helpers.activations_fp8(rng, m, kb * 32)[1] if fp8 else helpers.activations(rng, m, kb * 32)[1]
    w = mxfp4_w(rng, n, kb)
    if bad:
        w.reshape(-1, 144)[::997, 129] = 200
    ops = ops_fn(rng, m, n)
    tbuf = helpers.activation_table("silu")
    c0 = helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None
    dev_ops = [(k, dev(v.view(np.float32)) if isinstance(v, np.ndarray) else v) for k, v in ops]
    c_d = (dev(c0.view(np.float32)) if onto else torch.zeros((m, n), dtype=torch.float32, device=DEV)) \
        if keep_c else None
    q_d = torch.full(((m + 3) // 4 * (n // 32), 144), 0xA5, dtype=torch.uint8, device=DEV)
    say("stream ops", dict(m=m, n=n, kb=kb, ops=[o[0] for o in ops], keep_c=keep_c, onto=onto,
                           bad=bad, fp8=fp8))
    hb.linear(gpu, a=dev(a), planes=[to_panels(gpu, dev(w), n, kb)], modes=[0], c=c_d, m=m, n=n,
              kb_total=kb, ops=dev_ops, tbuf=dev(tbuf.view(np.int64)), q_out=q_d, mode=hb.FAST,
              panels=True, onto=onto, a_fp8=fp8)
    gq = host(q_d)
    want, wq = helpers.oracle_linear_mt(m, n, kb, a, [w], [0], ops=ops, tbuf=tbuf, quantize=True,
                                        onto=c0, a_fp8=fp8)
    if keep_c:
        helpers.check_fast(host(c_d).view(np.uint32), want)
    helpers.check_requantized(gq, wq)


@pytest.mark.parametrize("m", [4096, 4093])
def test_stream_all_ops_requantize_mxfp8(gpu, m):
    """The streaming kernel's fused epilogue (MXFP8 layers with ops or the
    requantize stream): 4096 (and 4093: a partial last quad) x 2560 x 160,
    32 x 8 = 256 tiles, every op kind, C and the requantize."""
    stream_ops(gpu, m, 2560, 5, all_ops, seed=620 + m, fp8=True)


def test_stream_ops_without_c_mxfp8(gpu):
    stream_ops(gpu, 4096, 2560, 5, lambda r, m, n: all_ops(r, m, n)[:3], seed=625, keep_c=False,
               fp8=True)


def test_stream_ops_exact_recompute_mxfp8(gpu):
    stream_ops(gpu, 4096, 2560, 5, lambda r, m, n: all_ops(r, m, n)[:5], seed=626, bad=True,
               fp8=True)


def test_stream_ops_onto_mxfp8(gpu):
    """From C (a residual start), bias and ReLU."""
    stream_ops(gpu, 32768, 320, 3, lambda r, m, n: [all_ops(r, m, n)[1], (hb.EP_RELU, None)],
               seed=627, onto=True, fp8=True)


@pytest.mark.parametrize("m", [4096, 4093])
def test_tile_kernel_all_ops_requantize(gpu, m):
    """MXINT8 layers with ops over panels take the 128-row tile kernel: every
    op kind, C and the requantize."""
    stream_ops(gpu, m, 2560, 5, all_ops, seed=630 + m)


# ---- the skinny kernel over panels: batches of layers of up to 16 rows ----

def skinny_batch(gpu, m, n, kb, layers, w8=False, pieces=None, bad=False, seed=0):
    """`layers` layers of m <= 16 rows over weight panels in one fast batched
    launch (the skinny kernel), each checked against the oracle.  w8: both
    nibble planes packed as panels; pieces: a piece list; bad: weight scale
    bytes outside the fast window in each layer (those workgroups fold
    exactly)."""
    rng = np.random.default_rng(seed)
    a_h, w_h = [], []
    for i in range(layers):
        a_h.append(helpers.activations(rng, m, kb * 32)[1])
        planes, modes = (list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32)))), [1, 2]) \
            if w8 else ([mxfp4_w(rng, n, kb)], [0])
        if bad:
            planes[0].reshape(-1, 144)[::7, 128 + i % 8] = 200
        w_h.append(planes)
    a_d = dev(np.stack(a_h))
    pb = hb.panel_bytes(n, kb)
    w_p = torch.empty((len(modes), layers, pb), dtype=torch.uint8, device=DEV)
    for i in range(layers):
        for l, p in enumerate(w_h[i]):
            hb.pack_weights(dev(p), n, kb, w_p[l, i], ctx=gpu)
    c_d = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_d[i], [w_p[l, i] for l in range(len(modes))], modes, c_d[i],
                            mode=hb.FAST, panels=True, pieces=pieces) for i in range(layers)]
    torch.cuda.synchronize()
    say("skinny batch", dict(m=m, n=n, kb=kb, layers=layers, w8=w8, pieces=pieces, bad=bad))
    hb.linear_batched(descs, gpu)
    got = host(c_d).view(np.uint32)
    for i in range(layers):
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_h[i], w_h[i], modes, pieces=pieces)
        helpers.check_fast(got[i], want)


@pytest.mark.parametrize("m,n,kb", [(16, 72, 5), (16, 200, 7), (5, 136, 3)])
def test_skinny_partial_panel_odd_blocks(gpu, m, n, kb):
    """n not a multiple of 64 (the last panel partial), odd block counts."""
    skinny_batch(gpu, m, n, kb, 4, seed=640 + n)


def test_skinny_w8_planes_as_panels(gpu):
    skinny_batch(gpu, 8, 136, 9, 3, w8=True, seed=650)


def test_skinny_pieces(gpu):
    skinny_batch(gpu, 12, 256, 12, 3, pieces=[(4, 5), (0, 4), (9, 3)], seed=651)


def test_skinny_out_of_window_scales(gpu):
    skinny_batch(gpu, 16, 128, 6, 3, bad=True, seed=652)
