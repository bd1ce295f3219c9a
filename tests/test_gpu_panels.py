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
from test_gpu_bench_routes import DEV, batched_layers, dev, host, per_channel, say, single_layer

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
