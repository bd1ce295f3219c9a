"""The oracle's restatement of the weight-panel layout (this build's own
GPU-native format for a weight plane, hb_pack_weights): every byte of a
packed chunk is the DDR word byte the layout names (brute force over all
(column, block) pairs of small shapes, partial last panel and odd block
counts included), the padding is zero codes with scale 127, and unpacking
gives back the DDR words (tools/compiler/tensors.cpp:66-90 PackWbuf) bit for
bit.  Also hb_panel_bytes (host-only) against the oracle's size."""
from __future__ import annotations

import numpy as np
import pytest

import helpers
import hotarubi_amd as hb
import oracle


def ddr_words(rng, n, kb):
    w = rng.integers(0, 256, (n // 8, kb, 144), dtype=np.uint8)
    w[:, :, 136:] = 0  # PackWbuf's padding
    return w.reshape(-1, 144)


@pytest.mark.parametrize("n,kb", [(8, 1), (64, 2), (72, 3), (136, 5), (960, 80), (320, 23)])
def test_every_byte_by_its_address(n, kb):
    rng = np.random.default_rng(n * 100 + kb)
    w = ddr_words(rng, n, kb)
    p = oracle.pack_panels(w, n, kb)
    assert p.size == oracle.panel_bytes(n, kb) == hb.panel_bytes(n, kb)
    S = (kb + 1) // 2
    wd = w.reshape(n // 8, kb, 144)
    seen = np.zeros(p.size, bool)
    for col in range(0, ((n + 63) // 64) * 64):
        for blk in range(2 * S):
            chunk = ((col // 64) * S + blk // 2) * 2176
            c, b = col % 64, blk % 2
            at = chunk + (b * 64 + c) * 16
            sat = chunk + 2048 + 2 * (b * 32 + c % 32) + c // 32
            if col < n and blk < kb:
                assert np.array_equal(p[at: at + 16], wd[col // 8, blk, (col % 8) * 16: (col % 8) * 16 + 16])
                assert p[sat] == wd[col // 8, blk, 128 + col % 8]
            else:
                assert not p[at: at + 16].any() and p[sat] == 127
            seen[at: at + 16] = True
            seen[sat] = True
    assert seen.all()  # the layout covers every byte exactly


@pytest.mark.parametrize("n,kb", [(8, 1), (72, 3), (960, 80), (2048, 23)])
def test_round_trip(n, kb):
    rng = np.random.default_rng(kb)
    w = ddr_words(rng, n, kb)
    assert np.array_equal(oracle.unpack_panels(oracle.pack_panels(w, n, kb), n, kb), w)


def test_linear_over_unpacked_panels_is_the_same_layer():
    """A layer whose weights went through pack and unpack is the same layer:
    the oracle's GEMM over the round-tripped words equals the original."""
    rng = np.random.default_rng(3)
    m, n, kb = 8, 72, 3
    a = helpers.activations(rng, m, kb * 32)[1]
    code, e = helpers.mxfp4_weights(rng, n, kb * 32)
    w = oracle.pack_wbuf(code, e)
    back = oracle.unpack_panels(oracle.pack_panels(w, n, kb), n, kb)
    assert np.array_equal(oracle.linear(m, n, kb, a, [back], [0])[0],
                          oracle.linear(m, n, kb, a, [w], [0])[0])


def test_panel_bytes_rejects_bad_shapes():
    assert hb.panel_bytes(12, 3) == 0 and hb.panel_bytes(8, 0) == 0
    assert hb.panel_bytes(960, 80) == 15 * 40 * 2176 == 960 * 2560 * (0.5 + 1 / 32)


def test_w8_panel_bytes():
    """W8 panels (host-only size): 6400-byte chunks per 64 columns and two
    blocks (both planes' FP6 codes, 1.5 bytes a weight, and their scale
    bytes), then one flag dword per panel padded to 16 bytes."""
    assert hb.w8_panel_bytes(12, 3) == 0 and hb.w8_panel_bytes(8, 0) == 0
    assert hb.w8_panel_bytes(768, 24) == 12 * 12 * 6400 + 48
    assert hb.w8_panel_bytes(72, 3) == 2 * 2 * 6400 + 16
    n, kb = 3072, 24
    codes = n * kb * 32 * 2 * 6 // 8
    assert hb.w8_panel_bytes(n, kb) == codes + n * kb * 2 + (n // 64) * 4
