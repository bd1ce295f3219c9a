"""SparseDrive-S detection head GEMMs on an MI355X against the oracle, at the
shapes the head's compiler emits (tools/compiler/sparsedrive_head.cpp):
928 anchor rows per frame (900 padded), 608 temporal key rows.

  * attention projections (800-886): q over the anchors and k over the
    temporal keys, 512 -> 512 W8 with bias (ADDP) and requantize, the input
    as the two 256-wide pieces the head concatenates (feature, anchor
    embedding);
  * the out projection (889-990): 512 -> 512 W8, bias, the residual add,
    requantize;
  * the FFN (1535-1620): fc1 512 -> 1024 MXFP4 with bias, ReLU and
    requantize; fc2 1024 -> 256 over fc1's words, then the identity
    projection 512 -> 256 onto fc2's output with bias (its `onto` fold
    starts from fc2's C);
  * fc1 at 16 frames (14,848 rows).

Exact mode bitwise; fast mode within the fast-mode tolerance."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
from test_gpu_bench_routes import DEV, dev, host, mxfp4_planes, say, single_layer, w8_planes

pytestmark = pytest.mark.gpu

ROWS, TEMP = 928, 608


def bias(rng, n):
    return np.asarray(rng.normal(0, 0.1, n), np.float32).view(np.uint32)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
@pytest.mark.parametrize("m", [ROWS, TEMP])
def test_attention_projection(gpu, mode, m):
    single_layer(gpu, m, 512, 16, True, mode, lambda r, mm, n: [(hb.EP_ADDP, bias(r, n))],
                 quantize=True, seed=601 + m, pieces=[(0, 8), (8, 8)])


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_out_projection_residual(gpu, mode):
    single_layer(gpu, ROWS, 512, 16, True, mode,
                 lambda r, m, n: [(hb.EP_ADDP, bias(r, n)),
                                  (hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))],
                 quantize=True, seed=610)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_ffn_fc1_relu_requantize(gpu, mode):
    single_layer(gpu, ROWS, 1024, 16, False, mode,
                 lambda r, m, n: [(hb.EP_ADDP, bias(r, n)), (hb.EP_RELU, None)],
                 quantize=True, seed=620)


def test_ffn_fc1_16_frames(gpu):
    single_layer(gpu, 16 * ROWS, 1024, 16, False, hb.FAST,
                 lambda r, m, n: [(hb.EP_ADDP, bias(r, n)), (hb.EP_RELU, None)],
                 quantize=True, seed=621)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_ffn_fc2_then_identity_onto(gpu, mode):
    """fc2 (K = 1024) writes C; the identity projection (K = 512) folds onto
    it and adds the bias, as Ffn emits them into one FBUF tile."""
    rng = np.random.default_rng(630)
    m, n = ROWS, 256
    h = helpers.activations(rng, m, 1024)[1]
    a = helpers.activations(rng, m, 512)[1]
    p2, modes = mxfp4_planes(rng, n, 32)
    pi, _ = mxfp4_planes(rng, n, 16)
    b = bias(rng, n)
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    say("ffn fc2 + identity onto", dict(mode=mode))
    hb.linear(gpu, a=dev(h), planes=[dev(p) for p in p2], modes=modes, c=c_d, m=m, n=n,
              kb_total=32, mode=mode)
    fc2 = host(c_d).view(np.uint32).copy()
    hb.linear(gpu, a=dev(a), planes=[dev(p) for p in pi], modes=modes, c=c_d, m=m, n=n,
              kb_total=16, onto=True, ops=[(hb.EP_ADDP, dev(b.view(np.float32)))], mode=mode)
    got = host(c_d).view(np.uint32)
    want2, _ = helpers.oracle_linear_mt(m, n, 32, h, p2, modes)
    want, _ = helpers.oracle_linear_mt(m, n, 16, a, pi, modes, onto=fc2,
                                       ops=[(hb.EP_ADDP, b)])
    if mode == hb.EXACT:
        assert np.array_equal(fc2, want2)
        assert np.array_equal(got, want)
    else:
        helpers.check_fast(fc2, want2)
        helpers.check_fast(got, want)
