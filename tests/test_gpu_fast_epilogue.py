"""Fast-mode MXFP4 layers of more than 64 rows (128-row tiles) with epilogue
ops and the MXINT8 requantize, unsplit: a single layer of at most 4 K-steps,
and a batch of layers (the tiles finish their own epilogue).  Each case is checked against the oracle's linear layer
(tools/iss/gemm_array.cpp:112-149, ops per tools/iss/vec_rom.cpp and
tools/iss/lane.cpp, requantize per tools/iss/lane.cpp:384-424): per output
row r, max_n |gpu - ref| <= 1e-5 max_n |ref|; requantized bytes differ by at
most 1 in under 1% of places (the fast ops round differently near a step)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
from test_gpu_linear import DEV, dev, host, make_layer, oracle_linear, run_linear, say

pytestmark = pytest.mark.gpu


def check_fast(got, want, gq=None, wq=None):
    g, w = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
    row_scale = np.abs(w).max(axis=1, keepdims=True)
    assert (np.abs(g - w) <= 1e-5 * row_scale).all(), float((np.abs(g - w) / row_scale).max())
    if gq is not None:
        gqb = gq.reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
        wqb = wq.reshape(-1, 144)[:, :128].view(np.int8).astype(np.int32)
        assert np.abs(gqb - wqb).max() <= 1 and (gqb != wqb).mean() < 0.01
        gs, ws = gq.reshape(-1, 144)[:, 128:], wq.reshape(-1, 144)[:, 128:]
        assert (gs[:, 4:] == 0).all()
        assert (gs[:, :4] != ws[:, :4]).mean() < 0.01


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_single_layer_ops_and_requantize(gpu, act):
    """M = 198 (a partly used second row tile, a last quad of 2 rows),
    N = 320 (a partly used column tile), K = 256 (4 steps: not split)."""
    rng = np.random.default_rng(300)
    m, n, k = 198, 320, 256
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
            got, gq = run_linear(gpu, m, n, kb, a, planes, modes, ops, tbuf=tbuf,
                                 quantize=quantize, mode=hb.FAST)
            want, wq = oracle_linear(m, n, kb, a, planes, modes, ops, tbuf=tbuf,
                                     quantize=quantize)
            check_fast(got, want, gq, wq)


@pytest.mark.parametrize("slow", [False, True])
def test_batched_pieces_onto_ops_requantize(gpu, slow):
    """Three layers in one launch over a piece list, starting from C, with
    per-channel MULP / ADDP, the residual ADD and the requantize.  slow: a
    few weight words carry scale bytes outside the fast path's window, so
    their tiles are recomputed with the exact fold before the ops."""
    rng = np.random.default_rng(310 + slow)
    layers, m, n, k = 3, 198, 320, 640
    data = [make_layer(rng, m, n, k, False) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    if slow:
        for d in data:
            d[2][0].reshape(-1, 144)[::37, 128] = 200
    pieces = [(13, 7), (0, 5), (5, 8)]
    onto = np.stack([helpers.random_fp32_words(rng, (m, n), 120, 130) for _ in range(layers)])
    scale = np.stack([helpers.random_fp32_words(rng, (n,), 117, 122) for _ in range(layers)])
    bias = np.stack([helpers.random_fp32_words(rng, (n,), 118, 124) for _ in range(layers)])
    res = np.stack([helpers.random_fp32_words(rng, (m, n), 118, 128) for _ in range(layers)])
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = dev(np.stack([d[2][0] for d in data]))
    c_all = dev(onto.view(np.float32))
    s_all, b_all, r_all = dev(scale.view(np.float32)), dev(bias.view(np.float32)), \
        dev(res.view(np.float32))
    nb = n // 32
    q_all = torch.zeros((layers, (m + 3) // 4 * nb, 144), dtype=torch.uint8, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], modes, c_all[i], pieces=pieces,
                            onto=True, ops=[(hb.EP_MULP, s_all[i]), (hb.EP_ADDP, b_all[i]),
                                            (hb.EP_ADD, r_all[i])],
                            q_out=q_all[i], mode=hb.FAST) for i in range(layers)]
    torch.cuda.synchronize()
    say("fp4 batched pieces onto ops requantize", dict(layers=layers, slow=slow))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    gq = host(q_all)
    for i, d in enumerate(data):
        ops = [(hb.EP_MULP, scale[i]), (hb.EP_ADDP, bias[i]), (hb.EP_ADD, res[i])]
        want, wq = oracle_linear(m, n, kb, d[1], d[2], d[3], ops, pieces=pieces, onto=onto[i],
                                 quantize=True)
        check_fast(got[i], want, gq[i], wq)


def test_unaligned_output_of_a_streaming_layer(gpu):
    """C 4 bytes past a 16-byte boundary: a batched MXFP4 layer of 128 rows
    that would take the streaming kernel (16-byte stores) is still correct."""
    rng = np.random.default_rng(320)
    layers, m, n, k = 2, 128, 256, 320
    data = [make_layer(rng, m, n, k, False) for _ in range(layers)]
    kb, modes = data[0][0], data[0][3]
    a_all = dev(np.stack([d[1] for d in data]))
    w_all = dev(np.stack([d[2][0] for d in data]))
    flat = torch.zeros((layers * m * n + 1,), dtype=torch.float32, device=DEV)
    c_all = flat[1:].view(layers, m, n)
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], modes, c_all[i], mode=hb.FAST)
             for i in range(layers)]
    torch.cuda.synchronize()
    say("unaligned C", dict(layers=layers, m=m, n=n))
    hb.linear_batched(descs, gpu)
    got = host(c_all).view(np.uint32)
    for i, d in enumerate(data):
        want, _ = oracle_linear(m, n, kb, d[1], d[2], d[3])
        check_fast(got[i], want)
