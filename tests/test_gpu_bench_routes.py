"""The kernels bench.py times, at the shapes and through the routes it times
them, against the oracle (tools/iss/gemm_array.cpp:112-149 folded as
tools/compiler/kernels.cpp:343-395 emits a layer, epilogue per
tools/iss/lane.cpp):

  * batched MXFP4 M=128 K=2560 N=960 (the headline): one tile per workgroup
    (2 layers) and the persistent multi-tile route (80 layers, 320 tiles);
  * batched M=1024 (10 layers, 320 tiles);
  * batched M=1 and M=16 (the skinny route with a layer index per workgroup),
    over DDR words and over weight panels (the bench's layout);
  * the SparseDrive-S stage-1 im2col shape K=576 N=64 at 16,384 rows (128
    row tiles: the streaming route, not the small-layer split), both modes;
  * the SigLIP-style W8 MLP, up 768->3072 with MULP, ADDP, GELU and the
    requantize and down 3072->768 with MULP and ADDP, at M=2048, both modes;
  * SmolVLA prefix layers at batch 32 (M=4512: q with requantize and down
    with the residual add on 96-row tiles, a two-piece layer on them, k with
    requantize on 64-row tiles) and the action expert's layers
    at batch 32 (M=1600: q with requantize, down with the residual add, both
    K-split over 64-row tiles; the 720->2048 gate with ACT_MUL(up) and
    requantize, 200 unsplit 64-row tiles);
  * A operands whose codes cover all 256 int8 values, -128 included, through
    every fast route and the exact kernel.

Fast mode: per output row max |gpu - ref| <= 1e-5 max |ref| and, on plain
layers, per element |gpu - ref| <= 2^-17 sum_b |block value|; exact mode:
bitwise.  Layers of a batch that the oracle checks are spread over the
batch (first, last and between)."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def mxfp4_planes(rng, n, kb, lo=-10, hi=-2):
    code, e = helpers.mxfp4_weights(rng, n, kb * 32, lo, hi)
    import oracle
    return [oracle.pack_wbuf(code, e)], [0]


def w8_planes(rng, n, kb):
    return list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32)))), [1, 2]


def to_panels(gpu, w_d, n, kb):
    """Device DDR words -> device weight panels (hb_pack_weights)."""
    out = torch.empty((hb.panel_bytes(n, kb),), dtype=torch.uint8, device=DEV)
    hb.pack_weights(w_d, n, kb, out, ctx=gpu)
    return out


def batched_layers(gpu, m, n, kb, layers, check, mode, all_codes=False, seed=0, panels=False,
                   onto=False, bad_scales=False):
    """`layers` MXFP4 layers of one shape in one batched launch; the oracle
    checks the layers in `check`.  panels: the weights go through
    hb_pack_weights and the layers read the panels.  onto: start from C.
    bad_scales: a few weight scale bytes outside the fast path's window (those
    tiles are recomputed with the exact fold)."""
    rng = np.random.default_rng(seed)
    a_host, w_host, c0 = [], [], []
    for i in range(layers):
        if all_codes:
            a = helpers.random_a_words(rng, m, kb)
        else:
            a = helpers.activations(rng, m, kb * 32)[1]
        a_host.append(a)
        w = mxfp4_planes(rng, n, kb)[0][0]
        if bad_scales:
            w.reshape(-1, 144)[::53, 128 + (i % 8)] = 200
        w_host.append(w)
        c0.append(helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None)
    a_d, w_d = dev(np.stack(a_host)), dev(np.stack(w_host))
    if panels:
        pb = hb.panel_bytes(n, kb)
        w_p = torch.empty((layers, pb), dtype=torch.uint8, device=DEV)
        for i in range(layers):
            hb.pack_weights(w_d[i], n, kb, w_p[i], ctx=gpu)
        w_d = w_p
    c_d = dev(np.stack(c0).view(np.float32)) if onto else \
        torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    descs = [hb.linear_desc(m, n, kb, a_d[i], [w_d[i]], [0], c_d[i], mode=mode, panels=panels,
                            onto=onto)
             for i in range(layers)]
    torch.cuda.synchronize()
    say("batched", dict(m=m, n=n, kb=kb, layers=layers, mode=mode, all_codes=all_codes,
                        panels=panels, onto=onto, bad_scales=bad_scales))
    hb.linear_batched(descs, gpu)
    got = host(c_d).view(np.uint32)
    for i in check:
        want, _ = helpers.oracle_linear_mt(m, n, kb, a_host[i], [w_host[i]], [0], onto=c0[i])
        if mode == hb.EXACT:
            assert np.array_equal(got[i], want), i
        else:
            helpers.check_fast(got[i], want,
                               bound=None if onto or bad_scales else
                               helpers.block_abs_sums(m, n, kb, a_host[i], [w_host[i]], [0]))


@pytest.mark.parametrize("layers,check", [(2, (0, 1)), (80, (0, 1, 37, 63, 79))])
def test_headline_batched_m128(gpu, layers, check):
    batched_layers(gpu, 128, 960, 80, layers, check, hb.FAST, seed=layers)


def test_headline_batched_m1024(gpu):
    batched_layers(gpu, 1024, 960, 80, 10, (0, 9), hb.FAST, seed=1024)


@pytest.mark.parametrize("panels", [False, True])
@pytest.mark.parametrize("m", [1, 16])
def test_skinny_batched(gpu, m, panels):
    batched_layers(gpu, m, 960, 80, 6, range(6), hb.FAST, seed=m, panels=panels)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_all_int8_codes_batched(gpu, mode):
    """A covering all 256 codes: the streaming route (M=128, batched) and, in
    exact mode, the exact tile kernel."""
    batched_layers(gpu, 128, 256, 12, 3, range(3), mode, all_codes=True, seed=77)


@pytest.mark.parametrize("m", [16, 48])
def test_all_int8_codes_skinny(gpu, m):
    batched_layers(gpu, m, 256, 12, 2, range(2), hb.FAST, all_codes=True, seed=78 + m)


def single_layer(gpu, m, n, kb, w8, mode, ops_fn=None, quantize=False, tbuf=None,
                 all_codes=False, seed=0, bound=False, panels=False, pieces=None):
    rng = np.random.default_rng(seed)
    a = helpers.random_a_words(rng, m, kb) if all_codes else helpers.activations(rng, m, kb * 32)[1]
    planes, modes = w8_planes(rng, n, kb) if w8 else mxfp4_planes(rng, n, kb)
    w_dev = [dev(p) for p in planes]
    if panels:
        w_dev = [to_panels(gpu, w, n, kb) for w in w_dev]
    ops = ops_fn(rng, m, n) if ops_fn else []
    dev_ops = [(k, dev(v.view(np.float32)) if isinstance(v, np.ndarray) else v) for k, v in ops]
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    q_d = torch.zeros(((m + 3) // 4 * (n // 32), 144), dtype=torch.uint8, device=DEV) \
        if quantize else None
    tb_d = dev(tbuf.view(np.int64)) if tbuf is not None else None
    torch.cuda.synchronize()
    say("layer", dict(m=m, n=n, kb=kb, w8=w8, mode=mode, ops=[o[0] for o in ops],
                      quantize=quantize, all_codes=all_codes, panels=panels, pieces=pieces))
    hb.linear(gpu, a=dev(a), planes=w_dev, modes=modes, c=c_d, m=m, n=n,
              kb_total=kb, ops=dev_ops, tbuf=tb_d, q_out=q_d, mode=mode, panels=panels,
              pieces=pieces)
    got = host(c_d).view(np.uint32)
    gq = host(q_d) if quantize else None
    want, wq = helpers.oracle_linear_mt(m, n, kb, a, planes, modes, ops=ops, tbuf=tbuf,
                                        quantize=quantize, pieces=pieces)
    if mode == hb.EXACT:
        assert np.array_equal(got, want)
        if quantize:
            assert np.array_equal(gq, wq)
    else:
        helpers.check_fast(got, want, gq, wq,
                           bound=helpers.block_abs_sums(m, n, kb, a, planes, modes, pieces)
                           if bound else None)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_sparsedrive_stage1_shape_128_row_tiles(gpu, mode):
    single_layer(gpu, 16384, 64, 18, False, mode, seed=90, bound=True)


def per_channel(rng, n, gelu=False):
    scale = np.asarray(rng.uniform(0.001, 0.02, n), np.float32).view(np.uint32)
    bias = np.asarray(rng.normal(0, 0.1, n), np.float32).view(np.uint32)
    return [(hb.EP_MULP, scale), (hb.EP_ADDP, bias)] + ([(hb.EP_ACT, None)] if gelu else [])


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_siglip_mlp_up_gelu_requantize(gpu, mode):
    single_layer(gpu, 2048, 3072, 24, True, mode, lambda r, m, n: per_channel(r, n, True),
                 quantize=True, tbuf=helpers.activation_table("gelu"), seed=91)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_siglip_mlp_down(gpu, mode):
    single_layer(gpu, 2048, 768, 96, True, mode, lambda r, m, n: per_channel(r, n), seed=92)


def test_prefix_b32_q_requantize(gpu):
    single_layer(gpu, 4512, 960, 30, False, hb.FAST, quantize=True, seed=93)


def test_prefix_b32_k_requantize(gpu):
    single_layer(gpu, 4512, 320, 30, False, hb.FAST, quantize=True, seed=94)


def test_prefix_b32_pieces_96_row_tiles(gpu):
    """4512 x 960 MXFP4 in two pieces with the residual add: 188 tiles of 96
    rows (128-row tiles would leave CUs idle, 64-row tiles take two rounds)."""
    single_layer(gpu, 4512, 960, 30, False, hb.FAST,
                 lambda r, m, n: [(hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))],
                 quantize=True, pieces=[(0, 14), (14, 16)], seed=90)


def test_prefix_b32_down_residual(gpu):
    single_layer(gpu, 4512, 960, 80, False, hb.FAST,
                 lambda r, m, n: [(hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))],
                 seed=95)


def test_expert_b32_q_requantize(gpu):
    """720 -> 960 at M=1600: 100 tiles of 64 rows, K split, epilogue kernel."""
    single_layer(gpu, 1600, 960, 23, False, hb.FAST, quantize=True, seed=98)


def test_expert_b32_down_residual(gpu):
    """2048 -> 720 at M=1600: 75 tiles of 64 rows, K split over 64 blocks."""
    single_layer(gpu, 1600, 720, 64, False, hb.FAST,
                 lambda r, m, n: [(hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128))],
                 seed=99)


def test_expert_b32_gate_act_mul_requantize(gpu):
    single_layer(gpu, 1600, 2048, 23, False, hb.FAST,
                 lambda r, m, n: [(hb.EP_ACT_MUL, helpers.random_fp32_words(r, (m, n), 120, 130))],
                 quantize=True, tbuf=helpers.activation_table("silu"), seed=96)


@pytest.mark.parametrize("m,n,kb,w8,quantize", [
    (141, 960, 30, False, False),   # K-split path + epilogue kernel
    (50, 2048, 23, False, False),   # skinny kernel, one layer of up to 64 rows
    (4512, 960, 30, False, True),   # 128-row tile kernel, unsplit, requantize
    (2048, 3072, 24, True, False),  # 128-row tile kernel, W8, unsplit
    (200, 768, 24, True, False)])   # K-split path, W8
def test_all_int8_codes_single_layer(gpu, m, n, kb, w8, quantize):
    """A covering all 256 codes through the fast single-layer routes."""
    single_layer(gpu, m, n, kb, w8, hb.FAST, quantize=quantize, all_codes=True, seed=97 + m,
                 bound=not quantize)
