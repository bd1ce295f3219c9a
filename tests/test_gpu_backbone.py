"""SparseDrive-S backbone GEMMs on an MI355X against the oracle, at the row
counts bench.py times them (so each takes the same kernel route), with the
weights in panels as the bench streams them.

The layers are the reference compiler's lowering of the ResNet-50 backbone
over 6 cameras at 256 x 704 (tools/compiler/sparsedrive_encoder.cpp: stem
571-640, bottlenecks 817-874, EmitConv 187-475): the W8 stem (K = 192,
N = 64, bias + ReLU, fp32 out); per stage of mid width 64/128/256/512,
conv1 (1x1) and conv2 (3x3 im2col) with bias, ReLU and the MXINT8
requantize, conv3 (1x1, N = 4 x mid) with bias, ReLU, fp32 out and the
requantize, folding the downsample as a second K range in block 0 and
starting from the residual in later blocks.  Every distinct layer at one
frame (rows 6 x H x W), and the stage-3 and stage-4 layers again at 16
frames, where their grids grow past the small-layer K split.

Fast mode against the oracle's exact fold (tools/iss/gemm_array.cpp:
112-149, epilogue tools/iss/lane.cpp): per output row max |gpu - ref| <=
1e-5 max |ref|, requantized bytes within one step; exact mode bitwise."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
from test_gpu_bench_routes import DEV, dev, host, mxfp4_planes, say, to_panels, w8_planes

pytestmark = pytest.mark.gpu

CAMS = 6
ROWS = {0: CAMS * 128 * 352, 1: CAMS * 64 * 176, 2: CAMS * 32 * 88, 3: CAMS * 16 * 44,
        4: CAMS * 8 * 22}
MID = {1: 64, 2: 128, 3: 256, 4: 512}


def layers():
    """(name, stage of the rows, K, N, w8, onto, fp32 out) of every distinct
    backbone GEMM; rows are ROWS[stage] per frame."""
    out = [("stem", 0, 192, 64, True, False, True)]
    cin = 64
    for s in (1, 2, 3, 4):
        mid, cout = MID[s], 4 * MID[s]
        out += [(f"s{s}_conv1_b0", s - 1 if s > 1 else 1, cin, mid, False, False, False),
                (f"s{s}_conv2", s, 9 * mid, mid, False, False, False),
                (f"s{s}_conv3_down", s, mid + cin, cout, False, False, True),
                (f"s{s}_conv1", s, cout, mid, False, False, False),
                (f"s{s}_conv3_residual", s, mid, cout, False, True, True)]
        cin = cout
    return out


LAYERS = {ly[0]: ly for ly in layers()}


def conv_layer(gpu, name, frames, mode, seed):
    _, stage, k, n, w8, onto, _ = LAYERS[name]
    m, kb = ROWS[stage] * frames, k // 32
    rng = np.random.default_rng(seed)
    a = helpers.random_a_words(rng, m, kb)
    planes, modes = w8_planes(rng, n, kb) if w8 else mxfp4_planes(rng, n, kb)
    w_dev = [to_panels(gpu, dev(p), n, kb) for p in planes]
    bias = np.asarray(rng.normal(0, 0.1, n), np.float32).view(np.uint32)
    ops = [(hb.EP_ADDP, bias), (hb.EP_RELU, None)]
    dev_ops = [(hb.EP_ADDP, dev(bias.view(np.float32))), (hb.EP_RELU, None)]
    c0 = helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None
    c_d = dev(c0.view(np.float32)) if onto else \
        torch.zeros((m, n), dtype=torch.float32, device=DEV)
    quantize = not w8
    q_d = torch.zeros(((m + 3) // 4 * (n // 32), 144), dtype=torch.uint8, device=DEV) \
        if quantize else None
    torch.cuda.synchronize()
    say("backbone", dict(layer=name, frames=frames, m=m, k=k, n=n, w8=w8, onto=onto, mode=mode))
    hb.linear(gpu, a=dev(a), planes=w_dev, modes=modes, c=c_d, m=m, n=n, kb_total=kb,
              ops=dev_ops, q_out=q_d, mode=mode, panels=True, onto=onto)
    got = host(c_d).view(np.uint32)
    gq = host(q_d) if quantize else None
    want, wq = helpers.oracle_linear_mt(m, n, kb, a, planes, modes, ops=ops, onto=c0,
                                        quantize=quantize)
    if mode == hb.EXACT:
        assert np.array_equal(got, want)
        if quantize:
            assert np.array_equal(gq, wq)
    else:
        helpers.check_fast(got, want, gq, wq)


@pytest.mark.parametrize("name", list(LAYERS))
def test_backbone_one_frame(gpu, name):
    conv_layer(gpu, name, 1, hb.FAST, seed=700 + list(LAYERS).index(name))


@pytest.mark.parametrize("name", [n for n in LAYERS if n[:2] in ("s3", "s4")])
def test_backbone_sixteen_frames(gpu, name):
    conv_layer(gpu, name, 16, hb.FAST, seed=730 + list(LAYERS).index(name))


@pytest.mark.parametrize("name", ["s1_conv2", "s3_conv3_residual", "s4_conv2", "stem"])
def test_backbone_exact(gpu, name):
    conv_layer(gpu, name, 1, hb.EXACT, seed=760 + list(LAYERS).index(name))
