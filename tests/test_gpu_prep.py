"""Weight preparation on an MI355X, byte for byte against the oracle:
hb_w8_from_fp32 against PadRows + EncodeMxint8 + SplitW8 + PackWbuf of both
planes (tools/compiler/smolvla_common.cpp:95-103, weights.cpp:72-88,
tools/runtime/formats.cpp:35-56, tools/compiler/tensors.cpp:66-90), and
hb_mxfp4_canonical against CanonicalMxfp4 + PackWbuf (weights.cpp:39-70) over
the codes and scale bytes ReadMxfp4 reads (weights.cpp:120-138): padded rows
and K, zero and sign-only blocks, denormal and extreme values, exponent
shifts, the rejections; and a W8 layer whose planes come from
hb_w8_from_fp32 against the oracle's layer over the oracle's planes."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
import oracle
from test_gpu_bench_routes import DEV, dev, host, say

pytestmark = pytest.mark.gpu


def w8_expected(w, rows, cols, out_rows):
    pad = np.zeros((out_rows, cols), np.float32)
    pad[:rows] = w
    q, e = oracle.encode_mxint8(oracle.f32_bits(pad))
    hi, lo = oracle.split_w8(q)
    return oracle.pack_wbuf(hi, e), oracle.pack_wbuf(lo, e)


def w8_gpu(gpu, w, rows, cols, out_rows):
    words = out_rows // 8 * ((cols + 31) // 32)
    hi = torch.full((words, 144), 0xA5, dtype=torch.uint8, device=DEV)
    lo = torch.full_like(hi, 0x5A)
    hb.w8_from_fp32(dev(np.ascontiguousarray(w, np.float32)), rows, cols, out_rows, hi, lo, ctx=gpu)
    return host(hi), host(lo)


@pytest.mark.parametrize("rows,cols,out_rows", [(8, 32, 8), (2560, 960, 2560), (13, 50, 16),
                                                 (720, 736, 728), (3, 1, 8)])
def test_w8_from_fp32(gpu, rows, cols, out_rows):
    rng = np.random.default_rng(rows + cols)
    w = rng.integers(-127, 128, (rows, cols)).astype(np.float32)  # int8-valued weights
    w[: rows // 2] = rng.standard_normal((rows // 2, cols)).astype(np.float32) * 0.02
    if rows > 2 and cols > 40:
        w[1, :32] = 0.0                                            # a zero block
        w[2, 32:40] = np.float32(1e-40)                            # denormals
        w[2, 40] = np.float32(-3.4e38)                             # the top exponent
    say("w8_from_fp32", dict(rows=rows, cols=cols, out_rows=out_rows))
    got = w8_gpu(gpu, w, rows, cols, out_rows)
    want = w8_expected(w, rows, cols, out_rows)
    assert np.array_equal(got[0], want[0])
    assert np.array_equal(got[1], want[1])


def test_w8_from_fp32_rejections(gpu):
    buf = torch.zeros((64, 144), dtype=torch.uint8, device=DEV)
    w = dev(np.ones((8, 32), np.float32))
    for args in ((w, 8, 32, 4, buf, buf), (w, 8, 32, 12, buf, buf), (w, 0, 32, 8, buf, buf),
                 (w, 8, 32, 8, buf[:, 1:], buf)):
        with pytest.raises(hb.HbError) as err:
            hb.w8_from_fp32(*args, ctx=gpu)
        assert err.value.code == hb.HB_EINVAL
    bad = np.ones((8, 32), np.float32)
    bad[3, 7] = np.inf
    with pytest.raises(hb.HbError) as err:
        hb.w8_from_fp32(dev(bad), 8, 32, 8, buf, buf, ctx=gpu)
    assert err.value.code == hb.HB_EINVAL and "infinite" in err.value.message


def mxfp4_expected(codes, scales, shift, out_rows):
    e = scales.astype(np.int32) - 127
    oc, oe = oracle.canonical_mxfp4(codes, e, shift, out_rows)
    return oracle.pack_wbuf(oc, oe)


def mxfp4_gpu(gpu, codes, scales, shift, out_rows):
    rows, cols = codes.shape
    w = torch.full((out_rows // 8 * (cols // 32), 144), 0xA5, dtype=torch.uint8, device=DEV)
    hb.mxfp4_canonical(dev(codes), dev(scales), rows, cols, out_rows, w, exponent_shift=shift,
                       ctx=gpu)
    return host(w)


@pytest.mark.parametrize("rows,cols,shift,out_rows", [(8, 32, 0, 8), (960, 2560, 0, 960),
                                                      (720, 736, -3, 728), (5, 64, 2, 16)])
def test_mxfp4_canonical(gpu, rows, cols, shift, out_rows):
    rng = np.random.default_rng(rows * 3 + cols)
    codes = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    # blocks whose largest magnitude is each of 1..7, a zero block, a sign-only block
    for top in range(1, 8):
        if top < rows:
            codes[top, :32] = rng.integers(0, top + 1, 32) | (rng.integers(0, 2, 32) << 3)
            codes[top, 0] = top
    codes[0, :32] = 0
    if cols >= 64:
        codes[0, 32:64] = 8
    scales = rng.integers(110, 140, (rows, cols // 32), dtype=np.uint8)
    say("mxfp4_canonical", dict(rows=rows, cols=cols, shift=shift, out_rows=out_rows))
    assert np.array_equal(mxfp4_gpu(gpu, codes, scales, shift, out_rows),
                          mxfp4_expected(codes, scales, shift, out_rows))


def test_mxfp4_canonical_rejections(gpu):
    buf = torch.zeros((64, 144), dtype=torch.uint8, device=DEV)
    codes = dev(np.full((8, 32), 7, np.uint8))
    scales_ok = dev(np.full((8, 1), 127, np.uint8))
    for args in ((codes, scales_ok, 8, 30, 8, buf), (codes, scales_ok, 8, 32, 4, buf),
                 (codes, scales_ok, 8, 32, 8, buf[:, 1:])):
        with pytest.raises(hb.HbError) as err:
            hb.mxfp4_canonical(*args, ctx=gpu)
        assert err.value.code == hb.HB_EINVAL
    # the canonical exponent leaves E8M0: scale byte 254 (+127) with a top
    # code of 1 (floor log2 -1, so -3) and a shift of +4 make 128
    hi = np.zeros((8, 32), np.uint8)
    hi[:, 0] = 1
    with pytest.raises(hb.HbError) as err:
        hb.mxfp4_canonical(dev(hi), dev(np.full((8, 1), 254, np.uint8)), 8, 32, 8, buf,
                           exponent_shift=4, ctx=gpu)
    assert err.value.code == hb.HB_EINVAL and "E8M0" in err.value.message


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_w8_layer_from_prepared_weights(gpu, mode):
    """Config-0-shaped W8 layer (M=64, K=960, N=2560, per-channel scale and
    bias) whose planes hb_w8_from_fp32 made from int8-valued fp32 weights."""
    rng = np.random.default_rng(40)
    m, n, k = 64, 2560, 960
    w = rng.integers(-127, 128, (n, k)).astype(np.float32)
    hi, lo = w8_gpu(gpu, w, n, k, n)
    a = helpers.activations(rng, m, k)[1]
    scale = np.asarray(rng.uniform(0.001, 0.02, n), np.float32).view(np.uint32)
    bias = np.asarray(rng.normal(0, 0.1, n), np.float32).view(np.uint32)
    ops = [(hb.EP_MULP, scale), (hb.EP_ADDP, bias)]
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    say("w8 layer from prepared weights", dict(mode=mode))
    hb.linear(gpu, a=dev(a), planes=[dev(hi), dev(lo)], modes=[1, 2], c=c_d, m=m, n=n,
              kb_total=k // 32, ops=[(kk, dev(v.view(np.float32))) for kk, v in ops], mode=mode)
    got = host(c_d).view(np.uint32)
    want_hi, want_lo = w8_expected(w, n, k, n)
    want, _ = helpers.oracle_linear_mt(m, n, k // 32, a, [want_hi, want_lo], [1, 2], ops=ops)
    if mode == hb.EXACT:
        assert np.array_equal(got, want)
    else:
        helpers.check_fast(got, want)
