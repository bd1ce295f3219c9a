"""DDR images in device memory on an MI355X: bytes put and read back (a new
image is zero, DdrImage's Put test, tools/compiler/ddr_image_test.cpp:56-65),
puts past the capacity refused, and linear layers whose A, W, C and q_out
are regions of one image, placed the way the compiler places them
(tools/compiler/smolvla_common.cpp:95-103), against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import helpers
import hotarubi_amd as hb
from test_gpu_bench_routes import mxfp4_planes, say, w8_planes

pytestmark = pytest.mark.gpu


def test_put_writes_the_bytes(gpu):
    im = hb.Image(1 << 16, ctx=gpu)
    off = im.alloc("a", 4)
    im.put(off + 1, b"\x12\x34")
    assert im.get(0, 4) == b"\x00\x12\x34\x00"
    assert im.get((1 << 16) - 8, 8) == bytes(8)
    with pytest.raises(hb.HbError) as err:
        im.put((1 << 16) - 1, b"\x00\x00")
    assert err.value.code == hb.HB_EINVAL and "exceed the image" in err.value.message
    im.close()


@pytest.mark.parametrize("w8,mode", [(False, hb.FAST), (True, hb.EXACT), (True, hb.FAST)])
def test_layer_over_image_regions(gpu, w8, mode):
    rng = np.random.default_rng(7 + w8)
    m, n, kb = 132, 256, 9
    a = helpers.activations(rng, m, kb * 32)[1]
    planes, modes = w8_planes(rng, n, kb) if w8 else mxfp4_planes(rng, n, kb)
    scale = np.asarray(rng.uniform(0.001, 0.02, n), np.float32).view(np.uint32)
    im = hb.Image(16 << 20, ctx=gpu)
    im.set_reuse(True)
    im.put(im.alloc("x.a", a.nbytes), a.tobytes())
    for i, p in enumerate(planes):
        im.put(im.alloc(f"x.w{i}", p.nbytes), p.tobytes())
    im.put(im.alloc("x.scale", scale.nbytes), scale.tobytes())
    im.alloc("x.c", m * n * 4)
    im.alloc("x.q", (m + 3) // 4 * (n // 32) * 144)
    d = hb.linear_desc(m, n, kb, im.ptr("x.a"), [im.ptr(f"x.w{i}") for i in range(len(planes))],
                       modes, im.ptr("x.c"), ops=[(hb.EP_MULP, im.ptr("x.scale"))],
                       q_out=im.ptr("x.q"), mode=mode)
    say("layer over image regions", dict(w8=w8, mode=mode))
    hb.launch(d, gpu)
    gpu.synchronize()
    got = np.frombuffer(im.get(im.region("x.c")[0], m * n * 4), np.uint32).reshape(m, n)
    gq = np.frombuffer(im.get(im.region("x.q")[0], im.region("x.q")[1]), np.uint8)
    want, wq = helpers.oracle_linear_mt(m, n, kb, a, planes, modes, ops=[(hb.EP_MULP, scale)],
                                        quantize=True)
    if mode == hb.EXACT:
        assert np.array_equal(got, want)
        assert np.array_equal(gq, wq.reshape(-1))
    else:
        helpers.check_fast(got, want, gq, wq)
    im.close()
