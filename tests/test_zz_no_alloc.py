"""hb_linear_noalloc_async: hb_linear_batched_async without device
allocation, its K-split scratch a fixed per-device array.  Its results are
checked bitwise against hb_linear_batched_async's on the same descriptors
(the same kernels run; only the scratch buffer differs):

  * two calls in a row on small layers whose K splits meet in the scratch
    (the second one smaller, so it runs over what the first left there),
    then an exact-mode layer whose epilogue is deferred through the scratch;
  * batched and skinny layers, which need no scratch;
  * capture in a HIP graph, replayed between eager work (the point of the
    entry point: no allocation happens inside the capture, even for a shape
    never run before), and a captured layer whose K splits meet in the
    array replayed between eager calls that overwrite it;
  * a layer whose partial sums exceed the array is rejected with HB_ENOMEM
    before anything is launched.

The first call's result is also checked against the oracle (fast-mode
tolerance), so the comparison does not rest on the existing entry point
alone."""
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


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host_u32(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32)


def mxfp4_layer(rng, m, n, kb):
    a = helpers.activations(rng, m, kb * 32)[1]
    code, e = helpers.mxfp4_weights(rng, n, kb * 32)
    return a, [oracle.pack_wbuf(code, e)], [0]


def w8_layer(rng, m, n, kb):
    a = helpers.activations(rng, m, kb * 32)[1]
    planes = list(helpers.w8_planes_from_int8(rng.integers(-127, 128, (n, kb * 32))))
    return a, planes, [1, 2]


def run_both(gpu, m, n, kb, a, planes, modes, mode, ops=(), layers=1):
    """The same descriptors through both entry points; returns (existing,
    no-allocation) outputs as uint32."""
    # `layers` copies of the layer, each one's buffers at a fixed stride
    a_d = dev(np.concatenate([a] * layers))
    w_d = [dev(np.concatenate([p] * layers)) for p in planes]
    outs = []
    for fn in (hb.linear_batched, hb.linear_noalloc):
        c = torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
        descs = [hb.linear_desc(m, n, kb, a_d[i * len(a):(i + 1) * len(a)],
                                [w[i * len(p):(i + 1) * len(p)] for w, p in zip(w_d, planes)],
                                modes, c[i], ops=list(ops), mode=mode)
                 for i in range(layers)]
        fn(descs, gpu)
        outs.append(host_u32(c))
    return outs


def test_two_calls_in_a_row_second_smaller(gpu):
    rng = np.random.default_rng(11)
    # 1100 x 512 x 512 MXFP4: more than 1,024 rows on 36 tiles of 64 x 256,
    # so K splits through the array (2 splits, ~4.5 MB of partial sums)
    m, n, kb = 1100, 512, 16
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    say("call 1", dict(m=m, n=n, kb=kb))
    ref, got = run_both(gpu, m, n, kb, a, planes, modes, hb.FAST)
    assert np.array_equal(got, ref)
    want, _ = helpers.oracle_linear_mt(m, n, kb, a, planes, modes)
    helpers.check_fast(got[0], want)
    # smaller: 100 x 256 x 256 exact with MULP and ADDP (the deferred
    # epilogue's sums in the array) over what call 1 left
    m, n, kb = 100, 256, 8
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    scale = rng.uniform(0.5, 2.0, n).astype(np.float32)
    bias = rng.normal(0, 0.1, n).astype(np.float32)
    say("call 2", dict(m=m, n=n, kb=kb))
    ref, got = run_both(gpu, m, n, kb, a, planes, modes, hb.EXACT,
                        ops=[(hb.EP_MULP, dev(scale)), (hb.EP_ADDP, dev(bias))])
    assert np.array_equal(got, ref)
    want, _ = helpers.oracle_linear_mt(m, n, kb, a, planes, modes,
                                       ops=[(hb.EP_MULP, scale.view(np.uint32)),
                                            (hb.EP_ADDP, bias.view(np.uint32))])
    assert np.array_equal(got[0], want)


def test_exact_deferred_epilogue(gpu):
    rng = np.random.default_rng(12)
    m, n, kb = 100, 256, 8
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    scale = dev(rng.uniform(0.5, 2.0, n).astype(np.float32))
    bias = dev(rng.normal(0, 0.1, n).astype(np.float32))
    say("exact with ops", dict(m=m, n=n, kb=kb))
    ref, got = run_both(gpu, m, n, kb, a, planes, modes, hb.EXACT,
                        ops=[(hb.EP_MULP, scale), (hb.EP_ADDP, bias)])
    assert np.array_equal(got, ref)


def test_batched_and_skinny_need_no_scratch(gpu):
    rng = np.random.default_rng(13)
    m, n, kb = 128, 320, 16
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    say("batched x3", dict(m=m, n=n, kb=kb))
    ref, got = run_both(gpu, m, n, kb, a, planes, modes, hb.FAST, layers=3)
    assert np.array_equal(got, ref)
    m = 8
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    say("skinny", dict(m=m, n=n, kb=kb))
    ref, got = run_both(gpu, m, n, kb, a, planes, modes, hb.FAST)
    assert np.array_equal(got, ref)


def test_graph_capture_of_a_new_shape(gpu):
    rng = np.random.default_rng(14)
    ctx = hb.Context(0)
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    m, n, kb = 141, 640, 48  # never run before on this context
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    a_d, w_d = dev(a), [dev(p) for p in planes]
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc = hb.linear_desc(m, n, kb, a_d, w_d, modes, c_d, mode=hb.FAST)
    c_ref = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc_ref = hb.linear_desc(m, n, kb, a_d, w_d, modes, c_ref, mode=hb.FAST)
    # eager work between replays: another small layer through the same array
    m2, n2, kb2 = 72, 512, 32
    a2, planes2, modes2 = mxfp4_layer(rng, m2, n2, kb2)
    c2_d = torch.zeros((m2, n2), dtype=torch.float32, device=DEV)
    desc2 = hb.linear_desc(m2, n2, kb2, dev(a2), [dev(p) for p in planes2], modes2, c2_d,
                           mode=hb.FAST)
    try:
        # leave the context's own stream before capturing (that synchronizes
        # and destroys it, which a capture does not allow)
        ctx.set_stream(side.cuda_stream)
        g = torch.cuda.CUDAGraph()
        say("capture", dict(m=m, n=n, kb=kb))
        with torch.cuda.graph(g, stream=side):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            hb.linear_noalloc([desc], ctx)
        ctx.set_stream(main.cuda_stream)
        hb.linear_batched([desc_ref], ctx)
        ref = host_u32(c_ref)
        hb.linear_noalloc([desc2], ctx)
        want2 = host_u32(c2_d)
        for rep in range(3):
            c_d.zero_()
            say("replay", rep)
            g.replay()
            assert np.array_equal(host_u32(c_d), ref)
            c2_d.zero_()
            hb.linear_noalloc([desc2], ctx)
            assert np.array_equal(host_u32(c2_d), want2)
        del g
    finally:
        ctx.set_stream(main.cuda_stream)
        torch.cuda.synchronize()
        ctx.close()


def test_graph_capture_through_the_array(gpu):
    """A captured layer whose K splits meet in the fixed array (1,100 x 512
    x 512 fast: more than 1,024 rows on fewer than 128 tiles), replayed
    between eager calls that overwrite the array (an exact 100-row layer
    with MULP and ADDP, its epilogue deferred through the array): every
    replay and every eager call equals hb_linear_batched_async's result."""
    rng = np.random.default_rng(16)
    ctx = hb.Context(0)
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    m, n, kb = 1100, 512, 16
    a, planes, modes = mxfp4_layer(rng, m, n, kb)
    a_d, w_d = dev(a), [dev(p) for p in planes]
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc = hb.linear_desc(m, n, kb, a_d, w_d, modes, c_d, mode=hb.FAST)
    c_ref = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc_ref = hb.linear_desc(m, n, kb, a_d, w_d, modes, c_ref, mode=hb.FAST)
    m2, n2, kb2 = 100, 256, 8
    a2, planes2, modes2 = mxfp4_layer(rng, m2, n2, kb2)
    ops2 = [(hb.EP_MULP, dev(np.asarray(rng.uniform(0.5, 2.0, n2), np.float32))),
            (hb.EP_ADDP, dev(np.asarray(rng.normal(0, 0.1, n2), np.float32)))]
    a2_d, w2_d = dev(a2), [dev(p) for p in planes2]
    c2_d = torch.zeros((m2, n2), dtype=torch.float32, device=DEV)
    desc2 = hb.linear_desc(m2, n2, kb2, a2_d, w2_d, modes2, c2_d, ops=ops2, mode=hb.EXACT)
    c2_ref = torch.zeros((m2, n2), dtype=torch.float32, device=DEV)
    desc2_ref = hb.linear_desc(m2, n2, kb2, a2_d, w2_d, modes2, c2_ref, ops=ops2, mode=hb.EXACT)
    try:
        ctx.set_stream(main.cuda_stream)
        hb.linear_batched([desc_ref], ctx)
        hb.linear_batched([desc2_ref], ctx)
        ref, ref2 = host_u32(c_ref), host_u32(c2_ref)
        want, _ = helpers.oracle_linear_mt(m, n, kb, a, planes, modes)
        helpers.check_fast(ref, want)
        ctx.set_stream(side.cuda_stream)
        hb.linear_noalloc([desc], ctx)  # the shape once, outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        say("capture through the array", dict(m=m, n=n, kb=kb))
        with torch.cuda.graph(g, stream=side):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            hb.linear_noalloc([desc], ctx)
        ctx.set_stream(main.cuda_stream)
        for rep in range(3):
            c2_d.zero_()
            hb.linear_noalloc([desc2], ctx)  # overwrites the array
            assert np.array_equal(host_u32(c2_d), ref2), rep
            c_d.zero_()
            say("replay", rep)
            g.replay()
            assert np.array_equal(host_u32(c_d), ref), rep
        del g
    finally:
        ctx.set_stream(main.cuda_stream)
        torch.cuda.synchronize()
        ctx.close()


def test_oversize_layer_is_rejected(gpu):
    # 2048 x 512 x 2048 MXFP4: 64 tiles of 64 x 256 (more than 1,024 rows,
    # so the K-split route), 2 K splits: 8 MiB of partial sums, plus the
    # split counters and flags, over the 8 MiB array
    rng = np.random.default_rng(15)
    m, n, kb = 2048, 512, 64
    a = helpers.activations(rng, m, kb * 32)[1]
    w = torch.zeros((n // 8 * kb, 144), dtype=torch.uint8, device=DEV)
    c = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc = hb.linear_desc(m, n, kb, dev(a), [w], [0], c, mode=hb.FAST)
    say("oversize", dict(m=m, n=n, kb=kb))
    with pytest.raises(hb.HbError) as e:
        hb.linear_noalloc([desc], gpu)
    assert e.value.args[0].startswith("[5]") and "scratch" in e.value.args[0]
    torch.cuda.synchronize()
    assert float(c.abs().max()) == 0.0  # nothing ran
