"""W8 panels on an MI355X: hb_pack_w8 and hb_unpack_w8 back to the DDR word
planes (tools/compiler/weights.cpp:72-88 SplitW8, tensors.cpp:66-90
PackWbuf) bit for bit, the packer's per-panel window flags against the
scale bytes, and W8 layers over W8 panels against the oracle's layer over
the same planes as DDR words (tools/iss/gemm_array.cpp:112-149 folded as
tools/compiler/kernels.cpp:343-395): exact mode bitwise, fast mode within
the fast-mode tolerance (normwise per row, and per element against the
block sums) -- every tile width of the W8 kernel, partial panels and tiles,
odd block counts, one row, onto C, every epilogue op, requantize, batched
layers, all 256 int8 codes of A, A and W scale bytes outside the fast
path's window (those waves fold exactly), and the SigLIP encoder's four
GEMM shapes at M = 2048."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
from test_gpu_bench_routes import DEV, dev, host, per_channel, say, w8_planes

pytestmark = pytest.mark.gpu


def random_planes(rng, n, kb, lo=120, hi=140):
    """Two W8 DDR word planes of random nibbles, each plane with its own
    random scale bytes in [lo, hi]; bytes 136..143 zero."""
    planes = []
    for _ in range(2):
        w = rng.integers(0, 256, (n // 8, kb, 144), dtype=np.uint8)
        w[:, :, 128:136] = rng.integers(lo, hi + 1, (n // 8, kb, 8), dtype=np.uint8)
        w[:, :, 136:] = 0
        planes.append(w.reshape(-1, 144))
    return planes


def pack(gpu, planes_d, n, kb):
    out = torch.full((hb.w8_panel_bytes(n, kb),), 0xA5, dtype=torch.uint8, device=DEV)
    hb.pack_w8(planes_d[0], planes_d[1], n, kb, out, ctx=gpu)
    return out


def panel_flags_expected(planes, n, kb):
    """Per 64-column panel: a scale byte of a column-block of either plane
    outside [70, 179]."""
    n_panels = (n + 63) // 64
    out = np.zeros(n_panels, bool)
    for w in planes:
        s = w.reshape(n // 8, kb, 144)[:, :, 128:136]  # [group][block][column in group]
        col = (np.arange(n // 8)[:, None, None] * 8 + np.arange(8)[None, None, :])
        col = np.broadcast_to(col, s.shape)
        bad = (s < 70) | (s > 179)
        np.logical_or.at(out, col[bad] // 64, True)
    return out


@pytest.mark.parametrize("n,kb", [(8, 1), (72, 3), (768, 24), (200, 96), (2304, 23)])
def test_pack_and_unpack(gpu, n, kb):
    rng = np.random.default_rng(n * 7 + kb)
    planes = random_planes(rng, n, kb, lo=60, hi=190)  # some scale bytes outside the window
    say("pack_w8", dict(n=n, kb=kb))
    p_d = pack(gpu, [dev(p) for p in planes], n, kb)
    n_panels, steps = (n + 63) // 64, (kb + 1) // 2
    assert hb.w8_panel_bytes(n, kb) == n_panels * steps * 6400 + (n_panels * 4 + 15) // 16 * 16
    flags = host(p_d)[n_panels * steps * 6400:][:n_panels * 4].view(np.uint32)
    assert np.array_equal(flags != 0, panel_flags_expected(planes, n, kb))
    hi = torch.full((n // 8 * kb, 144), 0x5A, dtype=torch.uint8, device=DEV)
    lo = torch.full_like(hi, 0x3C)
    hb.unpack_w8(p_d, n, kb, hi, lo, ctx=gpu)
    assert np.array_equal(host(hi), planes[0])
    assert np.array_equal(host(lo), planes[1])


def test_pack_rejects_bad_arguments(gpu):
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=DEV)
    for args in ((buf, buf, 12, 3, buf), (buf, buf, 8, 0, buf), (buf[1:], buf, 8, 1, buf),
                 (buf, buf, 8, 1, buf[4:])):
        with pytest.raises(hb.HbError) as err:
            hb.pack_w8(*args, ctx=gpu)
        assert err.value.code == hb.HB_EINVAL


def test_descriptor_rules(gpu):
    """W8 panels need planes {W8_HI, W8_LO} on one buffer and one piece."""
    m, n, kb = 8, 64, 2
    rng = np.random.default_rng(5)
    planes, _ = w8_planes(rng, n, kb)
    p_d = pack(gpu, [dev(p) for p in planes], n, kb)
    a_d = dev(helpers.activations(rng, m, kb * 32)[1])
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    for kw, code in ((dict(planes=[p_d, p_d[16:]], modes=[1, 2]), hb.HB_EINVAL),
                     (dict(planes=[p_d], modes=[1]), hb.HB_EINVAL),
                     (dict(planes=[p_d, p_d], modes=[1, 2], pieces=[(0, 1), (1, 1)]),
                      hb.HB_EUNSUPPORTED)):
        with pytest.raises(hb.HbError) as err:
            hb.linear(gpu, a=a_d, c=c_d, m=m, n=n, kb_total=kb, mode=hb.FAST, w8_panels=True, **kw)
        assert err.value.code == code, kw


def w8_layer(gpu, m, n, kb, mode, ops_fn=None, quantize=False, tbuf=None, all_codes=False,
             onto=False, seed=0, planes_fn=None, bad_a=False, layers=1):
    """`layers` W8 layers of one shape over W8 panels (one launch); every
    layer checked against the oracle over the DDR planes."""
    rng = np.random.default_rng(seed)
    a_h, pl_h, ops_h, c0_h = [], [], [], []
    for _ in range(layers):
        a = helpers.random_a_words(rng, m, kb) if all_codes else \
            helpers.activations(rng, m, kb * 32)[1]
        if bad_a:  # a few rows' scale bytes outside the window
            a.reshape(-1, kb, 144)[::7, kb // 2, 128 + 1] = 50
        a_h.append(a)
        pl_h.append(planes_fn(rng, n, kb) if planes_fn else w8_planes(rng, n, kb)[0])
        ops_h.append(ops_fn(rng, m, n) if ops_fn else [])
        c0_h.append(helpers.random_fp32_words(rng, (m, n), 118, 128) if onto else None)
    a_d = dev(np.stack(a_h))
    pb = hb.w8_panel_bytes(n, kb)
    p_d = torch.empty((layers, pb), dtype=torch.uint8, device=DEV)
    for i in range(layers):
        p_d[i] = pack(gpu, [dev(p) for p in pl_h[i]], n, kb)
    c_d = dev(np.stack(c0_h).view(np.float32)) if onto else \
        torch.zeros((layers, m, n), dtype=torch.float32, device=DEV)
    q_d = torch.zeros((layers, (m + 3) // 4 * (n // 32), 144), dtype=torch.uint8, device=DEV) \
        if quantize else None
    tb_d = dev(tbuf.view(np.int64)) if tbuf is not None else None
    # op operands: one device array per op kind over the layers
    kinds = [k for k, _ in ops_h[0]]
    op_d = []
    for j, k in enumerate(kinds):
        vals = [ops_h[i][j][1] for i in range(layers)]
        op_d.append(dev(np.stack(vals).view(np.float32)) if isinstance(vals[0], np.ndarray)
                    else None)
    descs = []
    for i in range(layers):
        ops = [(k, op_d[j][i] if op_d[j] is not None else ops_h[i][j][1])
               for j, k in enumerate(kinds)]
        descs.append(hb.linear_desc(m, n, kb, a_d[i], [p_d[i], p_d[i]], [1, 2], c_d[i], ops=ops,
                                    tbuf=tb_d, q_out=q_d[i] if quantize else None, mode=mode,
                                    onto=onto, w8_panels=True))
    torch.cuda.synchronize()
    say("w8 panels", dict(m=m, n=n, kb=kb, mode=mode, ops=kinds, quantize=quantize,
                          all_codes=all_codes, onto=onto, bad_a=bad_a, layers=layers))
    hb.linear_batched(descs, gpu)
    got = host(c_d).view(np.uint32)
    gq = host(q_d) if quantize else None
    for i in range(layers):
        want, wq = helpers.oracle_linear_mt(m, n, kb, a_h[i], pl_h[i], [1, 2], ops=ops_h[i],
                                            tbuf=tbuf, quantize=quantize, onto=c0_h[i])
        if mode == hb.EXACT:
            assert np.array_equal(got[i], want), i
            if quantize:
                assert np.array_equal(gq[i], wq), i
        else:
            bound = None if (onto or ops_h[i]) else \
                helpers.block_abs_sums(m, n, kb, a_h[i], pl_h[i], [1, 2])
            helpers.check_fast(got[i], want, gq[i] if quantize else None, wq, bound=bound)


# ---- the tile widths (1 to 4 panels, chosen by rows and column count) ----

@pytest.mark.parametrize("m,n,kb", [
    (128, 256, 12),    # 1 panel per tile, 4 tiles
    (256, 768, 24),    # out-proj width
    (128, 2304, 8),    # QKV width
    (200, 72, 3),      # a partial last panel and tile, odd blocks
    (1, 96, 5),        # one row
    (131, 512, 1),     # one block
    (2048, 1536, 4),   # 2 panels per tile (192 tiles)
    (2048, 2304, 5),   # 3 panels (192 tiles), odd blocks
    (2048, 4096, 4)])  # 4 panels (256 tiles)
def test_fast_shapes(gpu, m, n, kb):
    w8_layer(gpu, m, n, kb, hb.FAST, seed=m + n + kb)


def test_fast_independent_plane_scales(gpu):
    """hi and lo planes with different random scale bytes and nibbles."""
    w8_layer(gpu, 160, 320, 9, hb.FAST, seed=11, planes_fn=random_planes)


def test_fast_all_codes_onto(gpu):
    w8_layer(gpu, 128, 256, 12, hb.FAST, all_codes=True, onto=True, seed=12)


def test_fast_batched(gpu):
    w8_layer(gpu, 130, 200, 7, hb.FAST, layers=3, seed=13)


def test_fast_out_of_window_scales(gpu):
    """W scale bytes outside the window in some panels (the packer's flags)
    and A scale bytes outside it in some rows: those waves fold exactly."""
    w8_layer(gpu, 256, 640, 6, hb.FAST, seed=14,
             planes_fn=lambda r, n, kb: random_planes(r, n, kb, lo=60, hi=130))
    w8_layer(gpu, 256, 384, 10, hb.FAST, seed=15, bad_a=True)


@pytest.mark.parametrize("mode", [hb.FAST, hb.EXACT])
def test_every_op_and_requantize(gpu, mode):
    tb = helpers.activation_table("silu")

    def ops(r, m, n):
        return per_channel(r, n) + [
            (hb.EP_SCALE, int(np.float32(0.75).view(np.uint32))),
            (hb.EP_ADD, helpers.random_fp32_words(r, (m, n), 118, 128)),
            (hb.EP_RELU, None), (hb.EP_COPY, None),
            (hb.EP_ACT_MUL, helpers.random_fp32_words(r, (m, n), 120, 130))]
    w8_layer(gpu, 132, 192, 7, mode, ops, quantize=True, tbuf=tb, seed=16)


@pytest.mark.parametrize("m,n,kb,onto,codes", [(64, 96, 3, False, False), (133, 200, 5, True, True)])
def test_exact_bitwise(gpu, m, n, kb, onto, codes):
    w8_layer(gpu, m, n, kb, hb.EXACT, onto=onto, all_codes=codes, seed=17 + m,
             planes_fn=random_planes)


# ---- the SigLIP encoder's GEMMs at M = 2 x 1024 patches (fast) ----

def test_siglip_qkv(gpu):
    w8_layer(gpu, 2048, 2304, 24, hb.FAST, lambda r, m, n: per_channel(r, n), seed=21)


def test_siglip_out_proj(gpu):
    w8_layer(gpu, 2048, 768, 24, hb.FAST, lambda r, m, n: per_channel(r, n), seed=22)


def test_siglip_mlp_up_gelu_requantize(gpu):
    w8_layer(gpu, 2048, 3072, 24, hb.FAST, lambda r, m, n: per_channel(r, n, True),
             quantize=True, tbuf=helpers.activation_table("gelu"), seed=23)


def test_siglip_mlp_down(gpu):
    w8_layer(gpu, 2048, 768, 96, hb.FAST, lambda r, m, n: per_channel(r, n), seed=24)
