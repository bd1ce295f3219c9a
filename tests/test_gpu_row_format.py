"""hb_row_load / hb_row_store (the DMA engine's MXINT8 row format, kinds
ROW and ROW_INDEXED; tools/iss/dma_engine.cpp:96-279) on an MI355X against
the oracle, bitwise on every output byte, and tokens of an MXINT8 matrix
loaded as the A of hb_linear."""
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


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def token_pool(rng, count, tok):
    size = hb.row_token_bytes(tok)
    t = np.zeros((count, size), np.uint8)
    t[:, :33 * tok] = rng.integers(0, 256, (count, 33 * tok), dtype=np.uint8)
    return t


@pytest.mark.parametrize("tok,rows,row_words,pad", [(3, 4, 3, 16), (17, 2, 2, 0), (1, 3, 4, 32),
                                                    (32, 1, 4, 0), (16, 5, 4, 48), (30, 64, 512, 0)])
def test_load_and_store(gpu, tok, rows, row_words, pad):
    rng = np.random.default_rng(tok * 100 + rows)
    size = hb.row_token_bytes(tok)
    stride = row_words * size + pad
    src = np.full(rows * stride, 0xEE, np.uint8)
    t = token_pool(rng, rows * row_words, tok)
    for r in range(rows):
        src[r * stride: r * stride + row_words * size] = t[r * row_words:(r + 1) * row_words].reshape(-1)
    n_words = rows * row_words // 4 * tok
    say("row load", dict(tok=tok, rows=rows, row_words=row_words, stride=stride))
    out = torch.full((n_words, 144), 0xA5, dtype=torch.uint8, device=DEV)
    src_d = dev(src)
    hb.row_load(src_d, rows, row_words, tok, out, stride, ctx=gpu)
    want = oracle.row_load(src, rows, row_words, tok, stride)
    got = host(out)
    assert np.array_equal(got, want), np.argwhere(got != want)[:3]
    say("row store", dict(tok=tok))
    back = torch.full((rows * stride,), 0xEE, dtype=torch.uint8, device=DEV)
    hb.row_store(out, rows, row_words, tok, back, stride, ctx=gpu)
    assert np.array_equal(host(back), src)
    assert np.array_equal(host(back), oracle.row_store(want, rows, row_words, tok, stride, fill=0xEE))


@pytest.mark.parametrize("tok", [1, 5, 32])
def test_indexed_load_with_null_entries(gpu, tok):
    rng = np.random.default_rng(7 + tok)
    size = hb.row_token_bytes(tok)
    pool = token_pool(rng, 40, tok)
    count = 24
    index = (rng.integers(0, 40, count) * (size // 16)).astype(np.uint32)
    index[[0, 5, 23]] = 0xFFFFFFFF
    say("row load indexed", dict(tok=tok))
    out = torch.full((count // 4 * tok, 144), 0xA5, dtype=torch.uint8, device=DEV)
    hb.row_load(dev(pool), 6, 4, tok, out, index=dev(index.view(np.int32)), ctx=gpu)
    want = oracle.row_load(pool, 6, 4, tok, index=index)
    assert np.array_equal(host(out), want)


def test_tokens_feed_a_linear_layer(gpu):
    """Token-major MXINT8 activations (141 tokens of 960) -> A words -> the
    MXFP4 projection 960 -> 960, exact, against the oracle on PackAbuf."""
    rng = np.random.default_rng(11)
    m, k, n = 141, 960, 960
    tok = k // 32
    mp = (m + 3) // 4 * 4
    x = np.zeros((mp, k), np.float32)
    x[:m] = rng.standard_normal((m, k))
    q, e = oracle.encode_mxint8(oracle.f32_bits(x))
    size = hb.row_token_bytes(tok)
    src = np.zeros((mp, size), np.uint8)
    src[:, :32 * tok] = q.view(np.uint8)
    src[:, 32 * tok: 33 * tok] = (e + 127).astype(np.uint8)
    a_d = torch.zeros((mp // 4 * tok, 144), dtype=torch.uint8, device=DEV)
    hb.row_load(dev(src), mp, 1, tok, a_d, ctx=gpu)
    a = oracle.pack_abuf(q, e)
    assert np.array_equal(host(a_d), a)
    code, ew = helpers.mxfp4_weights(rng, n, k)
    w = oracle.pack_wbuf(code, ew)
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    hb.linear(gpu, a=a_d, planes=[dev(w)], modes=[0], c=c_d, m=m, n=n, kb_total=tok)
    want, _ = oracle.linear(mp, n, tok, a, [w], [0])
    assert np.array_equal(host(c_d).view(np.uint32), want[:m])


@pytest.mark.parametrize("args,text", [
    ((1, 4, 0), "row format with tok = 0"), ((1, 4, 33), "row format with tok = 33"),
    ((3, 1, 2), "row format with 3 tokens, not a multiple of 4"),
    ((0, 4, 2), "a DMA transfer with 0 rows of 4 words"),
    ((4, 1000, 32), "row format with 1000 tokens of 1056 bytes per row")])
def test_rejections(gpu, args, text):
    rows, row_words, tok = args
    buf = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    with pytest.raises(hb.HbBadCommand) as err:
        hb.row_load(buf, rows, row_words, tok, buf, row_stride=16, ctx=gpu)
    assert err.value.message == text
    with pytest.raises(hb.HbError) as err:  # a stride that is not whole beats
        hb.row_load(buf, 1, 4, 1, buf, row_stride=200, ctx=gpu)
    assert err.value.code == hb.HB_EINVAL
