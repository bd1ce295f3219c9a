"""The context workspace (K-split partial sums of small fast-mode layers) and
HIP graphs: a graph captured over a small layer keeps working after a later,
larger small layer has grown the workspace (the superseded buffer is
retired, not freed, until the context is destroyed).  Each replay runs
between eager work on the same context and is checked against the oracle
(tolerance as for every fast-mode layer)."""
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


def layer(rng, m, n, kb):
    a = helpers.activations(rng, m, kb * 32)[1]
    code, e = helpers.mxfp4_weights(rng, n, kb * 32)
    w = oracle.pack_wbuf(code, e)
    return a, w


def test_graph_survives_workspace_growth():
    rng = np.random.default_rng(5)
    ctx = hb.Context(0)
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    # small layer: 141 x 320 x 960 (4 tiles: K-split path, workspace ~1.5 MB)
    m, n, kb = 141, 320, 30
    a, w = layer(rng, m, n, kb)
    a_d, w_d = dev(a), dev(w)
    c_d = torch.zeros((m, n), dtype=torch.float32, device=DEV)
    desc = hb.linear_desc(m, n, kb, a_d, [w_d], [0], c_d, mode=hb.FAST)
    want, _ = helpers.oracle_linear_mt(m, n, kb, a, [w], [0])
    # larger small layer: 141 x 2048 x 2560 (16 tiles, workspace ~9 MB)
    m2, n2, kb2 = 141, 2048, 80
    a2, w2 = layer(rng, m2, n2, kb2)
    a2_d, w2_d = dev(a2), dev(w2)
    c2_d = torch.zeros((m2, n2), dtype=torch.float32, device=DEV)
    desc2 = hb.linear_desc(m2, n2, kb2, a2_d, [w2_d], [0], c2_d, mode=hb.FAST)
    want2, _ = helpers.oracle_linear_mt(m2, n2, kb2, a2, [w2], [0])
    try:
        say("warm up the small layer on the capture stream")
        with torch.cuda.stream(side):
            ctx.set_stream(side.cuda_stream)
            hb.launch(desc, ctx)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            ctx.set_stream(torch.cuda.current_stream().cuda_stream)
            hb.launch(desc, ctx)
        ctx.set_stream(main.cuda_stream)
        say("grow the workspace with the larger layer")
        hb.launch(desc2, ctx)
        torch.cuda.synchronize()
        helpers.check_fast(c2_d.cpu().numpy().view(np.uint32), want2)
        for rep in range(3):
            c_d.zero_()
            say("replay", rep)
            g.replay()
            torch.cuda.synchronize()
            helpers.check_fast(c_d.cpu().numpy().view(np.uint32), want)
            c2_d.zero_()
            hb.launch(desc2, ctx)  # eager work on the same context between replays
            torch.cuda.synchronize()
            helpers.check_fast(c2_d.cpu().numpy().view(np.uint32), want2)
        del g
    finally:
        ctx.set_stream(main.cuda_stream)
        torch.cuda.synchronize()
        ctx.close()
