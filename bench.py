"""Benchmark: quantized GEMM TOPS and roofline fraction on one MI355X.

Headline workload: an MXFP4 linear layer, weights E2M1 [N=960][K=2560] with
E8M0 block-32 scales (exponents -10..-2), MXINT8 activations [M=128][K=2560]
from N(0,1), FP32 output, fast mode (block-scaled FP6 x FP4 matrix cores,
FP32 accumulation order differs from the NPU's; max relative error <= 1e-5).
One step = one pass over L independent layers of that shape (distinct weights
and activations, L * 2.1 MB > the 256 MB last-level cache) in one batched
launch; inputs are resident in HBM before timing starts.

Extra fields (skipped with --quick): the same workload in exact mode (bitwise
equal to the NPU), the M sweep {1, 16, 1024} in fast mode, the W8 layer
M=64 K=960 N=2560 with per-channel scale (MULP) and bias (ADDP), the
SigLIP-style W8 encoder set (M=2048), the SparseDrive-S stage-1 3x3 conv
GEMM (MXFP4, M=67584 K=576 N=64), each in fast and exact mode, the
SmolVLA action-expert step (its GEMM chain) and the SmolVLA LM prefix (its
16 MXFP4 decoder layers' GEMMs) at batch 1 and 32.

    python bench.py [--steps K] [--warmup W] [--mode exact|fast] [--layers L]
                    [--quick] [--no-cpu] [--copy-probe MIB] [--settle S]

Prints one JSON line.  The CPU baseline times the oracle (a C restatement of
the reference's CPU path, single thread) on one layer of the same shape.
--copy-probe copies MIB MiB on the device three times first (a plain copy of
known size, to calibrate HBM byte counters under a profiler).  --settle runs
the headline untimed for S seconds before its warmup steps, so the clocks
have reached their sustained-load state (default 0.5; 0 under a counter
profiler, which would otherwise sample every one of those launches).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
# Dense MFMA peaks (TFLOP/s or TOPS) of the instruction class each kernel uses.
MFMA_PEAK = {"bf16": 2500.0, "fp6_fp4": 10100.0, "int8": 5000.0, "fp8": 5000.0}
METRIC = "quantized GEMM TOPS & % MFMA/HBM roofline (W8, MXFP4); SmolVLA step ms"
PROFILES = os.path.join(ROOT, "profiles")


def layer_bytes(m, n, kb, w_bits, n_vectors=0):
    """Algorithmic bytes of one layer: A MXINT8 + W (E8M0 per 32) + C fp32
    + fp32 epilogue vectors."""
    k = kb * 32
    return m * k * (1 + 1 / 32) + n * k * (w_bits / 8 + 1 / 32) + 4 * m * n + 4 * n * n_vectors


def make_inputs(rng, m, n, kb, w8=False):
    """Synthetic operands in DDR word layout, generated directly (no oracle):
    A words [m/4][kb][144] (MXINT8 of N(0,1) rows), W words [n/8][kb][144]
    per plane.  MXFP4: random E2M1 codes, E8M0 exponents -10..-2.  W8: int8
    weights U{-127..127} encoded MXINT8 (lossless, scale byte 133) and split
    into the hi (signed) and lo (unsigned) nibble planes."""
    quads = (m + 3) // 4
    a = np.zeros((quads, kb, 144), np.uint8)
    x = rng.standard_normal((quads * 4, kb, 32)).astype(np.float32)
    amax = np.abs(x).max(axis=2)
    e = np.floor(np.log2(np.maximum(amax, 1e-30))).astype(np.int32)
    q = np.clip(np.rint(x * np.exp2(6 - e)[..., None]), -128, 127).astype(np.int8)
    a[:, :, :128] = q.reshape(quads, 4, kb, 32).transpose(0, 2, 1, 3).reshape(quads, kb, 128).view(np.uint8)
    a[:, :, 128:132] = (e + 127).reshape(quads, 4, kb).transpose(0, 2, 1).astype(np.uint8)
    if not w8:
        w = np.zeros((n // 8, kb, 144), np.uint8)
        w[:, :, :128] = rng.integers(0, 256, (n // 8, kb, 128), dtype=np.uint8)
        w[:, :, 128:136] = (127 + rng.integers(-10, -1, (n // 8, kb, 8))).astype(np.uint8)
        return a.reshape(-1, 144), [w.reshape(-1, 144)]
    qw = rng.integers(-127, 128, (n, kb * 32)).astype(np.int8).view(np.uint8)
    planes = []
    for nib in (qw >> 4, qw & 15):  # hi plane code, lo plane code
        w = np.zeros((n // 8, kb, 144), np.uint8)
        v = nib.reshape(n // 8, 8, kb, 16, 2)
        w[:, :, :128] = (v[..., 0] | (v[..., 1] << 4)).transpose(0, 2, 1, 3).reshape(n // 8, kb, 128)
        w[:, :, 128:136] = 133
        planes.append(w.reshape(-1, 144))
    return a.reshape(-1, 144), planes


def cpu_baseline(m, n, kb, budget_s=15.0):
    """Single-thread oracle (the reference CPU path restated in C) on one
    layer; repeats while the budget allows and reports the median."""
    import oracle
    rng = np.random.default_rng(7)
    a, w = make_inputs(rng, m, n, kb)
    times = []
    t_end = time.perf_counter() + budget_s
    while True:
        t0 = time.perf_counter()
        oracle.linear(m, n, kb, a, w, [0])
        times.append(time.perf_counter() - t0)
        if time.perf_counter() + times[-1] > t_end or len(times) >= 5:
            break
    t = float(np.median(times))
    return {"value": round(2.0 * m * n * kb * 32 / t / 1e12, 6), "unit": "TOPS", "cores": 1,
            "kind": "port",
            "sample": f"{len(times)} run(s) of one {m}x{kb * 32}x{n} MXFP4 layer (exact fold), "
                      f"median {t:.3f} s"}


def cpu_baseline_cores(m, n, kb, budget_s=10.0):
    """The same layer on several host threads, each running the oracle over
    its own slice of column groups (independent in the reference's loop nest,
    gemm_array.cpp:123-147).  Threads: the host's cores, at most 16 (one
    GPU's share of a GPU box's cores)."""
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    rng = np.random.default_rng(7)
    a, w = make_inputs(rng, m, n, kb)
    groups = n // 8
    threads = max(1, min(16, os.cpu_count() or 1, groups))
    bounds = [groups * i // threads for i in range(threads + 1)]
    w0 = w[0].reshape(groups, kb, 144)
    slices = [np.ascontiguousarray(w0[bounds[i]:bounds[i + 1]]).reshape(-1, 144)
              for i in range(threads)]

    def part(i):  # ctypes releases the GIL for the duration of the call
        oracle.linear(m, 8 * (bounds[i + 1] - bounds[i]), kb, a, [slices[i]], [0])

    times = []
    t_end = time.perf_counter() + budget_s
    with ThreadPoolExecutor(threads) as pool:
        while True:
            t0 = time.perf_counter()
            list(pool.map(part, range(threads)))
            times.append(time.perf_counter() - t0)
            if time.perf_counter() + times[-1] > t_end or len(times) >= 5:
                break
    t = float(np.median(times))
    return {"value": round(2.0 * m * n * kb * 32 / t / 1e12, 6), "unit": "TOPS", "cores": threads,
            "kind": "port",
            "sample": f"{len(times)} run(s) of one {m}x{kb * 32}x{n} MXFP4 layer (exact fold) "
                      f"over {threads} threads by column groups, median {t:.3f} s"}


def counted_traffic(line):
    """HBM bytes per pass of a bench line, from the committed rocprofv3
    counter summary (FETCH_SIZE and WRITE_SIZE over the pass's dispatches,
    calibrated against a device copy of known size; `--profile-lines` makes
    it), or None when the summary has no row for the line."""
    path = os.path.join(PROFILES, "hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for row in open(path):
        m = re.match(r"\|\s*" + re.escape(line) + r"\s*\|.*\|\s*([0-9]+)\s*\|\s*$", row)
        if m:
            return int(m.group(1))
    return None


class Workload:
    """L layers of one shape on the device, with their descriptors.  Every
    layer's A is MXINT8 of its own N(0,1) fp32 matrix (hb_encode_mxint8:
    EncodeMxint8 + PackAbuf, max-abs rule); MXFP4 W has random E2M1 codes and
    E8M0 exponents uniform in [-10, -2]; W8 W is two nibble planes of random
    codes (int8 weights uniform over [-128, 127]) sharing the scale byte 133
    (MXINT8 of int8 values).  All drawn on the device from a seeded
    generator.  panels: the weights are packed once (hb_pack_weights) and the
    layers read the panels."""

    def __init__(self, hb, torch, ctx, m, n, kb, w8, layers, mode, epilogue=False, seed=1,
                 panels=False, a_fp8=False):
        dev = "cuda:0"
        self.m, self.n, self.kb, self.w8, self.layers = m, n, kb, w8, layers
        self.n_vectors = 2 if epilogue else 0
        self.panels = panels
        L, quads = layers, (m + 3) // 4
        g = torch.Generator(device=dev).manual_seed(seed)
        self.a = torch.empty((L, quads * kb, 144), dtype=torch.uint8, device=dev)
        for i in range(L):
            x = torch.randn((m, kb * 32), generator=g, device=dev)
            (hb.encode_mxfp8 if a_fp8 else hb.encode_mxint8)(x, m, kb * 32, self.a[i], ctx=ctx)
            del x
        planes = 2 if w8 else 1
        w = [torch.randint(0, 256, (L, n // 8 * kb, 144), generator=g, device=dev,
                           dtype=torch.uint8) for _ in range(planes)]
        for p in w:
            p[:, :, 136:] = 0
            if w8:
                p[:, :, 128:136] = 133
            else:
                p[:, :, 128:136] = torch.randint(117, 126, (L, n // 8 * kb, 8), generator=g,
                                                 device=dev, dtype=torch.uint8)
        if panels:
            pb = hb.panel_bytes(n, kb)
            self.w = [torch.empty((L, pb), dtype=torch.uint8, device=dev) for _ in range(planes)]
            for p in range(planes):
                for i in range(L):
                    hb.pack_weights(w[p][i], n, kb, self.w[p][i], ctx=ctx)
            del w
        else:
            self.w = w
        self.c = torch.zeros((L, m, n), dtype=torch.float32, device=dev)
        ops_t = []
        if epilogue:  # per-channel scale ~ U(0.001, 0.02), bias ~ N(0, 0.1)
            self.scale = torch.rand((L, n), generator=g, device=dev) * 0.019 + 0.001
            self.bias = torch.randn((L, n), generator=g, device=dev) * 0.1
            ops_t = [(hb.EP_MULP, self.scale), (hb.EP_ADDP, self.bias)]
        modes = [1, 2] if w8 else [0]
        self.descs = [hb.linear_desc(m, n, kb, self.a[i], [p[i] for p in self.w], modes,
                                     self.c[i], ops=[(k, t[i]) for k, t in ops_t], mode=mode,
                                     panels=panels, a_fp8=a_fp8)
                      for i in range(L)]
        torch.cuda.synchronize()

    def ops(self):
        return 2.0 * self.m * self.n * self.kb * 32 * self.layers

    def bytes(self):
        return layer_bytes(self.m, self.n, self.kb, 8 if self.w8 else 4, self.n_vectors) * self.layers


def activation_table(kind="silu"):
    """A 1024-entry TBUF in the layout of tools/compiler/tensors.cpp:28-62:
    [0, 512) 2^(i/512), [512, 1024) the activation at i/32, each entry
    {slope: hi32, value: lo32} as fp32 bits."""
    seg = 512
    i = np.arange(seg + 1, dtype=np.float64)
    x = i / 32.0
    act = 1.0 / (1.0 + np.exp(-x)) if kind == "silu" else \
        0.5 * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))
    out = np.zeros(1024, np.uint64)
    for base, v in ((0, np.exp2(i / seg)), (512, act)):
        vb = v.astype(np.float32)
        slope = (vb[1:].astype(np.float64) - vb[:-1].astype(np.float64)).astype(np.float32)
        out[base:base + seg] = (slope.view(np.uint32).astype(np.uint64) << np.uint64(32)) | \
            vb[:-1].view(np.uint32).astype(np.uint64)
    return out


class Chain:
    """A sequence of linear layers on synthetic device data, one descriptor
    per layer, run in order on one stream.  MXINT8 activation words carry
    random codes with scale bytes 122..127; MXFP4 weight words random codes
    with E8M0 exponents in [lo, hi]; W8 weights are two nibble planes of
    random codes sharing the scale byte 133 (MXINT8 of int8 values)."""

    def __init__(self, hb, torch, m, mode, seed, w8_panels=False, panels=False):
        self.hb, self.torch, self.m, self.mode = hb, torch, m, mode
        self.w8_panels = w8_panels  # W8 layers over W8 panels (packed once, here)
        # every weight plane (MXFP4, or each W8 nibble plane) in weight panels
        # (hb_pack_weights, once, here), the layout fast-mode kernels stream
        self.panels = panels
        self.dev = "cuda:0"
        self.g = torch.Generator(device=self.dev).manual_seed(seed)
        self.quads = (m + 3) // 4
        self.descs, self.keep, self.ops, self.bytes = [], [], 0.0, 0.0
        # launch plan: lists of descriptor indices; a list of several is one
        # hb_linear_group_async call (grouped=False: every layer on its own)
        self.plan, self.grouped, self._arrays = [], True, None

    def a_words(self, kb):
        t = self.torch.randint(0, 256, (self.quads * kb, 144), generator=self.g, device=self.dev,
                               dtype=self.torch.uint8)
        t[:, 128:132] = self.torch.randint(122, 128, (self.quads * kb, 4), generator=self.g,
                                           device=self.dev, dtype=self.torch.uint8)
        t[:, 132:] = 0
        self.keep.append(t)
        return t

    def w_words(self, n, kb, lo=-10, hi=-2):
        t = self.torch.randint(0, 256, (n // 8 * kb, 144), generator=self.g, device=self.dev,
                               dtype=self.torch.uint8)
        t[:, 128:136] = self.torch.randint(127 + lo, 127 + hi + 1, (n // 8 * kb, 8),
                                           generator=self.g, device=self.dev,
                                           dtype=self.torch.uint8)
        t[:, 136:] = 0
        self.keep.append(t)
        return t

    def w8(self, n, kb):
        return [self.w_words(n, kb, 6, 6), self.w_words(n, kb, 6, 6)]

    def f32(self, n, scale=1.0):
        t = self.torch.randn((self.m, n), generator=self.g, device=self.dev) * scale
        self.keep.append(t)
        return t

    def vec(self, n, scale, offset=0.0):
        t = self.torch.randn((n,), generator=self.g, device=self.dev) * scale + offset
        self.keep.append(t)
        return t

    def table(self, kind):
        tb = self.torch.from_numpy(activation_table(kind).view(np.int64)).to(self.dev)
        self.keep.append(tb)
        return tb

    def add(self, n, kb, a, planes, c, ops=(), q=None, onto=False, tbuf=None, c_out=True):
        """c_out=False: the model keeps only the requantized words q (the
        NPU leaves the fp32 result in its on-chip FBUF): not counted in the
        algorithmic bytes; with c None the layer does not write it either."""
        modes = [1, 2] if len(planes) == 2 else [0]
        w8p = self.w8_panels and len(planes) == 2
        pan_flag = False
        if w8p or self.panels:
            # the packers run on the default context's own stream: the weight
            # words drawn on torch's stream must be complete first
            self.torch.cuda.synchronize()
        if w8p:
            pan = self.torch.empty((self.hb.w8_panel_bytes(n, kb),), dtype=self.torch.uint8,
                                   device=self.dev)
            self.hb.pack_w8(planes[0], planes[1], n, kb, pan)
            self.keep.append(pan)
            planes = [pan, pan]
        elif self.panels:
            packed = []
            for p in planes:
                pan = self.torch.empty((self.hb.panel_bytes(n, kb),), dtype=self.torch.uint8,
                                       device=self.dev)
                self.hb.pack_weights(p, n, kb, pan)
                self.keep.append(pan)
                packed.append(pan)
            planes, pan_flag = packed, True
        self.descs.append(self.hb.linear_desc(self.m, n, kb, a, planes, modes, c, ops=ops,
                                              tbuf=tbuf, q_out=q, onto=onto, mode=self.mode,
                                              w8_panels=w8p, panels=pan_flag))
        self.plan.append([len(self.descs) - 1])
        self.ops += 2.0 * self.m * n * kb * 32
        vectors = sum(1 for k, _ in ops if k in (self.hb.EP_ADDP, self.hb.EP_MULP))
        # C (fp32) counts where the model stores it; the MXINT8 words (codes
        # and scale bytes) come on top, and every [m][n] operand (ADD,
        # ACT_MUL) and an `onto` C are read in full
        matrices = sum(1 for k, _ in ops if k in (self.hb.EP_ADD, self.hb.EP_ACT_MUL))
        self.bytes += layer_bytes(self.m, n, kb, 8 if len(planes) == 2 else 4, vectors) - \
            (0 if c_out or q is None else 4 * self.m * n) + \
            (self.m * n * (1 + 1 / 32) if q is not None else 0) + \
            4 * self.m * n * (matrices + (1 if onto else 0))

    def group(self, k):
        """The last k layers added form one group launch (layers the model
        computes from the same inputs, or a gated pair)."""
        self.plan[-k:] = [sum(self.plan[-k:], [])]

    def run(self, ctx):
        if not self.grouped:
            for d in self.descs:
                self.hb.launch(d, ctx)
            return
        if self._arrays is None:
            self._arrays = [self.descs[p[0]] if len(p) == 1 else
                            (type(self.descs[0]) * len(p))(*[self.descs[i] for i in p])
                            for p in self.plan]
        for p, arr in zip(self.plan, self._arrays):
            if len(p) == 1:
                self.hb.launch(arr, ctx)
            else:
                self.hb.linear_group(arr, ctx)


class ExpertStep(Chain):
    """One SmolVLA action-expert step as the GEMM chain the reference compiler
    emits for it (tools/compiler/smolvla_expert.cpp:250-420, 430-545): 16
    layers of width 720 (K 736), 15 query / 5 KV heads of 64, SiLU-gated MLP
    of 2048 (1920 rounded up to a multiple of 256, as the reference sizes it),
    on a chunk of 50 action tokens per batch element.  Per layer: q (and k, v
    on the self-attention layers, the even ones) requantized to MXINT8; o
    with the residual add; up; gate with ACT_MUL(up) and requantize; down
    with the residual add.  Then the W8 head GEMMs: action_in (+bias,
    requantize), mlp_in from action and time (+bias, SiLU, requantize),
    mlp_out (+bias), action_out (+bias).  MXFP4 weights except the W8 heads.
    Attention, RMSNorm and RoPE are outside this path: their outputs are
    synthetic MXINT8 tensors of the right shape."""

    WIDTH, KB, Q, KV, HID, KBQ, KBH, LAYERS, CHUNK, ACT = 720, 23, 960, 320, 2048, 30, 64, 16, 50, 32

    def __init__(self, hb, torch, batch, mode, panels=False):
        super().__init__(hb, torch, self.CHUNK * batch, mode, 11 + batch, panels=panels)
        tb = self.table("silu")
        x = [self.f32(self.WIDTH) for _ in range(3)]
        for layer in range(self.LAYERS):
            a1, ao, a2 = self.a_words(self.KB), self.a_words(self.KBQ), self.a_words(self.KB)
            heads = [("q", self.Q)] + ([("k", self.KV), ("v", self.KV)] if layer % 2 == 0 else [])
            for _, n in heads:
                self.add(n, self.KB, a1, [self.w_words(n, self.KB)], self.f32(n),
                         q=self.a_words(n // 32))
            self.group(len(heads))
            self.add(self.WIDTH, self.KBQ, ao, [self.w_words(self.WIDTH, self.KBQ)], x[1],
                     ops=[(hb.EP_ADD, x[0])])
            up = self.f32(self.HID)
            self.add(self.HID, self.KB, a2, [self.w_words(self.HID, self.KB)], up)
            h = self.a_words(self.KBH)
            self.add(self.HID, self.KB, a2, [self.w_words(self.HID, self.KB)], self.f32(self.HID),
                     ops=[(hb.EP_ACT_MUL, up)], q=h, tbuf=tb)
            self.group(2)
            self.add(self.WIDTH, self.KBH, h, [self.w_words(self.WIDTH, self.KBH)], x[2],
                     ops=[(hb.EP_ADD, x[1])])
        act, tim, hid, xin = self.a_words(1), self.a_words(self.KB), self.a_words(self.KB), \
            self.a_words(self.KB)
        pad = self.KB * 32
        self.add(pad, 1, act, self.w8(pad, 1), self.f32(pad), ops=[(hb.EP_ADDP, self.vec(pad, 0.1))],
                 q=xin)
        mlp_in = self.f32(pad)
        self.add(pad, self.KB, xin, self.w8(pad, self.KB), mlp_in)
        self.add(pad, self.KB, tim, self.w8(pad, self.KB), mlp_in, onto=True,
                 ops=[(hb.EP_ADDP, self.vec(pad, 0.1)), (hb.EP_ACT, None)], q=hid, tbuf=tb)
        self.add(self.WIDTH, self.KB, hid, self.w8(self.WIDTH, self.KB), x[0],
                 ops=[(hb.EP_ADDP, self.vec(self.WIDTH, 0.1))])
        self.add(self.ACT, self.KB, hid, self.w8(self.ACT, self.KB), self.f32(self.ACT),
                 ops=[(hb.EP_ADDP, self.vec(self.ACT, 0.1))])
        torch.cuda.synchronize()


class PrefixStep(Chain):
    """The SmolVLA language-model prefix as the GEMM chain the reference
    compiler emits for it (tools/compiler/smolvla_lm.cpp:86-100, 118-255): 16
    decoder layers of hidden 960 (K 960), 15 query / 5 KV heads of 64,
    SiLU-gated MLP of 2560, every linear MXFP4, over the prefix's 141 tokens
    per batch element (rows padded to whole quads).  Per layer: q, k, v
    requantized to MXINT8 (RoPE is outside this path); o with the residual
    add; up; gate with ACT_MUL(up) and requantize; down with the residual
    add.  RMSNorm and attention are outside this chain: their outputs are
    synthetic MXINT8 tensors of the right shape."""

    HIDDEN, KB, KV, INTER, KBI, LAYERS, TOKENS = 960, 30, 320, 2560, 80, 16, 141

    def __init__(self, hb, torch, batch, mode, panels=False):
        super().__init__(hb, torch, self.TOKENS * batch, mode, 23 + batch, panels=panels)
        tb = self.table("silu")
        x = [self.f32(self.HIDDEN) for _ in range(3)]
        for _ in range(self.LAYERS):
            a1, ao, a2 = self.a_words(self.KB), self.a_words(self.KB), self.a_words(self.KB)
            for n in (self.HIDDEN, self.KV, self.KV):
                self.add(n, self.KB, a1, [self.w_words(n, self.KB)], self.f32(n),
                         q=self.a_words(n // 32))
            self.group(3)
            self.add(self.HIDDEN, self.KB, ao, [self.w_words(self.HIDDEN, self.KB)], x[1],
                     ops=[(hb.EP_ADD, x[0])])
            up = self.f32(self.INTER)
            self.add(self.INTER, self.KB, a2, [self.w_words(self.INTER, self.KB)], up)
            h = self.a_words(self.KBI)
            self.add(self.INTER, self.KB, a2, [self.w_words(self.INTER, self.KB)],
                     self.f32(self.INTER), ops=[(hb.EP_ACT_MUL, up)], q=h, tbuf=tb)
            self.group(2)
            self.add(self.HIDDEN, self.KBI, h, [self.w_words(self.HIDDEN, self.KBI)], x[2],
                     ops=[(hb.EP_ADD, x[1])])
        torch.cuda.synchronize()


class ExpertAttention:
    """The attention of one SmolVLA action-expert step as the reference
    compiler emits it (tools/compiler/kernels.cpp:78-244, plan from
    smolvla_expert.cpp:361-390): 16 layers, 15 query / 5 KV heads of 64, a
    chunk of 50 query rows per batch element, keys = 128 on the cross-
    attention (odd) layers and 128 + 64 on the self-attention (even) layers.
    Per layer: SPLIT8 of K and T32_SPLIT8 of V over every KV head and batch
    element at once; per query head, scores = Q_h K_j^T (W8, with the mask
    add on self layers and the 1/8 scale fused); the SOFTMAX program with
    MXINT8 requantize over every head's scores at once (valid keys: all on
    self layers, the 77-token prefix on cross layers); per query head
    O_h = P_h V_j (W8).  The query head's words are read out of the
    projection output in place (a_stride 30).  Each (element, head) block
    of scores has 52 rows (13 quads; rows 50 and 51 stay zero), so its
    probabilities are whole MXINT8 words, the A of its PV layer."""

    LAYERS, HEADS, KV, HW, QW, KVW, ROWS, PREFIX, SUFFIX = 16, 15, 5, 2, 30, 10, 50, 128, 64
    VALID_PREFIX = 77  # smolvla_parts_test.cpp:36: one camera, Prefix() 77 of Tokens() 128
    STREAMS = 4  # the head groups are independent: side streams, one context each

    def __init__(self, hb, torch, batch, mode, seed=41):
        dev, self.hb, self.torch, self.batch = "cuda:0", hb, torch, batch
        g = torch.Generator(device=dev).manual_seed(seed)
        quads = (self.ROWS + 3) // 4
        self.keep, self.steps, self.ops = [], [], 0.0

        def words(n, lo=122, hi=128):
            t = torch.randint(0, 256, (n, 144), generator=g, device=dev, dtype=torch.uint8)
            t[:, 128:132] = torch.randint(lo, hi, (n, 4), generator=g, device=dev, dtype=torch.uint8)
            t[:, 132:] = 0
            self.keep.append(t)
            return t

        max_keys = self.PREFIX + self.SUFFIX
        kbk_max = max_keys // 32
        # intermediates reused by every layer: planes, scores, P, O
        kh = torch.empty((2, batch * max_keys // 8 * self.KVW, 144), dtype=torch.uint8, device=dev)
        vh = torch.empty((2, 4 * self.KVW * batch * kbk_max, 144), dtype=torch.uint8, device=dev)
        blocks = batch * self.HEADS
        s = torch.zeros((blocks * quads * 4 * max_keys,), dtype=torch.float32, device=dev)
        p_words = torch.zeros((blocks * quads * kbk_max, 144), dtype=torch.uint8, device=dev)
        o = torch.empty((batch, self.HEADS, self.ROWS, 64), dtype=torch.float32, device=dev)
        tb = torch.from_numpy(activation_table("silu").view(np.int64)).to(dev)
        mask = torch.zeros((self.ROWS, max_keys), dtype=torch.float32, device=dev)
        mask[:, self.PREFIX:] = -1e4 * torch.triu(torch.ones(self.ROWS, self.SUFFIX, device=dev), 1)
        self.keep += [kh, vh, s, p_words, o, mask, tb]
        scale = int(np.array(0.125, np.float32).view(np.uint32))
        for layer in range(self.LAYERS):
            keys = self.PREFIX + (self.SUFFIX if layer % 2 == 0 else 0)
            rows, kbk = batch * keys // 4, keys // 32
            q = words(batch * quads * self.QW).view(batch, quads * self.QW, 144)
            k, v = words(rows * self.KVW), words(rows * self.KVW)
            self.steps.append(("split8", k, rows, kh))
            self.steps.append(("t32", v, rows, vh))
            ops = ([(hb.EP_ADD, mask)] if keys == max_keys else []) + [(hb.EP_SCALE, scale)]
            share, kb_all = self.HEADS // self.KV, batch * kbk
            s_at, p_at = quads * 4 * keys, quads * kbk  # block (b, h) = b * 15 + h

            def qk(b, h):  # scores: W = K_j planes of element b, 10 words per group row
                j = h // share
                return hb.linear_desc(
                    self.ROWS, keys, self.KVW, q[b, 2 * h:],
                    [kh[pl, (b * keys // 8) * self.KVW + 2 * j:] for pl in range(2)], [1, 2],
                    s[(b * self.HEADS + h) * s_at:], pieces=[(0, 2, 0)], a_stride=self.QW,
                    ops=ops, mode=mode)

            def pv(b, h):  # O_h = P_h V_j: V^T planes of head j, element b's blocks per group row
                j = h // share
                return hb.linear_desc(
                    self.ROWS, 64, kb_all, p_words[(b * self.HEADS + h) * p_at:],
                    [vh[pl, 8 * j * kb_all + b * kbk:] for pl in range(2)], [1, 2], o[b, h],
                    pieces=[(0, kbk, 0)], a_stride=kbk, mode=mode)

            # one launch per (query head) over the batch elements, or, for one
            # element, per position within the KV group over the KV heads
            # (every operand then advances by one uniform stride)
            groups = ([[(0, share * j + r) for j in range(self.KV)] for r in range(share)]
                      if batch == 1 else
                      [[(b, h) for b in range(batch)] for h in range(self.HEADS)])
            # the head groups' QK^T on side streams in turn, one softmax over
            # every block's scores, then the groups' PV
            valid = keys if keys == max_keys else self.VALID_PREFIX
            for fn in (qk, None, pv):
                if fn is None:
                    self.steps.append(("softmax", s, blocks * quads * 4, keys, valid, tb, p_words))
                    continue
                self.steps.append(("fork",))
                for i, grp in enumerate(groups):
                    self.steps.append(("linear", [fn(b, h) for b, h in grp], i % self.STREAMS))
                self.steps.append(("join",))
            self.ops += batch * self.HEADS * 2.0 * self.ROWS * 64 * keys * 2
        self.side = [torch.cuda.Stream() for _ in range(self.STREAMS)]
        self.side_ctx = [hb.Context(0) for _ in range(self.STREAMS)]
        for c, st in zip(self.side_ctx, self.side):
            c.set_stream(st.cuda_stream)
        torch.cuda.synchronize()
        self.m, self.descs = batch * self.ROWS, [d for st in self.steps if st[0] == "linear" for d in st[1]]

    def run(self, ctx):
        hb, main = self.hb, self.torch.cuda.current_stream()
        for st in self.steps:
            if st[0] == "split8":
                hb.split8(st[1], st[2], self.KVW, st[3][0], st[3][1], ctx=ctx, sync=False)
            elif st[0] == "t32":
                hb.t32_split8(st[1], st[2], self.KVW, st[3][0], st[3][1], ctx=ctx, sync=False)
            elif st[0] == "softmax":
                hb.rows(hb.ROWS_SOFTMAX, st[1], st[2], st[3], st[4], tbuf=st[5], q_out=st[6],
                        ctx=ctx, sync=False)
            elif st[0] == "fork":
                for side in self.side:
                    side.wait_stream(main)
            elif st[0] == "join":
                for side in self.side:
                    main.wait_stream(side)
            else:
                hb.linear_batched(st[1], self.side_ctx[st[2]])

    def close(self):
        for c in self.side_ctx:
            c.close()


def time_row_programs(hb, torch, ctx, stream, steps=10):
    """The VEC row programs over device rows with MXINT8 output (hb_rows) at
    model shapes; algorithmic bytes = fp32 rows read + MXINT8 words written
    + the fp32 row vectors."""
    dev, out = "cuda:0", {}
    tb = torch.from_numpy(activation_table("silu").view(np.int64)).to(dev)
    eps = int(np.array(1e-6, np.float32).view(np.uint32))
    for name, entry, rows, cols, aux in (
            ("rmsnorm_q SmolVLA LM B=32 (4512 x 960)", hb.ROWS_RMSNORM, 32 * 141, 960, 960),
            ("layernorm_q SigLIP (2048 x 768)", hb.ROWS_LAYERNORM, 2048, 768, 768),
            ("softmax_q expert attention B=32 (24960 x 192)", hb.ROWS_SOFTMAX, 32 * 15 * 52, 192, 192)):
        x = torch.randn((rows, cols), device=dev)
        g = torch.rand(cols, device=dev) + 0.5
        b = torch.randn(cols, device=dev) * 0.1
        q = torch.empty(((rows + 3) // 4 * cols // 32, 144), dtype=torch.uint8, device=dev)

        def call():
            hb.rows(entry, x, rows, cols, aux, eps, g, b, tb, q_out=q, ctx=ctx, sync=False)
        for _ in range(2):
            call()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            call()
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        vectors = {hb.ROWS_RMSNORM: 1, hb.ROWS_LAYERNORM: 2}.get(entry, 0)
        nbytes = 4.0 * rows * cols + q.numel() + 4.0 * cols * vectors
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
        del x, g, b, q
    return out


def time_row_format(hb, torch, ctx, stream, tokens=262144, tok=30, steps=10):
    """hb_row_load / hb_row_store of `tokens` MXINT8 tokens of tok blocks (the
    SmolVLA width 960: 976 bytes each, past the last-level cache);
    algorithmic bytes = the tokens read + the A words written (or the
    reverse)."""
    dev = "cuda:0"
    size = hb.row_token_bytes(tok)
    src = torch.randint(0, 256, (tokens * size,), dtype=torch.uint8, device=dev)
    words = torch.empty((tokens // 4 * tok, 144), dtype=torch.uint8, device=dev)
    nbytes = float(tokens * size + words.numel())
    out = {"workload": f"{tokens} tokens of {tok} blocks ({tokens * size / 1e6:.0f} MB of tokens, "
                       f"{words.numel() / 1e6:.0f} MB of A words)"}
    for name, call in (
            ("load", lambda: hb.row_load(src, tokens, 1, tok, words, ctx=ctx, sync=False)),
            ("store", lambda: hb.row_store(words, tokens, 1, tok, src, ctx=ctx, sync=False))):
        for _ in range(2):
            call()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            call()
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    del src, words
    return out


def time_gacc(hb, torch, ctx, stream, frames=(1, 16), slots=52, blocks=8, cameras=6,
              feature_rows=100000, steps=5):
    """GACC at the SparseDrive-S head's deformable aggregation shape: 900
    anchors (225 quads) per frame, 256 channels (8 blocks), per camera a list
    of 52 slots (13 points x 4 levels, 4 bilinear corners per token), the 6
    cameras chained through the accumulators; random rows of a 100,000-row
    feature pool, 10% null entries.  Reported per frame batch: ms for the 6
    chained commands and the gathered rows per second."""
    dev, out = "cuda:0", {}
    row_bytes = hb.row_token_bytes(blocks)
    rng = np.random.default_rng(5)
    for f in frames:
        quads = 225 * f
        w_words = (slots + 7) // 8
        w_bytes, list_bytes = blocks * w_words * 128, 16 + 128 * slots
        w_base = feature_rows * row_bytes
        list_base = w_base + quads * w_bytes
        size = list_base + cameras * quads * list_bytes
        img = torch.randint(0, 256, (size,), dtype=torch.uint8, device=dev)
        img[w_base:list_base] = torch.randint(0x39000000 // 256, 0x3C000000 // 256,
                                              ((list_base - w_base) // 4,), device=dev,
                                              dtype=torch.int32).mul(256).view(torch.uint8)
        hdr = np.zeros((cameras * quads, 16), np.uint8)
        hdr[:, :4] = ((w_base + (np.arange(cameras * quads) % quads) * w_bytes) // 16
                      ).astype(np.uint32).view(np.uint8).reshape(-1, 4)
        rows = rng.integers(0, feature_rows, (cameras * quads, slots * 16))
        entries = (rows * row_bytes // 16).astype(np.uint64)
        entries[rng.random(entries.shape) < 0.1] = 0xFFFFFFFF
        bw = np.full(entries.shape, 0x3E800000, np.uint64)
        lists = np.concatenate([hdr, (entries | (bw << np.uint64(32))).view(np.uint8)], axis=1)
        img[list_base:] = torch.from_numpy(lists.reshape(-1)).to(dev)
        acc = torch.zeros((quads * 4, 32 * blocks), dtype=torch.float32, device=dev)

        def run():
            for c in range(cameras):
                hb.gacc(img, img[list_base + c * quads * list_bytes:], quads, slots, blocks,
                        w_words * 8, acc, list_stride=list_bytes, accumulate=c > 0, ctx=ctx,
                        sync=False)
        run()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            run()
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        gathered = float((entries != 0xFFFFFFFF).sum())
        out[f"frames={f}"] = {"quads": quads, "ms": round(ms, 4),
                              "rows_per_s": round(gathered / (ms * 1e-3), 0),
                              "gathered_bytes_per_s": round(gathered * row_bytes / (ms * 1e-3), 0)}
        del img, acc
    return out


def time_split_kernels(hb, torch, ctx, stream, rows=200000, row_words=10, steps=10):
    """HBM rate of SPLIT8 and T32_SPLIT8 over a K / V matrix of rows x
    row_words MXINT8 words (rows * row_words * 144 B, larger than the
    last-level cache): algorithmic bytes = the source read once plus both
    planes written once = 2 x the source size."""
    dev = "cuda:0"
    src = torch.randint(0, 256, (rows * row_words, 144), dtype=torch.uint8, device=dev)
    src[:, 128:132] = torch.randint(118, 136, (rows * row_words, 4), dtype=torch.uint8, device=dev)
    hi = torch.empty((rows * row_words // 2, 144), dtype=torch.uint8, device=dev)
    lo = torch.empty_like(hi)
    nbytes = 2.0 * rows * row_words * 144
    out = {"workload": f"{rows} rows x {row_words} MXINT8 words ({rows * row_words * 144 / 1e6:.0f} MB "
                       "source), bytes = source + both planes"}
    for name, fn in (("split8", hb.split8), ("t32_split8", hb.t32_split8)):
        for _ in range(2):
            fn(src, rows, row_words, hi, lo, ctx=ctx, sync=False)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(steps):
            fn(src, rows, row_words, hi, lo, ctx=ctx, sync=False)
        t1.record(stream)
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / steps
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 4), "roofline": {"bound": "hbm", "achieved": round(gbs, 1),
                                                      "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    del src, hi, lo
    return out


class SiglipSet(Chain):
    """SigLIP-style vision-encoder GEMM set, W8: per layer, on M = 2 cameras x
    1024 patch tokens = 2048 rows with hidden 768, QKV 768->2304, out-proj
    768->768, MLP up 768->3072 with GELU and MXINT8 requantize, MLP down
    3072->768; per-channel scale (MULP) and bias (ADDP) on every GEMM; 12
    layers of distinct random weights."""

    M, D, QKV, FF, LAYERS = 2048, 768, 2304, 3072, 12

    def __init__(self, hb, torch, mode, w8_panels=False):
        super().__init__(hb, torch, self.M, mode, 21, w8_panels)
        tb = self.table("gelu")
        kb, kbf = self.D // 32, self.FF // 32

        def ep(n):
            return [(hb.EP_MULP, self.vec(n, 0.005, 0.0105)), (hb.EP_ADDP, self.vec(n, 0.1))]

        for _ in range(self.LAYERS):
            x = self.a_words(kb)
            self.add(self.QKV, kb, x, self.w8(self.QKV, kb), self.f32(self.QKV), ops=ep(self.QKV))
            self.add(self.D, kb, self.a_words(kb), self.w8(self.D, kb), self.f32(self.D),
                     ops=ep(self.D))
            h = self.a_words(kbf)
            self.add(self.FF, kb, self.a_words(kb), self.w8(self.FF, kb), self.f32(self.FF),
                     ops=ep(self.FF) + [(hb.EP_ACT, None)], q=h, tbuf=tb)
            self.add(self.D, kbf, h, self.w8(self.D, kbf), self.f32(self.D), ops=ep(self.D))
        torch.cuda.synchronize()


class SparseDriveHead(Chain):
    """SparseDrive-S detection head GEMMs (tools/compiler/sparsedrive_head.cpp:
    HeadOrder 62-76, the attention projections 800-886, OutProjection
    889-990, Ffn 1535-1620), on 928 anchor rows (900 padded) per frame.
    Six decoder blocks: the first an FFN only, the other five a temporal
    and a self attention and an FFN.  Attention, per block: q (512 -> 512,
    W8, bias, requantize) over the anchors, k and v over the keys (the
    anchors, or 608 temporal rows), the out projection (512 -> 512, W8,
    bias, the residual add, requantize) and fc_after (512 -> 256, W8).
    FFN: fc1 (512 -> 1024, MXFP4, bias, ReLU, requantize), fc2 (1024 ->
    256, MXFP4) and the identity projection (512 -> 256, MXFP4) onto fc2's
    output, then bias.  The deformable aggregation's and refinement's small
    GEMMs, the norms and the attention itself are outside this chain (their
    outputs are synthetic MXINT8 tensors of the right shape)."""

    ROWS, TEMP, D, DQ, FF, BLOCKS = 928, 608, 256, 512, 1024, 6

    def __init__(self, hb, torch, frames, mode, panels=False):
        super().__init__(hb, torch, self.ROWS * frames, mode, 51 + frames, panels=panels)
        kd, kq, kf = self.D // 32, self.DQ // 32, self.FF // 32
        rows = self.m
        for blk in range(self.BLOCKS):
            for temporal in ((True, False) if blk else ()):
                x = self.a_words(kq)
                for part in range(3):  # q over the anchors, k and v over the keys
                    keys = self.TEMP * frames if (temporal and part) else rows
                    sub = Chain(hb, torch, keys, mode, 61 + part, panels=panels)
                    sub.keep, sub.descs, sub.plan = self.keep, self.descs, self.plan
                    sub.add(self.DQ, kq, sub.a_words(kq) if keys != rows else x,
                            sub.w8(self.DQ, kq), sub.f32(self.DQ),
                            ops=[(hb.EP_ADDP, sub.vec(self.DQ, 0.1))], q=sub.a_words(kq))
                    self.ops += sub.ops
                    self.bytes += sub.bytes
                o = self.a_words(kq)
                self.add(self.DQ, kq, self.a_words(kq), self.w8(self.DQ, kq), self.f32(self.DQ),
                         ops=[(hb.EP_ADDP, self.vec(self.DQ, 0.1)),
                              (hb.EP_ADD, self.f32(self.DQ))], q=o)
                self.add(self.D, kq, o, self.w8(self.D, kq), self.f32(self.D))
            a = self.a_words(kq)
            h = self.a_words(kf)
            self.add(self.FF, kq, a, [self.w_words(self.FF, kq)], self.f32(self.FF),
                     ops=[(hb.EP_ADDP, self.vec(self.FF, 0.1)), (hb.EP_RELU, None)], q=h)
            out = self.f32(self.D)
            self.add(self.D, kf, h, [self.w_words(self.D, kf)], out)
            self.add(self.D, kq, a, [self.w_words(self.D, kq)], out, onto=True,
                     ops=[(hb.EP_ADDP, self.vec(self.D, 0.1))])
        torch.cuda.synchronize()


class SparseDriveConv(Chain):
    """SparseDrive-S backbone stage-1 3x3 convolution as its im2col GEMM:
    6 cameras x 64 x 176 output positions = 67,584 rows, K = 3*3*64 = 576,
    N = 64, MXFP4 weights (E8M0 exponents -10..-2), fp32 output."""

    M, K, N = 6 * 64 * 176, 576, 64

    def __init__(self, hb, torch, mode, panels=False):
        super().__init__(hb, torch, self.M, mode, 31, panels=panels)
        kb = self.K // 32
        self.add(self.N, kb, self.a_words(kb), [self.w_words(self.N, kb)], self.f32(self.N))
        torch.cuda.synchronize()


class SparseDriveBackbone(Chain):
    """SparseDrive-S image backbone (ResNet-50) as the GEMM chain the
    reference compiler emits for it (tools/compiler/sparsedrive_encoder.cpp:
    stem 571-640, bottlenecks 817-874, EmitConv 187-475), over 6 cameras at
    256 x 704 input per frame:

      stem: 7x7 stride-2 conv as a W8 GEMM, 128 x 352 positions per camera,
            K = 192, N = 64, + bias + ReLU, fp32 out (the max-pool reads it);
      4 stages of {3, 4, 6, 3} bottleneck blocks, mid width {64, 128, 256,
      512}, output 4 x mid, positions {64 x 176, 32 x 88, 16 x 44, 8 x 22}
      per camera; per block:
        conv1  1x1, K = cin (block 0) or 4 x mid, N = mid, + bias, ReLU,
               MXINT8 out only (over the input positions in block 0);
        conv2  3x3 im2col, K = 9 x mid, N = mid, stride 2 in block 0 of
               stages 2-4, + bias, ReLU, MXINT8 out only;
        conv3  1x1, K = mid, N = 4 x mid, + bias, ReLU, fp32 and MXINT8
               out; block 0 also folds the downsample 1x1 (strided) over
               the block's input as a second K range (bias = the two
               biases' sum), later blocks start from the residual (the
               previous block's fp32 output, updated in place).

    MXFP4 weights (E8M0 exponents -10..-2) and the W8 stem; 1x1 convs read
    the previous layer's MXINT8 words, 3x3 convs and the concatenated
    downsample operand read synthetic im2col words of their shape (the
    gather is the DMA engine's, not a GEMM).  conv1 and conv2 keep only
    their MXINT8 words (C = NULL), as the compiler stores only those."""

    CAMS, STEM_H, STEM_W = 6, 128, 352
    STAGES = ((3, 64, 1), (4, 128, 2), (6, 256, 2), (3, 512, 2))

    def __init__(self, hb, torch, frames, mode, panels=True):
        rows0 = frames * self.CAMS * self.STEM_H * self.STEM_W
        super().__init__(hb, torch, rows0, mode, 71 + frames, panels=panels)
        self.frames = frames
        relu = (hb.EP_RELU, None)

        def rows(r):
            self.m, self.quads = r, (r + 3) // 4

        def bias(n):
            return (hb.EP_ADDP, self.vec(n, 0.1))

        # stem (W8), fp32 out
        self.add(64, 6, self.a_words(6), self.w8(64, 6), self.f32(64), ops=[bias(64), relu])
        r = frames * self.CAMS * (self.STEM_H // 2) * (self.STEM_W // 2)
        rows(r)
        x8 = self.a_words(2)  # the max-pool's MXINT8 output, 64 channels
        cin = 64
        plan = []
        rin = r
        for blocks, mid, stride in self.STAGES:
            rout = rin // (stride * stride)
            plan.append((blocks, mid, stride, rin, rout))
            rin = rout
        for blocks, mid, stride, rin, rout in plan:
            cout = 4 * mid
            y32 = None
            for j in range(blocks):
                r1 = rin if j == 0 else rout
                k1 = cin if j == 0 else cout
                # conv1 over the block's input positions
                rows(r1)
                t1 = self.a_words(mid // 32)
                self.add(mid, k1 // 32, x8, [self.w_words(mid, k1 // 32)], None,
                         ops=[bias(mid), relu], q=t1, c_out=False)
                # conv2: 3x3 im2col at the output positions
                rows(rout)
                t2 = self.a_words(mid // 32)
                kb2 = 9 * mid // 32
                self.add(mid, kb2, self.a_words(kb2), [self.w_words(mid, kb2)], None,
                         ops=[bias(mid), relu], q=t2, c_out=False)
                # conv3 (+ downsample in block 0, + residual after)
                y8 = self.a_words(cout // 32)
                if j == 0:
                    kb3 = (mid + cin) // 32
                    y32 = self.f32(cout)
                    self.add(cout, kb3, self.a_words(kb3), [self.w_words(cout, kb3)], y32,
                             ops=[bias(cout), relu], q=y8)
                else:
                    self.add(cout, mid // 32, t2, [self.w_words(cout, mid // 32)], y32,
                             ops=[bias(cout), relu], q=y8, onto=True)
                x8 = y8
            cin = cout
        self.m = rows0
        torch.cuda.synchronize()


def time_chain(torch, ctx, work, steps=10, graph=True):
    """Milliseconds per pass over the chain: eager launches on one stream,
    and (graph=True) the same chain replayed as one captured HIP graph."""
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    for _ in range(2):
        work.run(ctx)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        work.run(ctx)
    t1.record(stream)
    torch.cuda.synchronize()
    eager = t0.elapsed_time(t1) / steps
    out = {"m": work.m, "gemms": len(work.descs), "gops": round(work.ops / 1e9, 3),
           "eager_ms": round(eager, 4)}
    if getattr(work, "grouped", False) and len(work.plan) < len(work.descs):
        out["launch_calls"] = len(work.plan)
        work.grouped = False  # the same chain, one call per layer, for comparison
        for _ in range(2):
            work.run(ctx)
        t0.record(stream)
        for _ in range(steps):
            work.run(ctx)
        t1.record(stream)
        torch.cuda.synchronize()
        out["ungrouped_eager_ms"] = round(t0.elapsed_time(t1) / steps, 4)
        work.grouped = True
    if graph:
        try:
            side = torch.cuda.Stream()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                ctx.set_stream(side.cuda_stream)
                work.run(ctx)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=side):
                ctx.set_stream(torch.cuda.current_stream().cuda_stream)
                work.run(ctx)
            ctx.set_stream(stream.cuda_stream)
            g.replay()
            torch.cuda.synchronize()
            t0.record(stream)
            for _ in range(steps):
                g.replay()
            t1.record(stream)
            torch.cuda.synchronize()
            out["graph_ms"] = round(t0.elapsed_time(t1) / steps, 4)
        except Exception as e:  # capture is optional for the measurement
            ctx.set_stream(stream.cuda_stream)
            out["graph_error"] = str(e)[:200]
    return out


def time_expert_step(hb, torch, ctx, batch, mode, steps=10):
    """Milliseconds per SmolVLA action-expert step (eager and graph), with
    its roofline over the best of the two."""
    work = ExpertStep(hb, torch, batch, mode, panels=mode == hb.FAST)
    out = {"batch": batch, "weights": "panels" if mode == hb.FAST else "DDR words",
           **time_chain(torch, ctx, work, steps)}
    best = min(out["eager_ms"], out.get("graph_ms", out["eager_ms"]))
    out["tops"], out["roofline"] = chain_summary(
        work, best, "fp6_fp4", f"expert_b{batch}" if mode == hb.FAST else None)
    del work
    return out


def chain_summary(work, ms, mfma_class, line=None):
    """TOPS and roofline of one pass over a chain taking `ms` (traffic: the
    counted HBM bytes per pass of bench line `line`)."""
    tops = work.ops / (ms * 1e-3) / 1e12
    gbs = work.bytes / (ms * 1e-3) / 1e9
    peak = MFMA_PEAK[mfma_class]
    if work.ops / work.bytes * HBM_PEAK_GBS / 1e3 < peak:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 1), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tops / peak, 4), "mfma_class": mfma_class}
    roof["traffic"] = counted_traffic(line) if line else None
    return round(tops, 3), roof


def settle(fn, torch, seconds):
    """Run fn back to back for about `seconds` (untimed), so the GPU's clocks
    reach the state they keep under sustained load of this kind before a
    timed region starts (they ramp over a few hundred milliseconds)."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_steps(hb, torch, ctx, stream, work, steps, warmup, settle_s=0.0):
    """Average ms per step over `steps` back-to-back batched launches, timed
    with events on the stream the kernels run on (after `settle_s` seconds of
    untimed steps and `warmup` more)."""
    if settle_s > 0:
        settle(lambda: hb.linear_batched(work.descs, ctx), torch, settle_s)
    for _ in range(warmup):
        hb.linear_batched(work.descs, ctx)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        hb.linear_batched(work.descs, ctx)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def summarize(work, ms, mfma_class, line=None):
    ops, nbytes = work.ops(), work.bytes()
    tops = ops / (ms * 1e-3) / 1e12
    gbs = nbytes / (ms * 1e-3) / 1e9
    peak = MFMA_PEAK[mfma_class]
    hbm_bound = ops / nbytes * HBM_PEAK_GBS / 1e3 < peak
    if hbm_bound:
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4)}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 1), "peak": peak, "unit": "TFLOP/s",
                "frac": round(tops / peak, 4)}
    roof["traffic"] = counted_traffic(line) if line else None
    return tops, roof


def single_layer_latency(hb, torch, ctx, stream, m, n, kb, launches=50, a_fp8=False):
    """Milliseconds per launch of one MXFP4 layer (fast mode, weights in
    panels), launched back to back on one stream: its one-launch latency,
    as a chain of dependent layers sees it (a launch starts when the one
    before it has ended)."""
    work = Workload(hb, torch, ctx, m, n, kb, False, 1, hb.FAST, seed=9, panels=True, a_fp8=a_fp8)
    d = work.descs[0]
    settle(lambda: hb.launch(d, ctx), torch, 0.05)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(launches):
        hb.launch(d, ctx)
    t1.record(stream)
    torch.cuda.synchronize()
    return round(t0.elapsed_time(t1) / launches, 4)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


TOLERANCE = ("fast mode: per element |got - exact| <= 2^-17 * sum over blocks of |block value| "
             "(measured envelope; the normwise per-row max |got - exact| <= 1e-5 * max |exact| "
             "holds on N(0,1) data); exact mode: bitwise")


# Bench lines that --line runs alone (the counter and trace runs of
# --profile-lines): name -> (description, builder).  A builder returns an
# object with run(ctx), ops() / bytes() per pass.
class BatchedLine:
    def __init__(self, hb, work):
        self.hb, self.work = hb, work

    def run(self, ctx):
        self.hb.linear_batched(self.work.descs, ctx)

    def ops(self):
        return self.work.ops()

    def bytes(self):
        return self.work.bytes()


class ChainLine:
    def __init__(self, work):
        self.work = work

    def run(self, ctx):
        self.work.run(ctx)

    def ops(self):
        return self.work.ops

    def bytes(self):
        return self.work.bytes


def bench_lines(hb, torch, ctx):
    n, kb = 960, 80
    F, E = hb.FAST, hb.EXACT

    def wl(*a, **k):
        return lambda: BatchedLine(hb, Workload(hb, torch, ctx, *a, **k))

    return {
        "headline_fast": ("MXFP4 M=128 K=2560 N=960 x256 layers, fast, weights in panels",
                          wl(128, n, kb, False, 256, F, panels=True)),
        "headline_exact": ("MXFP4 M=128 K=2560 N=960 x256 layers, exact, DDR words",
                           wl(128, n, kb, False, 256, E)),
        "sweep_m1": ("MXFP4 M=1 K=2560 N=960 x256 layers, fast, weights in panels",
                     wl(1, n, kb, False, 256, F, seed=3, panels=True)),
        "sweep_m16": ("MXFP4 M=16 K=2560 N=960 x256 layers, fast, weights in panels",
                      wl(16, n, kb, False, 256, F, seed=3, panels=True)),
        "sweep_m1024": ("MXFP4 M=1024 K=2560 N=960 x64 layers, fast, weights in panels",
                        wl(1024, n, kb, False, 64, F, seed=3, panels=True)),
        "fp8_m1": ("MXFP8 x MXFP4 M=1 K=2560 N=960 x256 layers, fast, weights in panels",
                   wl(1, n, kb, False, 256, F, seed=5, panels=True, a_fp8=True)),
        "fp8_m16": ("MXFP8 x MXFP4 M=16 K=2560 N=960 x256 layers, fast, weights in panels",
                    wl(16, n, kb, False, 256, F, seed=5, panels=True, a_fp8=True)),
        "fp8_m128": ("MXFP8 x MXFP4 M=128 K=2560 N=960 x256 layers, fast, weights in panels",
                     wl(128, n, kb, False, 256, F, seed=5, panels=True, a_fp8=True)),
        "fp8_m1024": ("MXFP8 x MXFP4 M=1024 K=2560 N=960 x64 layers, fast, weights in panels",
                      wl(1024, n, kb, False, 64, F, seed=5, panels=True, a_fp8=True)),
        "w8_fast": ("W8 M=64 K=960 N=2560 + MULP + ADDP x128 layers, fast, planes in panels",
                    wl(64, 2560, 30, True, 128, F, epilogue=True, seed=4, panels=True)),
        "w8_exact": ("W8 M=64 K=960 N=2560 + MULP + ADDP x128 layers, exact",
                     wl(64, 2560, 30, True, 128, E, epilogue=True, seed=4)),
        "siglip_fast": ("SigLIP-style W8 set, 12 layers x 4 GEMMs, M=2048, fast, W8 panels",
                        lambda: ChainLine(SiglipSet(hb, torch, F, w8_panels=True))),
        "siglip_exact": ("SigLIP-style W8 set, 12 layers x 4 GEMMs, M=2048, exact, DDR words",
                         lambda: ChainLine(SiglipSet(hb, torch, E))),
        "sparsedrive_fast": ("SparseDrive-S stage-1 im2col M=67584 K=576 N=64, MXFP4, fast",
                             lambda: ChainLine(SparseDriveConv(hb, torch, F, panels=True))),
        "sparsedrive_exact": ("SparseDrive-S stage-1 im2col M=67584 K=576 N=64, MXFP4, exact",
                              lambda: ChainLine(SparseDriveConv(hb, torch, E))),
        "sparsedrive_head_f1": ("SparseDrive-S det head GEMMs, 6 blocks, 928 anchor rows (1 "
                                "frame), W8 attention + MXFP4 FFN, fast",
                                lambda: ChainLine(SparseDriveHead(hb, torch, 1, F, panels=True))),
        "sparsedrive_head_f16": ("SparseDrive-S det head GEMMs, 6 blocks, 16 frames (14848 "
                                 "anchor rows), W8 attention + MXFP4 FFN, fast",
                                 lambda: ChainLine(SparseDriveHead(hb, torch, 16, F, panels=True))),
        "backbone_f1": ("SparseDrive-S ResNet-50 backbone GEMM chain (stem + 16 bottlenecks, "
                        "49 GEMMs), 6 cameras, 1 frame, fast, weights in panels",
                        lambda: ChainLine(SparseDriveBackbone(hb, torch, 1, F))),
        "backbone_f16": ("SparseDrive-S ResNet-50 backbone GEMM chain (stem + 16 bottlenecks, "
                         "49 GEMMs), 6 cameras, 16 frames, fast, weights in panels",
                         lambda: ChainLine(SparseDriveBackbone(hb, torch, 16, F))),
        "expert_b1": ("SmolVLA action-expert step GEMM chain, B=1 (M=50), fast, grouped",
                      lambda: ChainLine(ExpertStep(hb, torch, 1, F, panels=True))),
        "expert_b32": ("SmolVLA action-expert step GEMM chain, B=32 (M=1600), fast, grouped",
                       lambda: ChainLine(ExpertStep(hb, torch, 32, F, panels=True))),
        "prefix_b1": ("SmolVLA LM prefix GEMM chain, B=1 (M=141), fast, grouped",
                      lambda: ChainLine(PrefixStep(hb, torch, 1, F, panels=True))),
        "prefix_b32": ("SmolVLA LM prefix GEMM chain, B=32 (M=4512), fast, grouped",
                       lambda: ChainLine(PrefixStep(hb, torch, 32, F, panels=True))),
    }


def run_line(args):
    """--line NAME: build that line's workload, copy --copy-probe MiB (the
    counters' calibration, and the marker after which the line's own
    dispatches start), run --steps passes, print one JSON line."""
    import torch
    import hotarubi_amd as hb
    ctx = hb.Context(0)
    ctx.set_stream(torch.cuda.current_stream().cuda_stream)
    desc, make = bench_lines(hb, torch, ctx)[args.line]
    work = make()
    torch.cuda.synchronize()
    x = torch.ones(max(args.copy_probe, 1) << 20, dtype=torch.uint8, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    del x, y
    for _ in range(args.steps):
        work.run(ctx)
    torch.cuda.synchronize()
    print(json.dumps({"line": args.line, "workload": desc, "passes": args.steps,
                      "ops_per_pass": work.ops(), "bytes_per_pass": work.bytes()}), flush=True)
    ctx.close()


SQ_COUNTERS = ["GRBM_GUI_ACTIVE", "SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_WAVE_CYCLES",
               "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_LDS",
               "SQ_WAIT_INST_ANY"]


def profile_lines(args):
    """--profile-lines A,B,...: for each line, four rocprofv3 runs of
    `bench.py --line` as child processes (kernel trace, FETCH_SIZE,
    WRITE_SIZE, SQ counters), each its own pass; writes one summary per line
    and the traffic rows into --profile-out."""
    import csv
    import shutil
    import subprocess
    out_dir = os.path.abspath(args.profile_out)
    os.makedirs(out_dir, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    me = os.path.abspath(__file__)
    rows = []
    for line in args.profile_lines.split(","):
        res = {}
        for kind, prof in (("trace", ["--kernel-trace", "--stats"]),
                           ("fetch", ["--pmc", "FETCH_SIZE"]), ("write", ["--pmc", "WRITE_SIZE"]),
                           ("sq", ["--pmc"] + SQ_COUNTERS)):
            d = os.path.join(out_dir, "raw", f"{line}_{kind}")
            cmd = ["timeout", "-s", "KILL", "150", "rocprofv3", *prof, "--output-format", "csv",
                   "-d", d, "-o", "run", "--", sys.executable, me, "--line", line,
                   "--steps", str(args.steps), "--copy-probe", "256"]
            print(f"profile {line} {kind}", flush=True)
            r = subprocess.run(cmd, cwd="/tmp", env=env, capture_output=True, text=True)
            info = [json.loads(t) for t in r.stdout.splitlines() if t.startswith('{"line"')]
            if r.returncode != 0 or not info:
                print(r.stdout[-2000:], r.stderr[-2000:], file=sys.stderr)
                sys.exit(f"rocprofv3 run failed: {line} {kind} (exit {r.returncode})")
            res["info"] = info[-1]
            name = "run_kernel_trace.csv" if kind == "trace" else "run_counter_collection.csv"
            recs = list(csv.DictReader(open(os.path.join(d, name))))
            res[kind] = recs
        rows.append(summarize_profile(line, res, out_dir))
        shutil.rmtree(os.path.join(out_dir, "raw"), ignore_errors=True)  # the CSVs are large
    with open(os.path.join(out_dir, "traffic_rows.md"), "w") as f:
        for r in rows:
            f.write(r + "\n")


def _dispatches_after_probe(recs, key="Dispatch_Id"):
    """The records of the dispatches after the last device copy of the
    probe (the line's passes), grouped by dispatch, in order."""
    by = {}
    for r in recs:
        by.setdefault(int(r[key]), []).append(r)
    ids = sorted(by)
    probe = [i for i in ids if "copyBuffer" in by[i][0]["Kernel_Name"]]
    last = probe[-1] if probe else -1
    return [by[i] for i in ids if i > last], [by[i] for i in probe[-3:]]


def summarize_profile(line, res, out_dir):
    info = res["info"]
    passes = info["passes"]
    # trace: per kernel, time over the passes
    recs, _ = _dispatches_after_probe(res["trace"])
    per = {}
    for grp in recs:
        r = grp[0]
        k = r["Kernel_Name"].replace("hb::(anonymous namespace)::", "").replace("void ", "")
        k = re.sub(r"\(.*", "", k)
        t = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        e = per.setdefault(k, [0, 0.0])
        e[0] += 1
        e[1] += t
    total_us = sum(v[1] for v in per.values())
    span = [(int(g[0]["Start_Timestamp"]), int(g[0]["End_Timestamp"])) for g in recs]
    wall_us = (max(b for _, b in span) - min(a for a, _ in span)) / 1000.0 if span else 0.0
    top = sorted(per.items(), key=lambda kv: -kv[1][1])

    def counter_sum(kind, name):
        recs_k, probe = _dispatches_after_probe(res[kind])
        tot = sum(float(r["Counter_Value"]) for g in recs_k for r in g if r["Counter_Name"] == name)
        pr = [sum(float(r["Counter_Value"]) for r in g if r["Counter_Name"] == name) for g in probe]
        return tot / passes, (sum(pr) / len(pr) if pr else 0.0)

    fetch, fetch_probe = counter_sum("fetch", "FETCH_SIZE")
    write, write_probe = counter_sum("write", "WRITE_SIZE")
    copy_kib = 256 * 1024
    f_read = copy_kib / fetch_probe if fetch_probe else float("nan")
    f_write = copy_kib / write_probe if write_probe else float("nan")
    read_b, write_b = fetch * 1024 * f_read, write * 1024 * f_write
    traffic = int(round(read_b + write_b))
    alg = info["bytes_per_pass"]
    sq = {c: counter_sum("sq", c)[0] for c in SQ_COUNTERS}
    cycles = sq["GRBM_GUI_ACTIVE"] / 8.0  # per XCD, summed over the 8
    simds = 1024.0
    # The clock over the line's kernel time; under the counter profiler a
    # short dispatch's GRBM window also covers the profiler's own work, so
    # lines of many short dispatches fall back to the 2.4 GHz peak clock.
    ghz = cycles / (total_us / passes) / 1e3 if total_us else 0.0
    clock_note = f"{ghz:.2f} GHz from GRBM_GUI_ACTIVE"
    if not 1.0 <= ghz <= 2.6:
        ghz, clock_note = 2.4, "2.4 GHz peak clock (GRBM_GUI_ACTIVE spans the profiler's gaps)"
    kernel_cycles = total_us / passes * ghz * 1e3
    waves = max(sq["SQ_WAVES"], 1.0)
    lines = [
        f"# {top[0][0] if top else '?'} — {info['workload']}",
        "",
        "Commands (each a child process of the first; run from `/tmp`, `TMPDIR=/tmp`):",
        "",
        f"    python3 bench.py --profile-lines {line} --profile-out <dir> --steps {passes}",
        f"    rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- \\",
        f"        python3 bench.py --line {line} --steps {passes} --copy-probe 256",
        f"    rocprofv3 --pmc FETCH_SIZE ... (same program), then --pmc WRITE_SIZE, then",
        f"    rocprofv3 --pmc {' '.join(SQ_COUNTERS)} ...",
        "",
        f"Per pass ({passes} passes after the 256 MiB copy probe): "
        f"{len(recs) // max(passes, 1)} dispatches, "
        f"{total_us / passes:.1f} us of kernel time, {wall_us / passes:.1f} us first start to "
        f"last end.",
        "",
        "| kernel | dispatches | total us | avg us | share |",
        "|---|---|---|---|---|",
    ]
    for k, (c, t) in top[:8]:
        lines.append(f"| `{k}` | {c} | {t:.1f} | {t / c:.2f} | {t / total_us:.1%} |")
    lines += [
        "",
        f"HBM traffic per pass (calibration: the probe's 256 MiB copy reads FETCH_SIZE "
        f"{fetch_probe:.1f} KiB, writes WRITE_SIZE {write_probe:.1f} KiB; factors "
        f"{f_read:.5f} / {f_write:.5f}): read {read_b / 1e6:.2f} MB, written "
        f"{write_b / 1e6:.2f} MB, total {traffic / 1e6:.2f} MB against {alg / 1e6:.2f} MB "
        f"algorithmic (x{traffic / alg:.3f}).",
        "",
        f"SQ counters per pass (summed over the chip; `GRBM_GUI_ACTIVE` per XCD, summed over "
        f"8: {cycles:.0f} cycles):",
        "",
        f"- waves {sq['SQ_WAVES']:.0f}; VALU instructions per wave "
        f"{sq['SQ_INSTS_VALU'] / waves:.0f}; MFMA instructions per wave "
        f"{sq['SQ_INSTS_MFMA'] / waves:.0f}; LDS instructions per wave "
        f"{sq['SQ_INSTS_LDS'] / waves:.0f}",
        f"- matrix cores busy {sq['SQ_VALU_MFMA_BUSY_CYCLES'] / simds / max(kernel_cycles, 1):.1%}"
        f" of the kernel time per SIMD ({sq['SQ_VALU_MFMA_BUSY_CYCLES'] / simds:.0f} of "
        f"{kernel_cycles:.0f} cycles at {clock_note})",
        f"- a wave lives {sq['SQ_WAVE_CYCLES'] / waves:.0f} cycles on average, waiting on "
        f"instruction issue dependencies (`SQ_WAIT_INST_ANY`) "
        f"{sq['SQ_WAIT_INST_ANY'] / max(sq['SQ_WAVE_CYCLES'], 1):.1%} of them",
    ]
    kname = re.sub(r"<.*", "", top[0][0]).lower() if top else "kernels"
    with open(os.path.join(out_dir, f"{kname}_{line}.md"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return (f"| {line} | {top[0][0] if top else '?'} | {passes} | {fetch:.1f} | {write:.1f} | "
            f"{int(read_b)} | {int(write_b)} | {traffic} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["exact", "fast"], default="fast")
    ap.add_argument("--layers", type=int, default=256)
    ap.add_argument("--m", type=int, default=128)
    ap.add_argument("--quick", action="store_true", help="headline only, no extra fields")
    ap.add_argument("--only", choices=["attention", "smolvla"], default=None,
                    help="headline plus this group of extra fields only")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB")
    ap.add_argument("--settle", type=float, default=0.5, metavar="S",
                    help="seconds of untimed headline steps before the warmup (0: none)")
    ap.add_argument("--line", default=None, help="run one bench line's workload alone")
    ap.add_argument("--profile-lines", default=None, metavar="A,B,...",
                    help="rocprofv3 trace and counter runs of these lines (child processes)")
    ap.add_argument("--profile-out", default="gpurun_out/lines")
    args = ap.parse_args()
    if args.profile_lines:
        profile_lines(args)
        return
    if args.line:
        run_line(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); nothing in this build "
              "spans several GPUs.", file=sys.stderr)
        sys.exit(2)

    import torch
    import hotarubi_amd as hb

    if args.copy_probe:
        x = torch.ones(args.copy_probe << 20, dtype=torch.uint8, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        del x, y

    ctx = hb.Context(0)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    fast = args.mode == "fast"
    mode = hb.FAST if fast else hb.EXACT
    n, kb = 960, 80

    # weights packed into panels once, before timing (fast mode reads them;
    # the exact kernel reads DDR words)
    work = Workload(hb, torch, ctx, args.m, n, kb, False, args.layers, mode, panels=fast)
    ms = time_steps(hb, torch, ctx, stream, work, args.steps, args.warmup, settle_s=args.settle)
    std = args.m == 128 and args.layers == 256  # the shape the counter runs cover
    tops, roof = summarize(work, ms, "fp6_fp4" if fast else "bf16",
                           ("headline_fast" if fast else "headline_exact") if std else None)
    del work

    out = {
        "metric": METRIC,
        "value": round(tops, 3),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxint8 x mxfp4 -> fp32",
        "data": "synthetic, seeded, drawn on the device: each layer's activations MXINT8 of "
                "its own N(0,1) fp32 matrix (max-abs rule), random E2M1 weight codes, E8M0 "
                "exponents uniform in -10..-2",
        "config": {"workload": f"MXFP4 linear M={args.m} K={kb * 32} N={n}, "
                               f"{args.layers} distinct layers per step",
                   "mode": args.mode, "layers_per_step": args.layers, "m": args.m,
                   "k": kb * 32, "n": n,
                   "weights": "panels (hb_pack_weights, once, untimed)" if fast else "DDR words",
                   "settle_s": args.settle},
        "tolerance": TOLERANCE,
        "roofline": roof,
    }

    if not args.quick and args.only is None:
        extra_steps, extra_warm = 5, 1
        # the same workload in the other mode
        other = hb.EXACT if fast else hb.FAST
        w2 = Workload(hb, torch, ctx, args.m, n, kb, False, args.layers, other,
                      panels=other == hb.FAST)
        ms2 = time_steps(hb, torch, ctx, stream, w2, extra_steps, extra_warm, settle_s=0.2)
        t2, r2 = summarize(w2, ms2, "bf16" if fast else "fp6_fp4",
                           ("headline_exact" if fast else "headline_fast") if std else None)
        out["exact" if fast else "fast"] = {"value": round(t2, 3), "unit": "TOPS",
                                            "ms_per_step": round(ms2, 4), "roofline": r2}
        del w2
        # M sweep (fast MXFP4), enough layers per step to exceed the caches
        sweep = {}
        # (weights in panels, packed once, untimed, as for the headline)
        for m, L, pan in ((1, 256, True), (16, 256, True), (1024, 64, True)):
            ws = Workload(hb, torch, ctx, m, n, kb, False, L, hb.FAST, seed=3, panels=pan)
            mss = time_steps(hb, torch, ctx, stream, ws, extra_steps, extra_warm, settle_s=0.2)
            ts, rs = summarize(ws, mss, "fp6_fp4", f"sweep_m{m}")
            sweep[f"M={m}"] = {"value": round(ts, 3), "unit": "TOPS", "layers": L,
                               "weights": "panels" if pan else "DDR words",
                               "ms_per_step": round(mss, 4), "roofline": rs}
            del ws
        sweep["M=128"] = {"value": out["value"], "unit": "TOPS", "layers": args.layers,
                          "ms_per_step": out["ms_per_step"], "roofline": roof}
        out["mxfp4_fast_m_sweep"] = sweep
        # one layer of the same shape, one launch at a time
        out["mxfp4_fast_single_layer_ms"] = {
            "workload": f"one MXFP4 layer K={kb * 32} N={n} per launch, launches back to back "
                        "on one stream, weights in panels",
            **{f"M={m}": single_layer_latency(hb, torch, ctx, stream, m, n, kb)
               for m in (1, 16, 128, 1024)}}
        # config 1 with MXFP8 E4M3 activations (OCP MX encoding; no reference
        # counterpart): one layer per launch on the FP8 x FP4 matrix cores
        fp8 = {"workload": f"one MXFP4 layer K={kb * 32} N={n} per launch, activations MXFP8 "
                           "E4M3 (hb_encode_mxfp8), weights in panels, fast mode"}
        for m in (1, 16, 128, 1024):
            ms_l = single_layer_latency(hb, torch, ctx, stream, m, n, kb, a_fp8=True)
            nbytes = layer_bytes(m, n, kb, 4)
            fp8[f"M={m}"] = {"ms": ms_l, "tops": round(2.0 * m * n * kb * 32 / (ms_l * 1e-3) / 1e12, 3),
                             "hbm_frac": round(nbytes / (ms_l * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        out["mxfp8_single_layer"] = fp8
        # config 1's sweep with MXFP8 activations, batched as the MXINT8 sweep
        sweep8 = {"workload": f"MXFP8 E4M3 x MXFP4 linear K={kb * 32} N={n}, activations "
                              "hb_encode_mxfp8 of N(0,1), weights in panels, fast mode (two "
                              "exponent planes per block on the FP8 x FP4 matrix cores)"}
        for m, L in ((1, 256), (16, 256), (128, 256), (1024, 64)):
            ws = Workload(hb, torch, ctx, m, n, kb, False, L, hb.FAST, seed=5, panels=True,
                          a_fp8=True)
            mss = time_steps(hb, torch, ctx, stream, ws, extra_steps, extra_warm, settle_s=0.2)
            ts, rs = summarize(ws, mss, "fp8", f"fp8_m{m}")
            sweep8[f"M={m}"] = {"value": round(ts, 3), "unit": "TOPS", "layers": L,
                                "ms_per_step": round(mss, 4), "roofline": rs}
            del ws
        out["mxfp8_fast_m_sweep"] = sweep8
        # W8 layer with per-channel scale and bias, fast and exact
        L8 = 128
        w8 = {"workload": f"W8 linear M=64 K=960 N=2560 + MULP + ADDP, {L8} layers per step; "
                          "fast: each weight plane in panels, exact: DDR words"}
        for name, md, cls in (("fast", hb.FAST, "int8"), ("exact", hb.EXACT, "bf16")):
            wk = Workload(hb, torch, ctx, 64, 2560, 30, True, L8, md, epilogue=True, seed=4,
                          panels=md == hb.FAST)
            ms8 = time_steps(hb, torch, ctx, stream, wk, extra_steps, extra_warm, settle_s=0.2)
            t8, r8 = summarize(wk, ms8, cls, f"w8_{name}")
            w8[name] = {"value": round(t8, 3), "unit": "TOPS", "ms_per_step": round(ms8, 4),
                        "roofline": r8}
            del wk
        out["w8"] = w8

        # SigLIP-style W8 encoder set (12 layers x 4 GEMMs, M=2048; fast mode
        # over W8 panels, the weights' layout for large-M W8 layers, exact
        # mode over DDR words) and the SparseDrive-S stage-1 3x3 im2col GEMM
        # (MXFP4), fast and exact
        for key, short, desc, cls_fast, make in (
                ("siglip_w8_set", "siglip", "W8 SigLIP-style encoder: 12 layers x {QKV 768->2304, out "
                 "768->768, up 768->3072 + GELU + requantize, down 3072->768}, M=2048, "
                 "MULP + ADDP; fast: W8 panels, exact: DDR words", "int8",
                 lambda md: SiglipSet(hb, torch, md, w8_panels=md == hb.FAST)),
                ("sparsedrive_stage1_conv_mxfp4", "sparsedrive", "MXFP4 im2col GEMM M=67584 K=576 N=64 "
                 "(SparseDrive-S stage-1 3x3 conv, 6 cameras)", "fp6_fp4",
                 lambda md: SparseDriveConv(hb, torch, md, panels=md == hb.FAST))):
            rec = {}
            for name, md, cls in (("fast", hb.FAST, cls_fast), ("exact", hb.EXACT, "bf16")):
                wk = make(md)
                t = time_chain(torch, ctx, wk, steps=5, graph=False)
                tops, roof = chain_summary(wk, t["eager_ms"], cls, f"{short}_{name}")
                rec[name] = {"value": tops, "unit": "TOPS", "ms_per_pass": t["eager_ms"],
                             "gemms": t["gemms"], "m": t["m"],
                             "weights": ("W8 panels" if key == "siglip_w8_set" else "panels")
                             if md == hb.FAST else "DDR words", "roofline": roof}
                del wk
            if key == "siglip_w8_set":  # the fast set over DDR words, for comparison
                wk = SiglipSet(hb, torch, hb.FAST)
                t = time_chain(torch, ctx, wk, steps=5, graph=False)
                tops, roof = chain_summary(wk, t["eager_ms"], cls_fast)
                rec["fast_ddr_words"] = {"value": tops, "unit": "TOPS", "ms_per_pass": t["eager_ms"],
                                         "roofline": roof}
                del wk
            rec["workload"] = desc
            out[key] = rec
        # SparseDrive-S detection head GEMMs at 1 frame (both modes) and 16
        head = {"workload": "SparseDrive-S det head GEMM chain: 6 blocks (5 with temporal "
                            "and self attention: q/k/v 512->512 W8 + bias + requantize, out "
                            "512->512 W8 + bias + residual + requantize, fc_after 512->256 W8; "
                            "6 FFNs: fc1 512->1024 MXFP4 + bias + ReLU + requantize, fc2 "
                            "1024->256, identity 512->256 onto + bias), 928 rows per frame"}
        for frames, modes in ((1, (("fast", hb.FAST, "fp6_fp4"), ("exact", hb.EXACT, "bf16"))),
                              (16, (("fast", hb.FAST, "fp6_fp4"),))):
            for name, md, cls in modes:
                wk = SparseDriveHead(hb, torch, frames, md, panels=md == hb.FAST)
                t = time_chain(torch, ctx, wk, steps=5, graph=False)
                tops, roof = chain_summary(wk, t["eager_ms"], cls,
                                           f"sparsedrive_head_f{frames}" if md == hb.FAST else None)
                head[f"frames={frames}"] = head.get(f"frames={frames}", {})
                head[f"frames={frames}"][name] = {"value": tops, "unit": "TOPS",
                                                  "ms_per_pass": t["eager_ms"],
                                                  "gemms": t["gemms"], "m": t["m"],
                                                  "weights": "panels" if md == hb.FAST
                                                  else "DDR words",
                                                  "roofline": roof}
                del wk
        out["sparsedrive_head"] = head
        # SparseDrive-S backbone: every bottleneck's GEMMs and the stem
        bb = {"workload": "SparseDrive-S ResNet-50 backbone GEMM chain over 6 cameras at "
                          "256x704: stem 7x7/2 (W8, K=192, N=64, bias + ReLU), 16 bottlenecks "
                          "(stages of 3/4/6/3, mid 64/128/256/512): conv1 1x1 and conv2 3x3 "
                          "im2col (MXFP4, bias + ReLU + requantize), conv3 1x1 (MXFP4, bias + "
                          "ReLU, fp32 + requantize; downsample folded as a second K range in "
                          "block 0, residual start after), 49 GEMMs per frame"}
        for frames, modes in ((1, (("fast", hb.FAST, "fp6_fp4"), ("exact", hb.EXACT, "bf16"))),
                              (16, (("fast", hb.FAST, "fp6_fp4"),))):
            for name, md, cls in modes:
                wk = SparseDriveBackbone(hb, torch, frames, md, panels=md == hb.FAST)
                t = time_chain(torch, ctx, wk, steps=5 if frames == 1 else 3, graph=False)
                tops, roof = chain_summary(wk, t["eager_ms"], cls,
                                           f"backbone_f{frames}" if md == hb.FAST else None)
                bb.setdefault(f"frames={frames}", {})[name] = {
                    "value": tops, "unit": "TOPS", "ms_per_pass": t["eager_ms"],
                    "gemms": t["gemms"], "rows_stage1": frames * 6 * 64 * 176,
                    "weights": "panels" if md == hb.FAST else "DDR words", "roofline": roof}
                del wk
        out["sparsedrive_backbone"] = bb
        ctx.set_stream(stream.cuda_stream)

    if not args.quick and args.only in (None, "smolvla"):
        # SmolVLA action-expert step (GEMM chain), B = 1 and 32
        out["smolvla_expert_step_ms"] = {f"B={b}": time_expert_step(hb, torch, ctx, b, mode)
                                         for b in (1, 32)}
        ctx.set_stream(stream.cuda_stream)
        # SmolVLA LM prefix (16 MXFP4 decoder layers' GEMMs over 141 tokens per element)
        prefix = {"workload": "SmolVLA LM prefix GEMM chain: 16 layers x {q 960, k 320, v 320 "
                              "(requantize), o 960 (+residual), up 2560, gate 2560 (ACT_MUL, "
                              "requantize), down 960 (+residual)}, MXFP4, 141 tokens per element"}
        for b in (1, 32):
            wk = PrefixStep(hb, torch, b, mode, panels=fast)
            t = time_chain(torch, ctx, wk, steps=5)
            best = min(t["eager_ms"], t.get("graph_ms", t["eager_ms"]))
            tops, roof = chain_summary(wk, best, "fp6_fp4", f"prefix_b{b}" if fast else None)
            prefix[f"B={b}"] = {**t, "weights": "panels" if fast else "DDR words", "tops": tops,
                                "roofline": roof}
            del wk
        ctx.set_stream(stream.cuda_stream)
        out["smolvla_prefix_ms"] = prefix

    if not args.quick and args.only in (None, "attention"):
        # attention operands built on device (SPLIT8 / T32_SPLIT8), the row
        # programs (norms, softmax) with requantize, and the expert step's
        # attention over them
        out["attention_operands"] = time_split_kernels(hb, torch, ctx, stream)
        out["row_programs"] = time_row_programs(hb, torch, ctx, stream)
        out["row_format"] = time_row_format(hb, torch, ctx, stream)
        out["gacc_sparsedrive"] = time_gacc(hb, torch, ctx, stream)
        att = {"workload": "SmolVLA expert attention: 16 layers x 15 heads, QK^T (mask, scale), "
                           "softmax + MXINT8, PV in W8 over SPLIT8 / T32_SPLIT8 operands, 50 rows "
                           "per element"}
        for b in (1, 32):
            wk = ExpertAttention(hb, torch, b, mode)
            t = time_chain(torch, ctx, wk, steps=5)
            best = min(t["eager_ms"], t.get("graph_ms", t["eager_ms"]))
            att[f"B={b}"] = {**t, "tops": round(wk.ops / (best * 1e-3) / 1e12, 3)}
            wk.close()
            del wk
        ctx.set_stream(stream.cuda_stream)
        out["smolvla_expert_attention_ms"] = att

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.m, n, kb)
        out["cpu_baseline_cores"] = cpu_baseline_cores(args.m, n, kb)
        out["cpu_baseline"]["cpu_model"] = out["cpu_baseline_cores"]["cpu_model"] = cpu_model()
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
