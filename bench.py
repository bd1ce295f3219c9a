"""Benchmark: quantized GEMM TOPS and roofline fraction on one MI355X.

Workload (the metric's configuration): an MXFP4 linear layer, weights
E2M1 [N=960][K=2560] with E8M0 block-32 scales (exponents -10..-2), MXINT8
activations [M=128][K=2560] from N(0,1), FP32 output.  One step = one pass
over a batch of L independent layers of that shape (distinct weights and
activations, L * 2.24 MB > the 256 MB last-level cache), launched as one
batched kernel; the inputs are resident in HBM before timing starts.

    python bench.py [--steps K] [--warmup W] [--mode exact|fast] [--layers L]

Prints one JSON line.  The CPU baseline times the oracle (a C restatement of
the reference's CPU path, single thread) on one layer of the same shape.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_PEAK_TOPS = {"int8": 5000.0, "fp8": 5000.0, "bf16": 2500.0, "fp4": 10100.0}


def layer_bytes(m, n, kb, w_bits=4):
    """Algorithmic bytes: A MXINT8 + W (4- or 8-bit + E8M0) + C fp32."""
    k = kb * 32
    a = m * k * (1 + 1 / 32)
    w = n * k * (w_bits / 8 + 1 / 32)
    c = 4 * m * n
    return a + w + c


def make_inputs(rng, m, n, kb):
    """Synthetic MXINT8 activations and MXFP4 weights in DDR word layout,
    generated directly (no oracle): A words [m/4][kb][144], W words [n/8][kb][144]."""
    quads = (m + 3) // 4
    a = np.zeros((quads, kb, 144), np.uint8)
    x = rng.standard_normal((quads * 4, kb, 32)).astype(np.float32)
    amax = np.abs(x).max(axis=2)
    e = np.floor(np.log2(np.maximum(amax, 1e-30))).astype(np.int32)
    q = np.clip(np.rint(x * np.exp2(6 - e)[..., None]), -128, 127).astype(np.int8)
    a[:, :, :128] = q.reshape(quads, 4, kb, 32).transpose(0, 2, 1, 3).reshape(quads, kb, 128).view(np.uint8)
    a[:, :, 128:132] = (e + 127).reshape(quads, 4, kb).transpose(0, 2, 1).astype(np.uint8)
    w = np.zeros((n // 8, kb, 144), np.uint8)
    w[:, :, :128] = rng.integers(0, 256, (n // 8, kb, 128), dtype=np.uint8)
    w[:, :, 128:136] = (127 + rng.integers(-10, -1, (n // 8, kb, 8))).astype(np.uint8)
    return a.reshape(-1, 144), w.reshape(-1, 144)


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
        oracle.linear(m, n, kb, a, [w], [0])
        times.append(time.perf_counter() - t0)
        if time.perf_counter() + times[-1] > t_end or len(times) >= 5:
            break
    t = float(np.median(times))
    return {"value": 2.0 * m * n * kb * 32 / t / 1e12, "unit": "TOPS", "cores": 1, "kind": "port",
            "sample": f"{len(times)} run(s) of one {m}x{kb * 32}x{n} MXFP4 layer, median {t:.3f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--mode", choices=["exact", "fast"], default="exact")
    ap.add_argument("--layers", type=int, default=256)
    ap.add_argument("--m", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); nothing in this build "
              "spans several GPUs.", file=sys.stderr)
        sys.exit(2)

    import torch
    import hotarubi_amd as hb

    m, n, kb, L = args.m, 960, 80, args.layers
    rng = np.random.default_rng(1)
    a1, w1 = make_inputs(rng, m, n, kb)
    dev = "cuda:0"
    # distinct layers: random weights/activations per layer, built on device
    a_all = torch.empty((L,) + a1.shape, dtype=torch.uint8, device=dev)
    w_all = torch.empty((L,) + w1.shape, dtype=torch.uint8, device=dev)
    for i in range(L):
        ai, wi = make_inputs(np.random.default_rng(100 + i), m, n, kb) if i < 4 else (a1, w1)
        a_all[i].copy_(torch.from_numpy(ai))
        w_all[i].copy_(torch.from_numpy(wi))
    if L > 4:  # decorrelate the rest cheaply on device: permute words, keep scales sane
        g = torch.Generator(device=dev).manual_seed(5)
        for i in range(4, L):
            w_all[i, :, :128] = torch.randint(0, 256, w_all[i, :, :128].shape, generator=g,
                                              device=dev, dtype=torch.uint8)
            a_all[i, :, :128] = torch.randint(0, 256, a_all[i, :, :128].shape, generator=g,
                                              device=dev, dtype=torch.uint8)
    c_all = torch.zeros((L, m, n), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    ctx = hb.Context(0)
    stream = torch.cuda.current_stream()
    ctx.set_stream(stream.cuda_stream)
    mode = hb.FAST if args.mode == "fast" else hb.EXACT
    descs = [hb.linear_desc(m, n, kb, a_all[i], [w_all[i]], [0], c_all[i], mode=mode) for i in range(L)]

    def step():
        hb.linear_batched(descs, ctx)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps

    ops = 2.0 * m * n * kb * 32 * L
    tops = ops / (ms * 1e-3) / 1e12
    bytes_step = layer_bytes(m, n, kb) * L
    gbs = bytes_step / (ms * 1e-3) / 1e9
    ai = ops / bytes_step
    peak_mfma = MFMA_PEAK_TOPS["int8"]
    bound = "hbm" if ai * HBM_PEAK_GBS / 1e3 < peak_mfma else "mfma"
    if bound == "hbm":
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None}
    else:
        roof = {"bound": "mfma", "achieved": round(tops, 1), "peak": peak_mfma, "unit": "TFLOP/s",
                "frac": round(tops / peak_mfma, 4), "traffic": None}

    out = {
        "metric": "quantized GEMM TOPS & % MFMA/HBM roofline (W8, MXFP4); SmolVLA step ms",
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
        "data": "synthetic (seeded MXINT8 activations, random E2M1 codes, E8M0 exponents -10..-2)",
        "config": {"workload": f"MXFP4 linear M={m} K={kb * 32} N={n}, {L} distinct layers per step",
                   "mode": args.mode, "layers_per_step": L, "m": m, "k": kb * 32, "n": n},
        "roofline": roof,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(m, n, kb)
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
