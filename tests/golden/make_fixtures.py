"""Write the golden fixtures under tests/golden/ from the reference's own code.

Run in the container that has /root/reference (after `make -C oracle ref`):

    python tests/golden/make_fixtures.py

The reference's FP32 arithmetic is compiled from its sources where they lie
(tools/iss/fp32.hpp, tb/fp32_ref.cpp) into oracle/_ref/libref_fp32.so; this
script only calls that library and stores inputs with outputs:

  fp32_ref_vectors.npz  ISS Fp32Add / Fp32Mul / Fp32MulFraction and tb
                        Fp32FromInt (the tb BlockValue, tb/gemm_ref.cpp:34-45)
                        on seeded operands, including the edge encodings
  tb_gemm_expected.npz  the FBUF words tb::ReferenceGemm (tb/gemm_ref.cpp:47-68)
                        produces for the six tb/gemm_test.cpp cases, whose
                        inputs tb_cases.py regenerates exactly; the loop nest is
                        restated here, every add and block value comes from the
                        compiled reference code
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, HERE)

import oracle  # noqa: E402
import tb_cases  # noqa: E402


def fp32_operands(rng, n):
    sign = rng.integers(0, 2, n, dtype=np.uint32) << 31
    exp = rng.integers(0, 256, n, dtype=np.uint32) << 23
    frac = rng.integers(0, 1 << 23, n, dtype=np.uint32)
    kind = rng.integers(0, 8, n)
    frac = np.where(kind == 0, frac & 0x7F0000, np.where(kind == 1, frac | 0x7FFF00, frac))
    return (sign | exp | frac).astype(np.uint32)


def near(rng, a, spread):
    e = ((a >> 23) & 0xFF).astype(np.int64) + rng.integers(-spread, spread + 1, a.size)
    e = np.clip(e, 0, 255).astype(np.uint32)
    return ((rng.integers(0, 2, a.size, dtype=np.uint32) << 31) | (e << 23) |
            rng.integers(0, 1 << 23, a.size, dtype=np.uint32)).astype(np.uint32)


def fp32_vectors():
    rng = np.random.default_rng(20240601)
    n = 10000
    a = fp32_operands(rng, 3 * n)
    b = np.concatenate([fp32_operands(rng, n), near(rng, a[n:2 * n], 2),
                        (a[2 * n:] ^ 0x80000000) + rng.integers(-3, 4, n).astype(np.uint32)])
    add = oracle.ref_batched("ref_iss_fp32_add_n", a, b)
    ma = fp32_operands(rng, 2 * n)
    mb = np.concatenate([fp32_operands(rng, n), near(rng, (0xFE000000 - ma[n:]) & 0x7FFFFFFF, 3)])
    mul = oracle.ref_batched("ref_iss_fp32_mul_n", ma, mb)
    fs = fp32_operands(rng, n)
    ff = rng.integers(0, 1 << 16, n, dtype=np.uint32)
    mulfrac = oracle.ref_batched("ref_iss_fp32_mul_fraction_n", fs, ff)
    sums = rng.integers(-61440, 61441, n).astype(np.int64)
    sums[: n // 10] = 0
    expo = rng.integers(-290, 140, n).astype(np.int32)
    fromint = np.zeros(n, np.uint32)
    R = oracle.ref()
    import ctypes as C
    R.ref_tb_fp32_from_int_n(sums.ctypes.data_as(C.POINTER(C.c_int64)),
                             expo.ctypes.data_as(C.POINTER(C.c_int32)),
                             fromint.ctypes.data_as(C.POINTER(C.c_uint32)), n)
    np.savez_compressed(os.path.join(HERE, "fp32_ref_vectors.npz"), add_a=a, add_b=b, add=add,
                        mul_a=ma, mul_b=mb, mul=mul, mf_s=fs, mf_f=ff, mulfrac=mulfrac,
                        fi_sum=sums, fi_exp=expo, fromint=fromint)


def weight_values(nibbles, wmode):
    mag = np.array([0, 1, 2, 3, 4, 6, 8, 12], np.int64)
    n = nibbles.astype(np.int64)
    if wmode == 0:
        return np.where(n & 8, -mag[n & 7], mag[n & 7])
    if wmode == 1:
        return np.where(n & 8, n - 16, n)
    return n


def reference_gemm(args, abuf, wbuf, fbuf):
    """tb::ReferenceGemm loop nest; arithmetic by the compiled reference."""
    bias = {0: -7, 1: -8, 2: -12}[args["wmode"]]
    for q in range(args["m"] // 4):
        for g in range(args["n8"]):
            out = fbuf[args["c_base"] + q * args["n8"] + g]
            acc = out.copy() if args["acc"] else np.zeros(32, np.uint32)
            for b in range(args["kb"]):
                aw = abuf[args["a_base"] + q * args["a_stride"] + b]
                ww = wbuf[args["w_base"] + g * args["w_stride"] + b]
                qa = aw[:128].view(np.int8).astype(np.int64).reshape(4, 32)
                nib = np.empty(256, np.uint8)
                nib[0::2] = ww[:128] & 15
                nib[1::2] = ww[:128] >> 4
                wv = weight_values(nib, args["wmode"]).reshape(8, 32)
                sums = (qa[:, None, :] * wv[None, :, :]).sum(-1).reshape(32)  # t*8 + c
                ea = aw[128:132].astype(np.int64)
                ew = ww[128:136].astype(np.int64)
                expo = ((ea[:, None] - 127) + (ew[None, :] - 127) + bias).reshape(32)
                bv = np.array([oracle.ref().ref_tb_fp32_from_int(int(s), int(e))
                               for s, e in zip(sums, expo)], np.uint32)
                acc = np.array([oracle.ref().ref_tb_fp32_add(int(x), int(y))
                                for x, y in zip(acc, bv)], np.uint32)
            out[:] = acc


def tb_expected():
    arrays = {}
    for name, seed, passes in tb_cases.tb_cases():
        fbuf = tb_cases.initial_fbuf(seed, passes)
        for p in passes:
            reference_gemm(p["args"], p["abuf"], p["wbuf"], fbuf)
        arrays[name] = fbuf
    np.savez_compressed(os.path.join(HERE, "tb_gemm_expected.npz"), **arrays)


if __name__ == "__main__":
    if oracle.ref() is None:
        sys.exit("oracle/_ref/libref_fp32.so is not built (make -C oracle ref)")
    fp32_vectors()
    tb_expected()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
