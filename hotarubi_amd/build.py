"""Build libhotarubi_gpu.so (gfx950 only) in-tree with hipcc.

    python -m hotarubi_amd.build            # compile
    python -m hotarubi_amd.build --asm      # also dump gfx950 assembly to _build/

Flags: -ffp-contract=off (no FMA contraction: the exact path depends on
separately rounded adds and multiplies), -fgpu-flush-denormals-to-zero (FP32
denormal inputs and results flush, the NPU's FTZ rule), and packed-FP32
instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libhotarubi_gpu.so")
SOURCES = ["hb_api.hip", "hb_gemm.hip", "hb_fast.hip", "hb_fast4.hip", "hb_skinny.hip", "hb_vec.hip",
           "hb_dma.hip", "hb_panel.hip", "hb_stream.hip", "hb_w8.hip", "hb_prep.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-fgpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
# Per-source flags.  hb_skinny.hip: the single-layer split kernel's leading
# arguments (pointers and sizes, 13 dwords) are preloaded into SGPRs by the
# hardware, so its first operand loads need no argument round trip.
SOURCE_FLAGS = {"hb_skinny.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=11"]}


def build(asm: bool = False, verbose: bool = False) -> str:
    """Compile each source to an object (in parallel), then link the library."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    objdir = os.path.join(ROOT, "_build", "obj")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in srcs]

    def compile_one(src_obj):
        src, obj = src_obj
        cmd = [HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(os.path.basename(src), []), "-fPIC", "-c",
               "-I", os.path.join(ROOT, "include"), "-o", obj, src]
        if verbose:
            print(" ".join(cmd))
        return subprocess.run(cmd, capture_output=True, text=True)

    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(compile_one, zip(srcs, objs)))
    for src, r in zip(srcs, results):
        if r.stderr and (verbose or r.returncode != 0):
            sys.stderr.write(r.stderr)
        if r.returncode != 0:
            raise subprocess.CalledProcessError(r.returncode, f"hipcc {os.path.basename(src)}")
    cmd = [HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", "-o", LIB + ".tmp", *objs]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(LIB + ".tmp", LIB)
    if asm:
        out = os.path.join(ROOT, "_build")
        os.makedirs(out, exist_ok=True)
        for s in srcs:
            name = os.path.splitext(os.path.basename(s))[0]
            subprocess.run([HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(os.path.basename(s), []),
                            "-I", os.path.join(ROOT, "include"),
                            "--cuda-device-only", "-S", "-o", os.path.join(out, name + ".s"), s],
                           check=True)
    return LIB


if __name__ == "__main__":
    build(asm="--asm" in sys.argv, verbose=True)
