"""The C-ABI library loads and exports every symbol include/hotarubi_gpu.h
declares; the host-side entry points (decode/encode/check/access/cycles)
agree with the oracle.  No compute call: these run without a GPU."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import helpers
import hotarubi_amd as hb
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "hotarubi_gpu.h")).read()
    return sorted(set(re.findall(
        r"^\s*(?:int|void\*?|uint32_t|uint64_t|const char\*)\s+(hb_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = hb.lib()
    syms = header_symbols()
    assert len(syms) >= 20
    assert set(syms) == set(hb.EXPORTS)
    for s in syms:
        assert hasattr(lib, s), s
    assert lib.hb_abi_version() == hb.ABI_VERSION == 3


def test_product_does_not_link_the_oracle():
    data = open(hb.LIB_PATH, "rb").read()
    assert b"hbo_" not in data and b"liboracle" not in data


def random_cmd(rng):
    return hb.GemmCommand(a_base=int(rng.integers(0, 1 << 20)), a_stride=int(rng.integers(0, 1024)),
                          kb=int(rng.integers(0, 1024)), m=int(rng.integers(0, 1024)),
                          w_base=int(rng.integers(0, 1 << 20)), w_stride=int(rng.integers(0, 1024)),
                          n8=int(rng.integers(0, 256)), c_base=int(rng.integers(0, 1 << 20)),
                          wmode=int(rng.integers(0, 4)), acc=bool(rng.integers(0, 2)))


def test_encode_decode_roundtrip_and_field_map():
    rng = np.random.default_rng(1)
    for _ in range(500):
        cmd = random_cmd(rng)
        word = hb.encode_gemm(cmd)
        v = int.from_bytes(word, "little")
        assert v >> 120 == 4
        assert (v >> 92) & 0xFFFFF == cmd.a_base and (v >> 82) & 0x3FF == cmd.a_stride
        assert (v >> 72) & 0x3FF == cmd.kb and (v >> 62) & 0x3FF == cmd.m
        assert (v >> 42) & 0xFFFFF == cmd.w_base and (v >> 32) & 0x3FF == cmd.w_stride
        assert (v >> 24) & 0xFF == cmd.n8 and (v >> 4) & 0xFFFFF == cmd.c_base
        assert (v >> 2) & 3 == cmd.wmode and (v >> 1) & 1 == int(cmd.acc)
        back = hb.decode_gemm(word)
        assert back == hb.GemmCommand(**{**cmd.__dict__, "acc": int(cmd.acc)})
    with pytest.raises(hb.HbError):
        hb.decode_gemm(bytes(16))


def test_check_messages_match_reference():
    for fields, text in [(dict(m=16, kb=1, a_stride=1, n8=1), "GEMM m = 16 is not a multiple of 32 from 32 to 992"),
                         (dict(m=32, kb=3, a_stride=2, n8=1), "GEMM kb = 3 is not in [1, a_stride = 2]"),
                         (dict(m=32, kb=1, a_stride=1, n8=0), "GEMM n8 = 0")]:
        with pytest.raises(hb.HbBadCommand) as err:
            hb.check_gemm(hb.GemmCommand(**fields))
        assert err.value.message == text
    hb.check_gemm(hb.GemmCommand(m=32, kb=1, a_stride=1, n8=1))
    hb.check_gemm(hb.GemmCommand(m=992, kb=1, a_stride=1, n8=255))


def test_n8_beyond_the_instruction_field_is_rejected():
    """n8 is an 8-bit field of the instruction word (isa.hpp:83); a command
    struct with more columns cannot come from a decoded word and is refused
    as a bad argument (the FBUF aliasing kernel keeps at most 16 writers per
    word, which 248 quads x 255 groups never exceed)."""
    with pytest.raises(hb.HbError) as err:
        hb.check_gemm(hb.GemmCommand(m=992, kb=1, a_stride=1, n8=265))
    assert err.value.code == hb.HB_EINVAL
    assert err.value.message == "GEMM n8 = 265 does not fit the instruction's 8-bit field"


def test_access_sets_and_cycles_match_oracle(olib):
    rng = np.random.default_rng(2)
    n = 0
    while n < 200:
        cmd = random_cmd(rng)
        cmd.m = int(rng.integers(1, 32)) * 32
        cmd.kb = int(rng.integers(1, 8))
        cmd.a_stride = cmd.kb + int(rng.integers(0, 4))
        cmd.n8 = int(rng.integers(1, 40))
        oc = helpers.gemm_cmd(**{k: int(v) for k, v in cmd.__dict__.items()})
        _, ra, rw, rf, wf = oracle.gemm_access(oc)
        ga, gw, gf, gwf = hb.gemm_access(cmd)
        assert np.array_equal(ra, ga) and np.array_equal(rw, gw)
        assert np.array_equal(rf, gf) and np.array_equal(wf, gwf)
        assert hb.gemm_cycles(cmd, 51) == olib.hbo_gemm_cycles(oc, 51)
        n += 1
