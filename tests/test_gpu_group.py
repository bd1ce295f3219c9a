"""hb_linear_group_async on an MI355X: several small fast layers in one
launch give the results of launching them one by one (bit for bit where
every layer keeps the K split plan of its own launch; a grid that would
not fit the CUs in one round takes fewer splits), and a gated pair (gate's ACT_MUL
operand is up's C, tools/compiler/smolvla_expert.cpp:400-420 and
smolvla_lm.cpp:226-245 emit them in that order) folds both layers in one
workgroup, the gate reading up's values there.  Shapes: the SmolVLA
action expert's q/k/v (M = 50, K = 720, N = 960/320/320, requantized) and
up/gate (N = 2048), the prefix's up/gate (M = 141, K = 960, N = 2560), a W8
pair, a pair whose splits do not fit one workgroup side by side, a pair
whose layers are not adjacent in the list, and groups that fall back to
one launch per layer.  Against the oracle (tools/iss/gemm_array.cpp:112-149
with the epilogue of tools/iss/lane.cpp) at the fast-mode tolerance."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import helpers
import hotarubi_amd as hb
from test_gpu_bench_routes import DEV, dev, host, mxfp4_planes, say, w8_planes

pytestmark = pytest.mark.gpu


class Layer:
    """One layer's host data and device buffers; desc() builds its
    descriptor, x2 (a device [m][n] tensor) standing for ACT_MUL's operand."""

    def __init__(self, rng, m, n, kb, w8=False, quantize=False, act_mul=False, mode=hb.FAST,
                 a=None, a_d=None):
        self.m, self.n, self.kb, self.w8, self.mode = m, n, kb, w8, mode
        self.a = helpers.activations(rng, m, kb * 32)[1] if a is None else a
        self.a_d = dev(self.a) if a_d is None else a_d
        self.planes, self.modes = w8_planes(rng, n, kb) if w8 else mxfp4_planes(rng, n, kb)
        self.w_d = [dev(p) for p in self.planes]
        self.quantize, self.act_mul = quantize, act_mul
        self.tbuf = helpers.activation_table("silu") if act_mul else None
        self.tb_d = dev(self.tbuf.view(np.int64)) if act_mul else None
        self.out()

    def out(self):
        self.c = torch.zeros((self.m, self.n), dtype=torch.float32, device=DEV)
        self.q = torch.zeros(((self.m + 3) // 4 * (self.n // 32), 144), dtype=torch.uint8,
                             device=DEV) if self.quantize else None

    def desc(self, x2=None):
        ops = [(hb.EP_ACT_MUL, x2)] if self.act_mul else []
        return hb.linear_desc(self.m, self.n, self.kb, self.a_d, self.w_d, self.modes, self.c,
                              ops=ops, tbuf=self.tb_d, q_out=self.q, mode=self.mode)

    def result(self):
        return host(self.c).view(np.uint32).copy(), (host(self.q).copy() if self.quantize else None)

    def check_oracle(self, x2_bits=None):
        got, gq = self.result()
        ops = [(hb.EP_ACT_MUL, x2_bits)] if self.act_mul else []
        want, wq = helpers.oracle_linear_mt(self.m, self.n, self.kb, self.a, self.planes,
                                            self.modes, ops=ops, tbuf=self.tbuf,
                                            quantize=self.quantize)
        if self.mode == hb.EXACT:
            assert np.array_equal(got, want)
            if self.quantize:
                assert np.array_equal(gq, wq)
        else:
            helpers.check_fast(got, want, gq, wq)


def run_both(gpu, layers, x2_of):
    """Launch the layers one by one, keep the results, then as a group; returns
    (separate results, group results).  x2_of[i]: the index of the layer
    whose C is layer i's ACT_MUL operand."""
    def descs():
        return [ly.desc(layers[x2_of[i]].c if i in x2_of else None) for i, ly in enumerate(layers)]
    for d in descs():
        hb.launch(d, gpu)
    sep = [ly.result() for ly in layers]
    for ly in layers:
        ly.out()
    torch.cuda.synchronize()
    hb.linear_group(descs(), gpu)
    return sep, [ly.result() for ly in layers]


def same(sep, grp):
    for (c0, q0), (c1, q1) in zip(sep, grp):
        assert np.array_equal(c0, c1)
        if q0 is not None:
            assert np.array_equal(q0, q1)


def test_group_expert_qkv(gpu):
    rng = np.random.default_rng(501)
    q = Layer(rng, 50, 960, 23, quantize=True)
    k = Layer(rng, 50, 320, 23, quantize=True, a=q.a, a_d=q.a_d)
    v = Layer(rng, 50, 320, 23, quantize=True, a=q.a, a_d=q.a_d)
    say("group q/k/v", dict(m=50, kb=23))
    sep, grp = run_both(gpu, [q, k, v], {})
    same(sep, grp)
    k.check_oracle()


@pytest.mark.parametrize("m,n,kb,w8,bitwise", [
    (50, 2048, 23, False, True),    # expert: 128 tiles x (3 + 3) waves, the separate plans
    (141, 2560, 30, False, False),  # prefix: 400 tiles do not fit one round at 4 + 4 waves,
                                    # so each layer takes 2 splits (other bits, same tolerance)
    (50, 736, 23, True, True)])
def test_group_gated_pair(gpu, m, n, kb, w8, bitwise):
    rng = np.random.default_rng(510 + m + kb)
    up = Layer(rng, m, n, kb, w8=w8)
    gate = Layer(rng, m, n, kb, w8=w8, quantize=True, act_mul=True, a=up.a, a_d=up.a_d)
    say("group gated pair", dict(m=m, n=n, kb=kb, w8=w8))
    sep, grp = run_both(gpu, [up, gate], {1: 0})
    if bitwise:
        same(sep, grp)
    else:
        helpers.check_fast(grp[0][0], sep[0][0])
    up.check_oracle()
    gate.check_oracle(x2_bits=grp[0][0])


def test_group_pair_not_adjacent_with_singles(gpu):
    """[up, q, gate, k]: units (up, gate), q, k in one launch."""
    rng = np.random.default_rng(520)
    up = Layer(rng, 50, 2048, 23)
    q = Layer(rng, 50, 960, 23, quantize=True)
    gate = Layer(rng, 50, 2048, 23, quantize=True, act_mul=True, a=up.a, a_d=up.a_d)
    k = Layer(rng, 50, 320, 30, quantize=True)
    say("group pair + singles")
    sep, grp = run_both(gpu, [up, q, gate, k], {2: 0})
    same(sep, grp)
    gate.check_oracle(x2_bits=grp[0][0])
    k.check_oracle()


def test_group_pair_replanned_splits(gpu):
    """K = 2560 (80 blocks, 8 splits each alone): side by side the pair's
    layers take 4 splits each, so the bits may differ from separate
    launches; both meet the oracle at the fast-mode tolerance."""
    rng = np.random.default_rng(530)
    up = Layer(rng, 50, 960, 80)
    gate = Layer(rng, 50, 960, 80, quantize=True, act_mul=True, a=up.a, a_d=up.a_d)
    say("group replanned pair")
    sep, grp = run_both(gpu, [up, gate], {1: 0})
    helpers.check_fast(grp[0][0], sep[0][0])
    up.check_oracle()
    gate.check_oracle(x2_bits=grp[0][0])


@pytest.mark.parametrize("case", ["exact", "rows", "mixed_formats"])
def test_group_falls_back_in_order(gpu, case):
    """Groups one launch cannot hold run layer by layer, in order: an exact
    layer, a layer of more than 160 rows, MXFP4 beside W8.  The gate still
    reads up's C after up wrote it."""
    rng = np.random.default_rng(540)
    m = 200 if case == "rows" else 50
    up = Layer(rng, m, 1024, 12, mode=hb.EXACT if case == "exact" else hb.FAST)
    gate = Layer(rng, m, 1024, 12, quantize=True, act_mul=True, a=up.a, a_d=up.a_d,
                 w8=case == "mixed_formats")
    say("group fallback", dict(case=case))
    sep, grp = run_both(gpu, [up, gate], {1: 0})
    same(sep, grp)
    up.check_oracle()
    gate.check_oracle(x2_bits=grp[0][0])


@pytest.mark.parametrize("case", ["two_consumers", "chain"])
def test_group_unpaired_consumers_run_in_order(gpu, case):
    """ACT_MUL dependencies a pair cannot hold: one producer read by two gates
    (the second gate cannot be its pair too), and a chain up -> gate -> third
    (the third reads the C of a pair's second layer).  The group runs one
    launch per layer, in order, so every consumer reads its producer's
    finished C: the results equal the one-by-one launches bit for bit."""
    rng = np.random.default_rng(560)
    up = Layer(rng, 50, 1024, 12)
    gate = Layer(rng, 50, 1024, 12, act_mul=True, a=up.a, a_d=up.a_d)
    third = Layer(rng, 50, 1024, 12, quantize=True, act_mul=True, a=up.a, a_d=up.a_d)
    x2_of = {1: 0, 2: 0} if case == "two_consumers" else {1: 0, 2: 1}
    say("group unpaired consumers", dict(case=case))
    sep, grp = run_both(gpu, [up, gate, third], x2_of)
    same(sep, grp)
    up.check_oracle()
    gate.check_oracle(x2_bits=grp[0][0])
    third.check_oracle(x2_bits=grp[x2_of[2]][0])


def test_group_rejections(gpu):
    rng = np.random.default_rng(550)
    ly = Layer(rng, 8, 64, 2)
    for descs in ([], [ly.desc()] * 5):
        with pytest.raises(hb.HbError) as err:
            hb.linear_group(descs, gpu)
        assert err.value.code == hb.HB_EINVAL


def test_group_sparsedrive_head_qkv(gpu):
    """The SparseDrive-S head's temporal attention projections as one group
    (tools/compiler/sparsedrive_head.cpp:800-886): q over the 928 anchor
    rows, k and v over 608 temporal rows with their own A, each 512 -> 512
    W8 with both planes packed as weight panels, bias (ADDP) and the
    requantize.  Each layer of the group meets the oracle at the fast-mode
    tolerance, and so do the same layers launched one by one."""
    rng = np.random.default_rng(520)
    n, kb = 512, 16
    layers = []
    for m in (928, 608, 608):
        a = helpers.activations(rng, m, kb * 32)[1]
        planes, modes = w8_planes(rng, n, kb)
        bias = helpers.random_fp32_words(rng, (n,), 118, 126)
        pan, src = [], [dev(p) for p in planes]  # src stays alive until the packers ran
        for p in src:
            t = torch.empty((hb.panel_bytes(n, kb),), dtype=torch.uint8, device=DEV)
            hb.pack_weights(p, n, kb, t, ctx=gpu)
            pan.append(t)
        layers.append(dict(m=m, a=a, a_d=dev(a), planes=planes, modes=modes, bias=bias,
                           bias_d=dev(bias.view(np.float32)), pan=pan, src=src))
    gpu.synchronize()

    def outputs():
        return [(torch.zeros((ly["m"], n), dtype=torch.float32, device=DEV),
                 torch.zeros(((ly["m"] + 3) // 4 * (n // 32), 144), dtype=torch.uint8, device=DEV))
                for ly in layers]

    def descs(outs):
        return [hb.linear_desc(ly["m"], n, kb, ly["a_d"], ly["pan"], ly["modes"], c,
                               ops=[(hb.EP_ADDP, ly["bias_d"])], q_out=q, mode=hb.FAST,
                               panels=True)
                for ly, (c, q) in zip(layers, outs)]

    say("group head q/k/v", dict(m=(928, 608, 608), n=n, kb=kb))
    sep = outputs()
    for d in descs(sep):
        hb.launch(d, gpu)
    grp = outputs()
    hb.linear_group(descs(grp), gpu)
    torch.cuda.synchronize()
    for ly, (c1, q1), (c2, q2) in zip(layers, sep, grp):
        want, wq = helpers.oracle_linear_mt(ly["m"], n, kb, ly["a"], ly["planes"], ly["modes"],
                                            ops=[(hb.EP_ADDP, ly["bias"])], quantize=True)
        for c, q in ((c1, q1), (c2, q2)):
            helpers.check_fast(host(c).view(np.uint32).copy(), want, host(q).copy(), wq)
