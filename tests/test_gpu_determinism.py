"""Repeat-call determinism of every kernel instantiation the SLAB entry points reach.

The MFMA kernels read their accumulators back on the VALU; a missed wait between a dependent
MFMA's write-back and such a read shows up as sums that change from run to run, not as a wrong
result every time. So each instantiation (weight type x vectors per pass x gate/up pair x one or
several slot groups per wave x fused norm, for the slab GEMV in its chunked and even splits, its
VALU form, the grouped GEMV, the exact small-M GEMM and the bf16 GEMM tile families) is run three times on the same inputs, with
other kernels in between, and every run must give the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import IQ4_XS, NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, SLAB_TYPES, isclose_bits, make_weights
from test_gpu_parity import dense_of, host, say, slab_of, to_dev

pytestmark = pytest.mark.gpu

VALU_TYPES = (Q4_0, Q8_0, Q4_K, Q6_K)  # the VALU slab GEMV's formats


def _matrix(hl, dev, t, rows, cols, seed):
    buf, stride = make_weights(t, rows, cols, seed=seed)
    return slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols)


def _x(n_vec, cols, seed):
    return np.random.default_rng(seed).standard_normal((n_vec, cols)).astype(np.float32)


def _three_runs(run, other):
    """run() three times with other() in between; every run's output bitwise the first's."""
    first = run()
    other()
    second = run()
    other()
    third = run()
    assert isclose_bits(second, first), "a second run gave different bits"
    assert isclose_bits(third, first), "a third run gave different bits"
    assert np.all(np.isfinite(first))


# (rows, cols): 9 slabs, one slot group per wave (ONE); 1025 slabs, two groups per wave
GEMV_SHAPES = [(576, 5120), (65600, 512)]


@pytest.mark.parametrize("t", SLAB_TYPES)
@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_slab_gemv_every_instantiation_repeats(hl, dev, t, rows, cols):
    """k_gemv_mx<T, NV, PAIR, ONE> for NV = 1..4 and both PAIR (the gate/up pair), the NORM
    instantiation at one vector, and the VALU form k_gemv_slab where the format has one."""
    import torch

    say("determinism slab gemv", NAMES[t], rows, cols)
    wg = _matrix(hl, dev, t, rows, cols, 3100 + t)
    wu = _matrix(hl, dev, t, rows, cols, 3150 + t)
    nw = to_dev(np.random.default_rng(3199).uniform(0.5, 1.5, cols).astype(np.float32), dev)
    scratch = torch.empty((4, rows), dtype=torch.float32, device=dev)

    def other():  # a different kernel on different data between the runs
        hl.gemv(t, wu, to_dev(_x(4, cols, 3198), dev), scratch, rows, cols, 4, variant=hl.Variant.SLAB_GEMV)

    for n_vec in (1, 2, 3, 4):
        xd = to_dev(_x(n_vec, cols, 3200 + n_vec), dev)
        y = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)

        def plain(v=hl.Variant.SLAB_GEMV, norm=None):
            def go():
                hl.gemv(t, wg, xd, y, rows, cols, n_vec, variant=v, norm_w=norm)
                return host(y).copy()
            return go

        def pair():
            hl.gate_up_swiglu(t, wg, wu, xd, y, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMV)
            return host(y).copy()

        _three_runs(plain(), other)
        _three_runs(pair, other)
        if n_vec == 1:
            _three_runs(plain(norm=nw), other)
        if t in VALU_TYPES:
            _three_runs(plain(v=hl.Variant.SLAB_GEMV_VALU), other)


@pytest.mark.parametrize("t", (Q4_K, Q4_0, IQ4_XS, Q5_K, Q8_0))
@pytest.mark.parametrize("rows,cols,pair", [(32768, 2048, False), (8192, 5120, True)])
def test_even_split_every_instantiation_repeats(hl, dev, t, rows, cols, pair):
    """k_gemv_mx_even<T, NV, PAIR, NORM> (512 workgroups with equal shares of a large launch's slot
    groups) for NV = 1..4, the gate/up pair, and the fused norm at one vector."""
    import torch

    say("determinism even split", NAMES[t], rows, cols, "pair" if pair else "")
    wg = _matrix(hl, dev, t, rows, cols, 3900 + t)
    wu = _matrix(hl, dev, t, rows, cols, 3950 + t) if pair else None
    nw = to_dev(np.random.default_rng(3999).uniform(0.5, 1.5, cols).astype(np.float32), dev)
    scratch = torch.empty((4, rows), dtype=torch.float32, device=dev)

    def other():
        hl.gemv(t, wg, to_dev(_x(4, cols, 3998), dev), scratch, rows, cols, 4, variant=hl.Variant.SLAB_GEMV)

    for n_vec in (1, 2, 3, 4):
        xd = to_dev(_x(n_vec, cols, 4000 + n_vec), dev)
        y = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)

        def go(norm=None):
            def run():
                if pair:
                    hl.gate_up_swiglu(t, wg, wu, xd, y, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMV, norm_w=norm)
                else:
                    hl.gemv(t, wg, xd, y, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMV, norm_w=norm)
                return host(y).copy()
            return run

        _three_runs(go(), other)
        if n_vec == 1:
            _three_runs(go(nw), other)


@pytest.mark.parametrize("ta,tb", [(Q4_K, Q6_K), (Q8_0, IQ4_XS), (Q5_K, Q4_0)])
@pytest.mark.parametrize("n_vec", [1, 4])
def test_grouped_gemv_repeats(hl, dev, ta, tb, n_vec):
    """k_gemv_mx_group<TA, TB, NV, NORM>: two weight types in one launch, with and without the
    fused norm (one vector)."""
    import torch

    cols = 5120
    say("determinism grouped gemv", NAMES[ta], NAMES[tb], n_vec)
    wa = _matrix(hl, dev, ta, 1024, cols, 3300 + ta)
    wb = _matrix(hl, dev, tb, 640, cols, 3350 + tb)
    ya = torch.empty((n_vec, 1024), dtype=torch.float32, device=dev)
    yb = torch.empty((n_vec, 640), dtype=torch.float32, device=dev)
    xd = to_dev(_x(n_vec, cols, 3400 + n_vec), dev)
    nw = to_dev(np.random.default_rng(3401).uniform(0.5, 1.5, cols).astype(np.float32), dev)
    scratch = torch.empty((n_vec, 1024), dtype=torch.float32, device=dev)

    def other():
        hl.gemv(ta, wa, to_dev(_x(n_vec, cols, 3402), dev), scratch, 1024, cols, n_vec, variant=hl.Variant.SLAB_GEMV)

    for norm in ((None, nw) if n_vec == 1 else (None,)):
        def go():
            hl.gemv_group([(ta, wa, 1024, ya), (tb, wb, 640, yb)], xd, cols, n_vec, norm_w=norm)
            return np.concatenate([host(ya).ravel(), host(yb).ravel()])

        _three_runs(go, other)


@pytest.mark.parametrize("t", SLAB_TYPES)
def test_exact_small_m_every_instantiation_repeats(hl, dev, t):
    """k_gemm_sx<T, PAIR, NP> for NP = 1..4 (1, 3, 5 and 8 vectors), plain and gate/up pair, and
    the passes of variant 9 past eight vectors."""
    import torch

    rows, cols = 1100, 5120
    say("determinism exact small-M", NAMES[t])
    wg = _matrix(hl, dev, t, rows, cols, 3500 + t)
    wu = _matrix(hl, dev, t, rows, cols, 3550 + t)
    scratch = torch.empty((8, rows), dtype=torch.float32, device=dev)

    def other():
        hl.gemv(t, wu, to_dev(_x(8, cols, 3598), dev), scratch, rows, cols, 8, variant=hl.Variant.SLAB_GEMM_EXACT_SMALL_M)

    for n_vec in (1, 3, 5, 8, 11):
        xd = to_dev(_x(n_vec, cols, 3600 + n_vec), dev)
        y = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)
        v = hl.Variant.SLAB_GEMM_EXACT_SMALL_M if n_vec <= 8 else hl.Variant.SLAB_GEMM_EXACT_INVARIANT

        def plain():
            hl.gemv(t, wg, xd, y, rows, cols, n_vec, variant=v)
            return host(y).copy()

        def pair():
            hl.gate_up_swiglu(t, wg, wu, xd, y, rows, cols, n_vec, variant=v)
            return host(y).copy()

        _three_runs(plain, other)
        _three_runs(pair, other)


@pytest.mark.parametrize("t", SLAB_TYPES)
@pytest.mark.parametrize("variant,n_vec", [(7, 16), (7, 32), (3, 40), (3, 100), (3, 200), (5, 600)])
def test_bf16_gemm_tile_families_repeat(hl, dev, t, variant, n_vec):
    """k_gemm_sm (16 and 32 rows kept), k_gemm_pc at its 64 / 128 / 256-row M tiles and k_gemm_lm,
    plain and gate/up pair, whole and split tiles (the 272-slab shape leaves a partial round)."""
    import torch

    rows, cols = 17408 if variant == 5 else 4352, 1024
    say("determinism bf16 gemm", NAMES[t], variant, n_vec)
    wg = _matrix(hl, dev, t, rows, cols, 3700 + t)
    wu = _matrix(hl, dev, t, rows, cols, 3750 + t)
    xd = to_dev(_x(n_vec, cols, 3800 + n_vec), dev)
    y = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)
    scratch = torch.empty((4, rows), dtype=torch.float32, device=dev)

    def other():
        hl.gemv(t, wu, to_dev(_x(4, cols, 3801), dev), scratch, rows, cols, 4, variant=hl.Variant.SLAB_GEMV)

    def plain():
        hl.gemv(t, wg, xd, y, rows, cols, n_vec, variant=variant)
        return host(y).copy()

    def pair():
        hl.gate_up_swiglu(t, wg, wu, xd, y, rows, cols, n_vec, variant=variant)
        return host(y).copy()

    _three_runs(plain, other)
    _three_runs(pair, other)
