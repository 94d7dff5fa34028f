"""The slab GEMV's even split (k_gemv_mx_even): 512 workgroups take equal shares of a large
launch's slot groups, in (slab, matrix, group) order, so that every CU streams the same bytes.

Each shape below drives one of its cases: slabs that lie wholly inside one workgroup (they meet
in LDS alone), slabs split over two or three workgroups (their pieces meet in the split-K words),
the gate/up pair (gate and up pieces of one slab, and whole pair slabs whose up half the gate
segment's wave takes), and the in-kernel RMS norm (one published word per workgroup). Acceptance
is the slab GEMV's: every output within the derived bound of cpu::matmul (the oracle), rows
bitwise independent of n_vec (GemvArgs::allow_gemm off, include/halo/backend/backend.h:298-302 of
the reference; the waves per workgroup change with n_vec, the sums must not), the fused norm
bitwise RMS_NORM then the unfused call, and repeated calls bitwise equal.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import IQ4_XS, NAMES, Q4_0, Q4_K, Q5_K, Q8_0, isclose_bits, max_ratio, slab_gemv_tol, swiglu_tol, synth_matrix
from test_gpu_parity import SENTINEL, host, say, slab_of, to_dev

pytestmark = pytest.mark.gpu

EPS = 1e-6
# the formats that take the even split (Q6_K runs chunked); Q5_K and Q8_0 with up to two units per wave
EVEN_TYPES = (Q4_K, Q4_0, IQ4_XS, Q5_K, Q8_0)
# (rows, cols, pair): 512 slabs x 8 groups = 4096 units, 8 per workgroup: every slab whole in one;
# 410 x 10 = 4100 units, 8 or 9 per workgroup: slabs over two workgroups; the headline, 272 x 20,
# 10 or 11 per workgroup: slabs over two or three; a pair of 128 slabs x 2 x 20; a pair of
# 512 slabs x 2 x 4, every slab (gate and up) whole in one workgroup
SHAPES = [(32768, 2048, False), (26240, 2560, False), (17408, 5120, False), (8192, 5120, True), (32768, 1024, True)]
N = 5


def _run(hl, dev, t, wg, wu, x, rows, cols, norm_w=None):
    import torch

    n_vec = x.shape[0]
    y = torch.full((n_vec, rows + 1), SENTINEL, dtype=torch.float32, device=dev)
    xd = to_dev(x, dev)
    nw = to_dev(norm_w, dev) if norm_w is not None else None
    if wu is None:
        hl.gemv(t, wg, xd, y, rows, cols, n_vec, y_stride=rows + 1, variant=hl.Variant.SLAB_GEMV, norm_w=nw,
                norm_eps=EPS)
    else:
        hl.gate_up_swiglu(t, wg, wu, xd, y, rows, cols, n_vec, out_stride=rows + 1, variant=hl.Variant.SLAB_GEMV)
    out = host(y)
    assert np.all(out[:, rows:] == SENTINEL), "y padding written"
    return out[:, :rows]


@pytest.mark.parametrize("t", EVEN_TYPES)
@pytest.mark.parametrize("rows,cols,pair", SHAPES)
def test_even_split_bound_invariance_repeat(hl, oracle, dev, t, rows, cols, pair):
    say("even split", NAMES[t], rows, cols, "pair" if pair else "")
    dg = synth_matrix(hl, t, rows, cols, 700 + rows + cols)
    du = synth_matrix(hl, t, rows, cols, 701 + rows + cols) if pair else None
    wg = slab_of(hl, dev, t, dg, rows, cols)
    wu = slab_of(hl, dev, t, du, rows, cols) if pair else None
    x = np.random.default_rng(7000 + rows).standard_normal((N, cols)).astype(np.float32)
    singles = np.concatenate([_run(hl, dev, t, wg, wu, x[i:i + 1], rows, cols) for i in range(N)])
    if pair:
        g = oracle.matmul(t, dg, rows, cols, x)
        u = oracle.matmul(t, du, rows, cols, x)
        ref = oracle.gate_up_swiglu(t, dg, du, rows, cols, x)
        tol = swiglu_tol(g, u, slab_gemv_tol(oracle, t, dg, rows, cols, x), slab_gemv_tol(oracle, t, du, rows, cols, x),
                         ref)
    else:
        ref = oracle.matmul(t, dg, rows, cols, x)
        tol = slab_gemv_tol(oracle, t, dg, rows, cols, x)
    err = np.abs(singles.astype(np.float64) - ref)
    print(f"    even split {NAMES[t]} {rows}x{cols} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    for n_vec in (2, 3, 4, 5):
        assert isclose_bits(_run(hl, dev, t, wg, wu, x[:n_vec], rows, cols), singles[:n_vec]), \
            f"n_vec={n_vec} changed a row"
    assert isclose_bits(_run(hl, dev, t, wg, wu, x[:4], rows, cols), singles[:4]), "a repeated call changed"


@pytest.mark.parametrize("t", EVEN_TYPES)
@pytest.mark.parametrize("rows,cols", [(32768, 2048), (26240, 2560), (17408, 5120)])
def test_even_split_fused_norm_bitwise(hl, oracle, dev, t, rows, cols):
    """One vector: the norm inside the even kernel (the first workgroup publishes 1 / rms to one
    word per workgroup) is bitwise RMS_NORM then the unfused GEMV; three calls in a row (the words
    are cleared by their readers, the generations move on), the last with a row of very large and
    widely spread magnitudes."""
    say("even split norm", NAMES[t], rows, cols)
    dg = synth_matrix(hl, t, rows, cols, 710 + rows)
    wg = slab_of(hl, dev, t, dg, rows, cols)
    rng = np.random.default_rng(7100 + rows)
    w = rng.uniform(0.25, 1.75, cols).astype(np.float32)
    for call in range(3):
        x = (rng.standard_normal((1, cols)) * 3.0).astype(np.float32)
        if call == 2:  # a row of 2^30 N(0, 1), each 256-column group scaled by 2^k (|k| <= 20)
            x *= np.float32(2.0 ** 30) * np.repeat(np.ldexp(1.0, rng.integers(-20, 21, cols // 256)), 256).astype(np.float32)
        xn = oracle.rms_norm(x, w, EPS)
        fused = _run(hl, dev, t, wg, None, x, rows, cols, norm_w=w)
        assert isclose_bits(fused, _run(hl, dev, t, wg, None, xn, rows, cols)), \
            f"call {call}: the fused norm is not bitwise rms_norm then the gemv"


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 26200, 2560), (IQ4_XS, 26200, 2560), (Q5_K, 26200, 2560),
                                          (Q4_0, 32768, 3104), (Q8_0, 32768, 3104)])
def test_even_split_partial_slab_and_group(hl, oracle, dev, t, rows, cols):
    """A last slab of 24 rows (410 slabs x 10 groups) and, for the 32-weight blocks, a last slot
    group of one slot (97 slots: 13 groups per row, 6656 units): within the bound, rows
    independent of n_vec, and nothing written past the rows."""
    say("even split partial", NAMES[t], rows, cols)
    dg = synth_matrix(hl, t, rows, cols, 720 + rows + cols)
    wg = slab_of(hl, dev, t, dg, rows, cols)
    x = np.random.default_rng(7200 + cols).standard_normal((3, cols)).astype(np.float32)
    singles = np.concatenate([_run(hl, dev, t, wg, None, x[i:i + 1], rows, cols) for i in range(3)])
    ref = oracle.matmul(t, dg, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, dg, rows, cols, x)
    err = np.abs(singles.astype(np.float64) - ref)
    print(f"    even split {NAMES[t]} {rows}x{cols} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    assert isclose_bits(_run(hl, dev, t, wg, None, x, rows, cols), singles), "n_vec=3 changed a row"


@pytest.mark.parametrize("n_vec", [1, 3])
def test_even_split_lm_head(hl, oracle, dev, n_vec):
    """The LM head's argmax epilogue on the even split (500 slabs x 16 groups = 8000 units): the
    result is the first maximum of its own logits, which are bitwise the plain GEMV's and within
    its bound of the CPU."""
    import torch

    t, rows, cols = Q4_K, 32000, 4096
    say("even split lm_head", rows, cols, n_vec)
    dg = synth_matrix(hl, t, rows, cols, 730)
    wg = slab_of(hl, dev, t, dg, rows, cols)
    x = np.random.default_rng(7300 + n_vec).standard_normal((n_vec, cols)).astype(np.float32)
    res = torch.full((n_vec, 3), 0xABCD, dtype=torch.int32, device=dev)
    logits = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.lm_head(t, wg, to_dev(x, dev), res, rows, cols, n_vec, logits=logits, variant=hl.Variant.SLAB_GEMV)
    r, y = host(res).view(np.uint32), host(logits)
    assert isclose_bits(y, _run(hl, dev, t, wg, None, x, rows, cols)), "the head's logits are not the GEMV's"
    ref = oracle.matmul(t, dg, rows, cols, x)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= slab_gemv_tol(oracle, t, dg, rows, cols, x))
    for v in range(n_vec):
        i = int(np.argmax(y[v]))
        assert r[v].tolist() == [i, int(y[v, i].view(np.uint32)), 0], f"vector {v}: not the first maximum"
