"""GPU parity of the RMS-norm prologue of the matmul (GemvArgs::norm_w / norm_eps,
include/halo/backend/backend.h:292-299), of RMS_NORM itself (cpu::rms_norm,
backends/cpu/ops_basic.cpp:18-33), of GET_ROWS (GetRowsArgs, backend.h:254-263; the HIP
status word of backends/hip/src/ops.cpp:982-1012) and of the grouped GEMV over matrices that
share x, against the oracle, through the C ABI.

Acceptance: RMS_NORM, GET_ROWS and the reference-order GEMV with the norm are bitwise the CPU's;
every variant with the fused norm is bitwise RMS_NORM then the same variant without it (the
reference's Limits::max_fused_norm_cols contract, backend.h:236-242: an R == 1 decode must stay
bitwise the unfused R > 1 verify forward), so the unfused bounds apply to the CPU's normalized x.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import (ALL_TYPES, GGUF_TYPES, PLAIN_TYPES, F16, F32, IQ4_XS, SLAB_TYPES, NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANT_TYPES, gemm_emulated, gemm_tol,
                     isclose_bits, make_weights, max_ratio, row_bytes, slab_gemv_tol, swiglu_tol)
from test_gpu_parity import SENTINEL, dense_of, host, say, slab_of, strided_xy, to_dev

pytestmark = pytest.mark.gpu

EPS = 1e-6


def norm_inputs(cols, n_vec, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n_vec, cols)) * 3.0).astype(np.float32)
    w = rng.uniform(0.25, 1.75, cols).astype(np.float32)
    return x, w


# ---- RMS_NORM ---------------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (4, 100), (2, 4097), (5, 5120), (2, 17408), (64, 256)])
def test_rms_norm_bitwise(hl, oracle, dev, rows, cols):
    import torch

    say("rms_norm", rows, cols)
    x, w = norm_inputs(cols, rows, 10 + cols)
    ref = oracle.rms_norm(x, w, EPS)
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    out = torch.full_like(xd, SENTINEL)
    hl.rms_norm(xd, wd, out, rows, cols, eps=EPS)
    assert isclose_bits(host(out), ref), "RMS_NORM differs from cpu::rms_norm"
    hl.rms_norm(xd, wd, xd, rows, cols, eps=EPS)  # in place, as the CPU allows
    assert isclose_bits(host(xd), ref), "in-place RMS_NORM differs"


def test_rms_norm_strided_and_rejects(hl, oracle, dev):
    import torch

    rows, cols = 3, 520
    say("rms_norm strided", rows, cols)
    x, w = norm_inputs(cols, rows, 7)
    xp = np.full((rows, cols + 3), 5.0, np.float32)
    xp[:, :cols] = x
    xd, wd = to_dev(xp, dev), to_dev(w, dev)
    out = torch.full((rows, cols + 5), SENTINEL, dtype=torch.float32, device=dev)
    hl.rms_norm(xd, wd, out, rows, cols, eps=EPS, x_stride=cols + 3, out_stride=cols + 5)
    o = host(out)
    assert isclose_bits(o[:, :cols], oracle.rms_norm(x, w, EPS))
    assert np.all(o[:, cols:] == SENTINEL), "padding written"
    with pytest.raises(hl.HaloError) as e:  # out overlapping x without being x
        hl.rms_norm(xd, wd, xd.data_ptr() + 4, rows, cols, eps=EPS, x_stride=cols + 3, out_stride=cols + 3)
    assert e.value.code == hl.ErrorCode.Kernel


# ---- GET_ROWS ---------------------------------------------------------------------------------


@pytest.mark.parametrize("t", GGUF_TYPES)
@pytest.mark.parametrize("layout", ["gguf", "slab"])
def test_get_rows_bitwise_and_bad_ids(hl, oracle, dev, t, layout):
    import torch

    if layout == "slab" and t not in SLAB_TYPES:
        pytest.skip(f"{NAMES[t]} has no SLAB layout")
    rows, cols = 70, 512
    say("get_rows", NAMES[t], layout, rows, cols)
    pad, off = ((4, 4) if t in PLAIN_TYPES else (3, 1)) if layout == "gguf" else (0, 0)
    buf, stride = make_weights(t, rows, cols, seed=900 + t, stride_pad=pad, offset=off)
    ref = oracle.dequantize_rows(t, buf[off:], rows, cols, stride)
    if layout == "gguf":
        wd = to_dev(buf, dev)
        table, lay, ts = wd.data_ptr() + off, hl.Layout.GGUF, stride
    else:
        table, lay, ts = slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, off), rows, cols), hl.Layout.SLAB, 0
    ids = np.array([5, 0, 69, 5, -1, 33, 70, 64, 1], np.int32)
    idd = to_dev(ids, dev)
    status = torch.full((1,), 0x55, dtype=torch.int32, device=dev)  # cleared by the call
    out = torch.full((ids.size, cols + 2), SENTINEL, dtype=torch.float32, device=dev)
    keep = torch.full((1,), 0x40, dtype=torch.int32, device=dev)  # status_keep: bits accumulate
    hl.get_rows(t, lay, table, rows, cols, idd, ids.size, out, table_stride=ts, out_stride=cols + 2, status=keep,
                status_keep=True)
    assert int(host(keep)[0]) == 0x40 | hl.STATUS_BAD_INDEX
    hl.get_rows(t, lay, table, rows, cols, idd, ids.size, out, table_stride=ts, out_stride=cols + 2, status=status)
    o = host(out)
    for i, r in enumerate(ids):
        if 0 <= r < rows:
            assert isclose_bits(o[i, :cols], ref[r]), f"row {i} (id {r}) differs from tensor::dequantize_row"
        else:
            assert np.all(o[i] == SENTINEL), f"row {i} (bad id {r}) was written"
    assert np.all(o[:, cols:] == SENTINEL)
    assert int(host(status)[0]) == hl.STATUS_BAD_INDEX
    good = to_dev(np.array([3, 2, 1], np.int32), dev)
    hl.get_rows(t, lay, table, rows, cols, good, 3, out, table_stride=ts, out_stride=cols + 2, status=status)
    assert int(host(status)[0]) == 0, "a call with valid ids leaves the status word clear"
    assert isclose_bits(host(out)[:3, :cols], ref[[3, 2, 1]])


def test_get_rows_rejects(hl, dev):
    import torch

    t, rows, cols = Q4_K, 8, 256
    buf, _ = make_weights(t, rows, cols, seed=1)
    wd = to_dev(buf, dev)
    ids = to_dev(np.zeros(2, np.int32), dev)
    out = torch.zeros((2, cols), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # out overlaps the table
        hl.get_rows(t, hl.Layout.GGUF, wd, rows, cols, ids, 2, wd)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:
        hl.get_rows(t, 7, wd, rows, cols, ids, 2, out)
    assert e.value.code == hl.ErrorCode.Config
    with pytest.raises(hl.HaloError) as e:
        hl.get_rows(11, hl.Layout.SLAB, wd, rows, cols, ids, 2, out)
    assert e.value.code == hl.ErrorCode.Unsupported


# ---- the fused norm in the matmul ---------------------------------------------------------


def run_norm_gemv(hl, dev, t, w, x, nw, rows, cols, variant, layout=None, w_stride=0, x_pad=0, y_pad=0):
    xd, xs, yd, ys = strided_xy(dev, x, rows, x_pad, y_pad)
    hl.gemv(t, w, xd, yd, rows, cols, x.shape[0], layout=hl.Layout.SLAB if layout is None else layout, w_stride=w_stride,
            x_stride=xs, y_stride=ys, variant=variant, norm_w=to_dev(nw, dev), norm_eps=EPS)
    y = host(yd)
    assert np.all(y[:, rows:] == SENTINEL), "y padding overwritten"
    return y[:, :rows]


@pytest.mark.parametrize("t", QUANT_TYPES + (F32,))
def test_gemv_norm_reference_variant_bitwise(hl, oracle, dev, t):
    rows, cols, n_vec = 37, (100 if t == F32 else 1024), 3
    say("gemv norm gguf_ref", NAMES[t], rows, cols, n_vec)
    pad, off = (4, 4) if t == F32 else (3, 1)
    buf, stride = make_weights(t, rows, cols, seed=950 + t, stride_pad=pad, offset=off)
    x, w = norm_inputs(cols, n_vec, 951 + t)
    ref = oracle.matmul(t, buf[off:], rows, cols, oracle.rms_norm(x, w, EPS), w_stride=stride)
    wd = to_dev(buf, dev)
    y = run_norm_gemv(hl, dev, t, wd.data_ptr() + off, x, w, rows, cols, hl.Variant.GGUF_REF, layout=hl.Layout.GGUF,
                      w_stride=stride, x_pad=5, y_pad=3)
    assert isclose_bits(y, ref), "reference-order gemv with the norm is not bitwise rms_norm + cpu::matmul"


# One vector with cols <= 8192 takes the norm inside the GEMV kernel (one dispatch: the norm wave
# of the first workgroup publishes 1 / rms); more vectors, and the 17408-column row, the RMS_NORM
# kernel then the GEMV. (17408, 5120, 1) is the headline shape (1088 workgroups of 5 + 1 waves);
# 65600 rows: more than 1024 slabs (two groups per wave).
NORM_CASES = [(130, 1024, 1), (130, 1024, 4), (576, 5120, 1), (576, 5120, 3), (640, 17408, 1), (70, 512, 6),
              (65600, 512, 1), (65600, 512, 4), (17408, 5120, 1), (64, 256, 1)]  # (64, 256, 1): one workgroup


def unfused_gemv(hl, dev, t, w, xn, rows, cols, variant):
    """The same variant without the norm, on RMS_NORM's output computed on the GPU."""
    import torch

    yd = torch.full((xn.shape[0], rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gemv(t, w, to_dev(xn, dev), yd, rows, cols, xn.shape[0], variant=variant)
    return host(yd)


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("case", NORM_CASES)
def test_gemv_norm_slab_bitwise(hl, oracle, dev, t, case):
    rows, cols, n_vec = case
    if rows > 10000 and t not in (Q4_K, Q6_K):
        pytest.skip("the many-slab and headline shapes run for Q4_K and Q6_K")
    say("gemv norm slab", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=960 + t + rows)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x, w = norm_inputs(cols, n_vec, 961 + cols + n_vec)
    xn = oracle.rms_norm(x, w, EPS)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    variants = [hl.Variant.SLAB_GEMV, hl.Variant.SLAB_AUTO]
    if cols % 256 == 0:
        variants.append(hl.Variant.SLAB_GEMM_EXACT_INVARIANT)
    for variant in variants:
        y = run_norm_gemv(hl, dev, t, slab, x, w, rows, cols, variant, x_pad=1, y_pad=2)
        assert isclose_bits(y, unfused_gemv(hl, dev, t, slab, xn, rows, cols, variant)), \
            f"variant {int(variant)}: the fused norm is not bitwise rms_norm then the gemv"
    ref = oracle.matmul(t, dense, rows, cols, xn)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, xn)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    fused-norm gemv {NAMES[t]} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_gemv_norm_in_kernel_sum_order(hl, oracle, dev, t):
    """The in-kernel norm's sum of squares follows cpu::detail::dot's order exactly: x[0] = 4096
    and ones everywhere else put 2^24 and then ones into one chain, where the order decides the
    sum (2^24 + 1 rounds back to 2^24 one addition at a time). The fused one-vector GEMV must equal
    RMS_NORM (bitwise the oracle) then the GEMV, and the two orders give different inv here."""
    rows, cols = 1024, 5120
    say("gemv norm sum order", NAMES[t], rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=965 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.ones((1, cols), np.float32)
    x[0, 0] = 4096.0
    x[0, 1::2] *= -1.0
    w = np.random.default_rng(966).uniform(0.25, 1.75, cols).astype(np.float32)
    xn = oracle.rms_norm(x, w, EPS)
    # a different order (the pairwise sum numpy uses in float32) gives a different inv
    inv_other = np.float32(1.0) / np.sqrt(np.float32(np.sum(x * x, dtype=np.float32)) / np.float32(cols) + np.float32(EPS))
    assert not isclose_bits((x * inv_other) * w, xn), "the test input does not separate the orders"
    for variant in (hl.Variant.SLAB_GEMV, hl.Variant.DEFAULT):
        y = run_norm_gemv(hl, dev, t, slab, x, w, rows, cols, variant)
        assert isclose_bits(y, unfused_gemv(hl, dev, t, slab, xn, rows, cols, variant)), \
            f"variant {int(variant)}: the in-kernel norm is not bitwise rms_norm then the gemv"


@pytest.mark.parametrize("t", (Q4_K, Q6_K, IQ4_XS))
@pytest.mark.parametrize("rows,cols", [(130, 1024), (576, 5120)])
@pytest.mark.parametrize("variant", ["SLAB_GEMV", "SLAB_GEMM_EXACT_INVARIANT"])
def test_gemv_norm_rows_do_not_depend_on_the_batch(hl, dev, t, rows, cols, variant):
    say("gemv norm batch invariance", variant, NAMES[t], rows, cols)
    v = getattr(hl.Variant, variant)
    buf, stride = make_weights(t, rows, cols, seed=970 + t + rows)
    slab = slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols)
    x, w = norm_inputs(cols, 9, 971)
    singles = np.stack([run_norm_gemv(hl, dev, t, slab, x[i:i + 1], w, rows, cols, v)[0] for i in range(9)])
    for n_vec in (2, 3, 4, 5, 9):
        y = run_norm_gemv(hl, dev, t, slab, x[:n_vec], w, rows, cols, v)
        assert isclose_bits(y, singles[:n_vec]), f"n_vec={n_vec} changed a row"


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("n_vec,variant", [(40, 3), (300, 3), (600, 5)])
def test_gemm_norm_within_bounds(hl, oracle, dev, t, n_vec, variant):
    rows, cols = 130, 1024
    say("gemm norm", NAMES[t], rows, cols, n_vec, variant)
    buf, stride = make_weights(t, rows, cols, seed=980 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x, w = norm_inputs(cols, n_vec, 981 + n_vec)
    xn = oracle.rms_norm(x, w, EPS)
    ref = oracle.matmul(t, dense, rows, cols, xn)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    y = run_norm_gemv(hl, dev, t, slab, x, w, rows, cols, variant, x_pad=4, y_pad=1)
    assert isclose_bits(y, unfused_gemv(hl, dev, t, slab, xn, rows, cols, variant)), \
        "the GEMM's fused norm is not bitwise rms_norm then the GEMM"
    err = np.abs(y.astype(np.float64) - ref)
    tol = gemm_tol(oracle, t, dense, rows, cols, xn)
    print(f"    gemm+norm vs cpu: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    emu, etol = gemm_emulated(oracle, t, dense, rows, cols, xn)  # the staged x is the CPU's xn in bf16
    assert np.all(np.abs(y.astype(np.float64) - emu) <= etol)


@pytest.mark.parametrize("t", (Q4_K, Q6_K, Q5_K, IQ4_XS, Q8_0, Q4_0))
@pytest.mark.parametrize("n_vec,variant", [(1, 2), (4, 2), (17, 3), (600, 5), (1, 9), (5, 9), (11, 9)])
def test_gate_up_norm(hl, oracle, dev, t, n_vec, variant):
    import torch

    rows, cols = 96, 1024
    say("gate_up norm", NAMES[t], rows, cols, n_vec, variant)
    bg, sg = make_weights(t, rows, cols, seed=990 + t)
    bu, su = make_weights(t, rows, cols, seed=995 + t)
    dg, du = dense_of(bg, t, rows, cols, sg, 0), dense_of(bu, t, rows, cols, su, 0)
    x, w = norm_inputs(cols, n_vec, 991 + n_vec)
    xn = oracle.rms_norm(x, w, EPS)
    ref = oracle.gate_up_swiglu(t, dg, du, rows, cols, xn)
    g, u = oracle.matmul(t, dg, rows, cols, xn), oracle.matmul(t, du, rows, cols, xn)
    if variant in (2, 9):  # the exact arithmetic: the slab GEMV's bound (9: IEEE SiLU in the kernel)
        tg, tu = slab_gemv_tol(oracle, t, dg, rows, cols, xn), slab_gemv_tol(oracle, t, du, rows, cols, xn)
    else:
        tg, tu = gemm_tol(oracle, t, dg, rows, cols, xn), gemm_tol(oracle, t, du, rows, cols, xn)
    tol = swiglu_tol(g, u, tg, tu, ref, fast=variant not in (2, 9))
    out = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    sg, su = slab_of(hl, dev, t, dg, rows, cols), slab_of(hl, dev, t, du, rows, cols)
    hl.gate_up_swiglu(t, sg, su, to_dev(x, dev), out, rows, cols, n_vec, variant=variant, norm_w=to_dev(w, dev),
                      norm_eps=EPS)
    plain = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gate_up_swiglu(t, sg, su, to_dev(xn, dev), plain, rows, cols, n_vec, variant=variant)
    assert isclose_bits(host(out), host(plain)), "the fused norm is not bitwise rms_norm then gate_up"
    err = np.abs(host(out).astype(np.float64) - ref)
    print(f"    gate_up+norm worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


@pytest.mark.parametrize("t", (Q4_K, Q6_K))
@pytest.mark.parametrize("variant", [0, 1, 3])
@pytest.mark.parametrize("n_vec", [1, 3])
def test_lm_head_norm(hl, oracle, dev, t, variant, n_vec):
    """The LM head with the output norm folded in: the argmax is the first maximum of the GPU's
    own logits, the logits are within the variant's bound of the CPU's (rms_norm then matmul).
    One vector on the SLAB GEMV takes the norm inside the kernel."""
    import torch

    rows, cols = 1000, 512
    say("lm_head norm", NAMES[t], rows, cols, n_vec, variant)
    buf, stride = make_weights(t, rows, cols, seed=1000 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x, w = norm_inputs(cols, n_vec, 1001)
    xn = oracle.rms_norm(x, w, EPS)
    if variant == 1:
        wt, lay = to_dev(dense, dev), hl.Layout.GGUF
    else:
        wt, lay = slab_of(hl, dev, t, dense, rows, cols), hl.Layout.SLAB
    res = torch.full((n_vec, 3), 0xABCD, dtype=torch.int32, device=dev)
    y = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.lm_head(t, wt, to_dev(x, dev), res, rows, cols, n_vec, logits=y, layout=lay, variant=variant,
               norm_w=to_dev(w, dev), norm_eps=EPS)
    r, yl = host(res).view(np.uint32), host(y)
    cpu, cpu_logits = oracle.lm_head(t, dense, rows, cols, xn)
    if variant == 1:
        assert isclose_bits(yl, cpu_logits) and np.array_equal(r, cpu), "reference variant: not the CPU's bits"
        return
    tol = gemm_tol(oracle, t, dense, rows, cols, xn) if variant == 3 else slab_gemv_tol(oracle, t, dense, rows, cols, xn)
    assert np.all(np.abs(yl.astype(np.float64) - cpu_logits) <= tol)
    # the same head on RMS_NORM's output, without the norm: bitwise the same logits and result
    res2 = torch.full((n_vec, 3), 0xABCD, dtype=torch.int32, device=dev)
    y2 = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    xg = torch.empty((n_vec, cols), dtype=torch.float32, device=dev)
    hl.rms_norm(to_dev(x, dev), to_dev(w, dev), xg, n_vec, cols, eps=EPS)
    hl.lm_head(t, wt, xg, res2, rows, cols, n_vec, logits=y2, layout=lay, variant=variant)
    assert isclose_bits(yl, host(y2)), "logits: the fused norm is not bitwise rms_norm then the head"
    assert np.array_equal(r, host(res2).view(np.uint32))
    for v in range(n_vec):
        i = int(np.argmax(yl[v]))
        assert r[v].tolist() == [i, int(yl[v, i:i + 1].view(np.uint32)[0]), 0]


def test_norm_rejects(hl, dev):
    import torch

    t, rows, cols = Q4_K, 64, 256
    buf, _ = make_weights(t, rows, cols, seed=2)
    slab = slab_of(hl, dev, t, buf[:rows * row_bytes(t, cols)], rows, cols)
    x = to_dev(np.ones((1, cols), np.float32), dev)
    y = torch.zeros((1, rows), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # norm_w overlapping y
        hl.gemv(t, slab, x, y, rows, cols, 1, norm_w=y)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:  # misaligned norm_w
        hl.gemv(t, slab, x, y, rows, cols, 1, norm_w=x.data_ptr() + 2)
    assert e.value.code == hl.ErrorCode.Kernel


# ---- grouped GEMV (halo_mi_gemv_group) ------------------------------------------------------


GROUPS = [
    [(Q4_K, 640), (Q4_K, 128), (Q6_K, 128)],             # q, k, v: two types, one launch
    [(Q5_K, 200), (IQ4_XS, 70), (Q6_K, 64), (Q8_0, 33)],  # four types: two launches
    [(Q4_K, 1088)],                                      # one segment
]


@pytest.mark.parametrize("g", range(len(GROUPS)))
@pytest.mark.parametrize("n_vec,norm", [(1, False), (3, False), (1, True), (6, True)])
def test_gemv_group_within_bounds(hl, oracle, dev, g, n_vec, norm):
    import torch

    cols = 1024
    say("gemv_group", g, n_vec, norm)
    x, w = norm_inputs(cols, n_vec, 1200 + g)
    xn = oracle.rms_norm(x, w, EPS) if norm else x
    segs, refs = [], []
    for i, (t, rows) in enumerate(GROUPS[g]):
        buf, stride = make_weights(t, rows, cols, seed=1210 + 10 * g + i)
        dense = dense_of(buf, t, rows, cols, stride, 0)
        y = torch.full((n_vec, rows + 3), SENTINEL, dtype=torch.float32, device=dev)
        segs.append((t, slab_of(hl, dev, t, dense, rows, cols), rows, y, rows + 3))
        tol = slab_gemv_tol(oracle, t, dense, rows, cols, xn)
        refs.append((oracle.matmul(t, dense, rows, cols, xn), tol))
    xd = to_dev(x, dev)
    plain = None
    if norm:  # the fused norm is bitwise rms_norm then the same group
        plain = [torch.zeros((n_vec, rows), dtype=torch.float32, device=dev) for (_, _, rows, _, _) in segs]
        hl.gemv_group([(t, wt, rows, p) for (t, wt, rows, _, _), p in zip(segs, plain)], to_dev(xn, dev), cols, n_vec)
    for rep in range(2):  # twice: the workspace words and counters are left clean
        hl.gemv_group(segs, xd, cols, n_vec, norm_w=to_dev(w, dev) if norm else None, norm_eps=EPS)
        for k, ((t, _, rows, y, _), (ref, tol)) in enumerate(zip(segs, refs)):
            out = host(y)
            assert np.all(out[:, rows:] == SENTINEL), "y padding written"
            err = np.abs(out[:, :rows].astype(np.float64) - ref)
            assert np.all(err <= tol), f"{NAMES[t]}: worst |d|/bound = {max_ratio(err, tol):.3f}"
            if plain is not None:
                assert isclose_bits(out[:, :rows], host(plain[k])), f"{NAMES[t]}: fused norm not bitwise"


def test_gemv_group_norm_layer_shapes(hl, dev):
    """The config-5 layer's q, k (Q4_K) and v (Q6_K) over the 5120-wide attention input, one
    vector with the input norm: the norm inside the grouped kernel, bitwise RMS_NORM then the
    same group."""
    import torch

    cols = 5120
    say("gemv_group norm layer shapes", cols)
    x, w = norm_inputs(cols, 1, 1250)
    segs = []
    for i, (t, rows) in enumerate([(Q4_K, 6144), (Q4_K, 1024), (Q6_K, 1024)]):
        buf, stride = make_weights(t, rows, cols, seed=1260 + i)
        segs.append((t, slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols), rows))
    xg = torch.empty((1, cols), dtype=torch.float32, device=dev)
    hl.rms_norm(to_dev(x, dev), to_dev(w, dev), xg, 1, cols, eps=EPS)
    plain = [torch.zeros((1, rows), dtype=torch.float32, device=dev) for _, _, rows in segs]
    hl.gemv_group([(t, wt, rows, p) for (t, wt, rows), p in zip(segs, plain)], xg, cols, 1)
    for rep in range(2):
        fused = [torch.full((1, rows), SENTINEL, dtype=torch.float32, device=dev) for _, _, rows in segs]
        hl.gemv_group([(t, wt, rows, f) for (t, wt, rows), f in zip(segs, fused)], to_dev(x, dev), cols, 1,
                      norm_w=to_dev(w, dev), norm_eps=EPS)
        for k, (f, p) in enumerate(zip(fused, plain)):
            assert isclose_bits(host(f), host(p)), f"segment {k}: the in-kernel norm is not bitwise rms_norm then the group"


def test_gemv_group_rows_do_not_depend_on_the_batch(hl, dev):
    import torch

    cols = 1024
    x, _ = norm_inputs(cols, 5, 1300)
    segs = []
    for i, (t, rows) in enumerate(GROUPS[0]):
        buf, stride = make_weights(t, rows, cols, seed=1310 + i)
        segs.append((t, slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols), rows))

    def run(xs):
        ys = [torch.zeros((xs.shape[0], rows), dtype=torch.float32, device=dev) for _, _, rows in segs]
        hl.gemv_group([(t, w, rows, y) for (t, w, rows), y in zip(segs, ys)], to_dev(xs, dev), cols, xs.shape[0])
        return [host(y) for y in ys]

    singles = [run(x[i:i + 1]) for i in range(5)]
    batch = run(x)
    for k in range(len(segs)):
        assert isclose_bits(batch[k], np.concatenate([s[k] for s in singles])), f"segment {k}: a row changed with n_vec"


@pytest.mark.parametrize("g", range(len(GROUPS)))
@pytest.mark.parametrize("n_vec,norm", [(9, False), (40, True), (130, False), (300, True), (600, False)])
def test_gemm_group_within_bounds(hl, oracle, dev, g, n_vec, norm):
    """The grouped bf16 GEMM (halo_mi_gemm_group): x staged once, one launch per pair of weight
    types (64-, 128- and 256-row M tiles; small groups split over K and reduced together), every
    output within the bf16 GEMM's bound against the CPU and the fp64 products of its own
    bf16-rounded operands; a second call bitwise the first; padding untouched."""
    import torch

    cols = 1024
    say("gemm_group", g, n_vec, norm)
    x, w = norm_inputs(cols, n_vec, 1400 + g)
    xn = oracle.rms_norm(x, w, EPS) if norm else x
    segs, refs = [], []
    for i, (t, rows) in enumerate(GROUPS[g]):
        buf, stride = make_weights(t, rows, cols, seed=1410 + 10 * g + i)
        dense = dense_of(buf, t, rows, cols, stride, 0)
        y = torch.full((n_vec, rows + 3), SENTINEL, dtype=torch.float32, device=dev)
        segs.append((t, slab_of(hl, dev, t, dense, rows, cols), rows, y, rows + 3))
        emu, etol = gemm_emulated(oracle, t, dense, rows, cols, xn)
        refs.append((oracle.matmul(t, dense, rows, cols, xn), gemm_tol(oracle, t, dense, rows, cols, xn), emu, etol))
    xd = to_dev(x, dev)
    first = None
    for rep in range(2):
        hl.gemm_group(segs, xd, cols, n_vec, norm_w=to_dev(w, dev) if norm else None, norm_eps=EPS)
        outs = [host(y) for (_, _, _, y, _) in segs]
        for (t, _, rows, _, _), out, (ref, tol, emu, etol) in zip(segs, outs, refs):
            assert np.all(out[:, rows:] == SENTINEL), "y padding written"
            o = out[:, :rows].astype(np.float64)
            assert np.all(np.abs(o - ref) <= tol), f"{NAMES[t]}: vs cpu worst |d|/bound = {max_ratio(np.abs(o - ref), tol):.3f}"
            assert np.all(np.abs(o - emu) <= etol), \
                f"{NAMES[t]}: vs bf16-exact products worst |d|/bound = {max_ratio(np.abs(o - emu), etol):.3f}"
        if first is None:
            first = outs
        else:
            for a, b in zip(first, outs):
                assert isclose_bits(a, b), "a second grouped GEMM call gave different bits"


@pytest.mark.parametrize("n_vec", [64, 512])
def test_gemm_group_layer_qkv(hl, oracle, dev, n_vec):
    """Config 5's q (6144 rows), k (1024) and v (1024 rows, Q6_K) over the 5120-wide input at
    M = 64 and 512 in one grouped GEMM call, every output within the bf16-exact-product bound."""
    import torch

    cols = 5120
    say("gemm_group layer q|k|v", n_vec)
    x = hl.fill_normal(1450 + n_vec, n_vec * cols).reshape(n_vec, cols)
    segs, refs = [], []
    for i, (t, rows) in enumerate([(Q4_K, 6144), (Q4_K, 1024), (Q6_K, 1024)]):
        from helpers import synth_matrix
        wq = synth_matrix(hl, t, rows, cols, 1460 + i)
        y = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
        segs.append((t, slab_of(hl, dev, t, wq, rows, cols), rows, y))
        refs.append(gemm_emulated(oracle, t, wq, rows, cols, x))
    hl.gemm_group(segs, to_dev(x, dev), cols, n_vec)
    for (t, _, rows, y), (emu, etol) in zip(segs, refs):
        err = np.abs(host(y).astype(np.float64) - emu)
        print(f"    {NAMES[t]} {rows} rows M={n_vec}: worst |d|/bound = {max_ratio(err, etol):.4f}")
        assert np.all(err <= etol)


def test_gemm_group_rejects(hl, dev):
    import torch

    cols = 256
    buf, _ = make_weights(Q4_K, 64, cols, seed=4)
    w = slab_of(hl, dev, Q4_K, buf[:64 * row_bytes(Q4_K, cols)], 64, cols)
    x = torch.ones((16, cols + 1), dtype=torch.float32, device=dev)
    y = torch.zeros((16, 128), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # x rows not 16-byte aligned (stride of cols + 1 floats)
        hl.gemm_group([(Q4_K, w, 64, y)], x, cols, 16, x_stride=cols + 1)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:  # two outputs overlapping
        hl.gemm_group([(Q4_K, w, 64, y), (Q4_K, w, 64, y.data_ptr() + 128)], x, cols, 16, x_stride=cols + 1)
    assert e.value.code == hl.ErrorCode.Kernel


def test_gemv_group_rejects(hl, dev):
    import torch

    cols = 256
    buf, _ = make_weights(Q4_K, 64, cols, seed=3)
    w = slab_of(hl, dev, Q4_K, buf[:64 * row_bytes(Q4_K, cols)], 64, cols)
    x = to_dev(np.ones((1, cols), np.float32), dev)
    y = torch.zeros((1, 128), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # two outputs overlapping
        hl.gemv_group([(Q4_K, w, 64, y), (Q4_K, w, 64, y.data_ptr() + 128)], x, cols, 1)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:  # an output inside x
        hl.gemv_group([(Q4_K, w, 64, x)], x, cols, 1)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:
        hl.gemv_group([(Q4_K, w, 64, y)] * 5, x, cols, 1)
    assert e.value.code == hl.ErrorCode.Unsupported
