"""GPU parity of the path's smaller ops and of the stream state, through the C ABI:

- SWIGLU (EltwiseArgs, include/halo/backend/backend.h:420-427; cpu::swiglu,
  backends/cpu/ops_basic.cpp:165-167) against oracle_swiglu, with strided views;
- ARGMAX (ArgmaxArgs, backend.h:463-468; cpu::argmax, backends/cpu/matmul.cpp:61-72) against the
  oracle's result words: ties to the lowest index, NaN poisoning per vector;
- the kernel variants chosen by id only (the VALU slab GEMV, the small-M GEMM);
- the split-K reduction's failure path, forced from the host (every kernel still exits): the
  stream's status word turns into a Device error at halo_mi_stream_check, and the workspace is
  clean afterwards; halo_mi_stream_release frees a stream's workspace.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import (NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANT_TYPES, U, gemm_emulated, gemm_tol, isclose_bits,
                     make_weights, max_ratio, row_bytes, slab_gemv_tol, swiglu_tol)
from test_gpu_parity import SENTINEL, dense_of, host, say, slab_of, to_dev

pytestmark = pytest.mark.gpu


# ---- SWIGLU -------------------------------------------------------------------------------


@pytest.mark.parametrize("rows,cols,pads", [(1, 1, (0, 0, 0)), (3, 1000, (2, 5, 1)), (64, 17408, (0, 0, 0)),
                                            (7, 333, (1, 0, 4))])
def test_swiglu_against_oracle(hl, oracle, dev, rows, cols, pads):
    """silu(g) u with g, u and out at their own row strides; padding untouched. The kernel's
    silu is v / (1 + expf(-v)): within a few ulp of the CPU's libm form, so the bound is 8 ulp of
    |out| plus the propagated exp error."""
    import torch

    say("swiglu", rows, cols, pads)
    rng = np.random.default_rng(rows * 31 + cols)
    g = (rng.standard_normal((rows, cols)) * 6).astype(np.float32)
    u = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    g.flat[:4] = [0.0, -0.0, 88.0, -104.0][: min(4, g.size)]  # zero, overflow of exp(-v) to inf
    ref = oracle.swiglu(g, u)
    pg, pu, po = pads

    def padded(a, p, fill):
        h = np.full((rows, cols + p), fill, np.float32)
        h[:, :cols] = a
        return to_dev(h, dev)

    gd, ud = padded(g, pg, 7.0), padded(u, pu, 9.0)
    out = torch.full((rows, cols + po), SENTINEL, dtype=torch.float32, device=dev)
    hl.swiglu(gd, ud, out, rows, cols, gate_stride=cols + pg, up_stride=cols + pu, out_stride=cols + po)
    o = host(out)
    assert np.all(o[:, cols:] == SENTINEL), "padding written"
    err = np.abs(o[:, :cols].astype(np.float64) - ref)
    tol = 8 * U * np.abs(ref.astype(np.float64)) + 1e-38
    print(f"    swiglu worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


def test_swiglu_rejects(hl, dev):
    import torch

    a = torch.zeros((4, 64), dtype=torch.float32, device=dev)
    b = torch.zeros((4, 64), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # out overlaps gate
        hl.swiglu(a, b, a.data_ptr() + 64, 4, 64)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:  # stride below cols
        hl.swiglu(a, b, torch.zeros_like(a), 4, 64, gate_stride=32)
    assert e.value.code == hl.ErrorCode.Kernel


# ---- ARGMAX -------------------------------------------------------------------------------


@pytest.mark.parametrize("n,n_vec", [(1, 1), (300, 5), (151936, 3), (64, 2), (65, 4)])
def test_argmax_words_against_oracle(hl, oracle, dev, n, n_vec):
    import torch

    say("argmax", n, n_vec)
    rng = np.random.default_rng(n + n_vec)
    lg = rng.standard_normal((n_vec, n)).astype(np.float32)
    if n > 64:
        lg[0, [n // 2, n - 1]] = 50.0  # a tie across 64-row parts: the lower index wins
    if n_vec > 1:
        lg[1, n // 3] = np.nan         # poisons vector 1 only
    if n_vec > 2:
        lg[2, :] = -np.inf
    ref = oracle.argmax_words(lg)
    ld = torch.full((n_vec, n + 3), -7.0, dtype=torch.float32, device=dev)
    ld[:, :n] = to_dev(lg, dev)
    res = torch.full((n_vec, 3), 0x5A5A, dtype=torch.int32, device=dev)
    hl.argmax(ld, res, n, n_vec, logits_stride=n + 3)
    got = host(res).view(np.uint32)
    for v in range(n_vec):
        if ref[v, 2]:
            assert got[v, 0] == 0xFFFFFFFF and got[v, 2] == 1 and np.isnan(got[v, 1:2].view(np.float32)[0]), v
        else:
            assert np.array_equal(got[v], ref[v]), (v, got[v], ref[v])


def test_argmax_rejects(hl, dev):
    import torch

    lg = torch.zeros((2, 10), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:  # result inside the logits
        hl.argmax(lg, lg, 10, 2)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:  # empty row
        hl.argmax(lg, torch.zeros(6, dtype=torch.int32, device=dev), 0, 2)
    assert e.value.code == hl.ErrorCode.Kernel


# ---- variants chosen by id ------------------------------------------------------------------


@pytest.mark.parametrize("t", (Q4_0, Q8_0, Q4_K, Q6_K))
@pytest.mark.parametrize("n_vec", [1, 3, 6])
def test_gemv_slab_valu_variant(hl, oracle, dev, t, n_vec):
    """HALO_MI_GEMV_SLAB_VALU: the VALU slab kernel, within the SLAB GEMV bound, rows bitwise
    independent of n_vec (the same split as the MFMA kernel)."""
    import torch

    rows, cols = 576, 5120
    say("gemv valu", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=1500 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.random.default_rng(1501).standard_normal((n_vec, cols)).astype(np.float32)
    y = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gemv(t, slab, to_dev(x, dev), y, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMV_VALU)
    yh = host(y)
    ref = oracle.matmul(t, dense, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, x)
    err = np.abs(yh.astype(np.float64) - ref)
    print(f"    valu {NAMES[t]} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    y1 = torch.full((1, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gemv(t, slab, to_dev(x[-1:], dev), y1, rows, cols, 1, variant=hl.Variant.SLAB_GEMV_VALU)
    assert isclose_bits(host(y1)[0], yh[-1]), "the VALU kernel's rows depend on n_vec"


def test_gemv_slab_valu_rejects_other_formats(hl, dev):
    import torch

    t, rows, cols = Q5_K, 64, 256
    buf, stride = make_weights(t, rows, cols, seed=3)
    slab = slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols)
    y = torch.zeros((1, rows), dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:
        hl.gemv(t, slab, to_dev(np.ones((1, cols), np.float32), dev), y, rows, cols, 1,
                variant=hl.Variant.SLAB_GEMV_VALU)
    assert e.value.code == hl.ErrorCode.Unsupported
    with pytest.raises(hl.HaloError) as e:  # past the last id
        hl.gemv(t, slab, to_dev(np.ones((1, cols), np.float32), dev), y, rows, cols, 1,
                variant=max(int(v) for v in hl.Variant) + 1)
    assert e.value.code == hl.ErrorCode.Config


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("n_vec", [2, 9, 12, 16, 24, 32])
def test_gemm_small_m_variant(hl, oracle, dev, t, n_vec):
    """HALO_MI_GEMM_SLAB_BF16_SMALL_M: the small-M kernel by id, within the bf16 GEMM bounds; more
    than 32 vectors or cols not a multiple of 256 is Unsupported."""
    import torch

    rows, cols = 130, 1024
    say("gemm small-M", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=1600 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.random.default_rng(1601 + n_vec).standard_normal((n_vec, cols)).astype(np.float32)
    y = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gemv(t, slab, to_dev(x, dev), y, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMM_BF16_SMALL_M)
    yh = host(y).astype(np.float64)
    ref = oracle.matmul(t, dense, rows, cols, x)
    assert np.all(np.abs(yh - ref) <= gemm_tol(oracle, t, dense, rows, cols, x))
    emu, etol = gemm_emulated(oracle, t, dense, rows, cols, x)
    assert np.all(np.abs(yh - emu) <= etol)
    x33 = to_dev(np.ones((33, cols), np.float32), dev)
    with pytest.raises(hl.HaloError) as e:
        hl.gemv(t, slab, x33, torch.zeros((33, rows), dtype=torch.float32, device=dev), rows, cols, 33,
                variant=hl.Variant.SLAB_GEMM_BF16_SMALL_M)
    assert e.value.code == hl.ErrorCode.Unsupported


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("rows,cols", [(130, 1024), (576, 5120)])
@pytest.mark.parametrize("n_vec", [1, 2, 3, 4, 5, 8])
def test_gemm_exact_small_m_variant(hl, oracle, dev, t, rows, cols, n_vec):
    """HALO_MI_GEMM_SLAB_EXACT_SMALL_M: the slab GEMV's arithmetic on 32x32 MFMA tiles, so within
    the slab GEMV's bound (not the bf16 GEMM's); a second call is bitwise the first; x rows
    4-byte aligned only, x and y strided with sentinels in the padding; more than 8 vectors is
    Unsupported."""
    import torch

    say("gemm exact small-M", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=1800 + t + rows)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.random.default_rng(1801 + n_vec).standard_normal((n_vec, cols)).astype(np.float32)
    xs, ys = cols + 1, rows + 3  # x rows 4-byte aligned only
    xh = np.full((n_vec, xs), 777.0, np.float32)
    xh[:, :cols] = x
    y = torch.full((n_vec, ys), SENTINEL, dtype=torch.float32, device=dev)
    xd = to_dev(xh, dev)
    hl.gemv(t, slab, xd, y, rows, cols, n_vec, x_stride=xs, y_stride=ys, variant=hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
    yh = host(y)
    assert np.all(yh[:, rows:] == SENTINEL), "y padding overwritten"
    ref = oracle.matmul(t, dense, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, x)
    err = np.abs(yh[:, :rows].astype(np.float64) - ref)
    print(f"    exact small-M {NAMES[t]} M={n_vec}: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    hl.gemv(t, slab, xd, y, rows, cols, n_vec, x_stride=xs, y_stride=ys, variant=hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
    assert isclose_bits(host(y), yh), "a second call gave different bits"
    if n_vec == 8 and rows == 130:
        x9 = to_dev(np.ones((9, cols), np.float32), dev)
        with pytest.raises(hl.HaloError) as e:
            hl.gemv(t, slab, x9, torch.zeros((9, rows), dtype=torch.float32, device=dev), rows, cols, 9,
                    variant=hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
        assert e.value.code == hl.ErrorCode.Unsupported


@pytest.mark.parametrize("t", (Q4_K, Q6_K, Q5_K))
@pytest.mark.parametrize("n_vec", [2, 4, 8])
def test_gate_up_exact_small_m_variant(hl, oracle, dev, t, n_vec):
    """The fused gate/up pair on the exact small-M GEMM: gate and up each within the slab GEMV's
    bound, through the chunk reduce's SwiGLU (the fast SiLU's error added)."""
    import torch

    rows, cols = 576, 5120
    say("gate_up exact small-M", NAMES[t], n_vec)
    bg, _ = make_weights(t, rows, cols, seed=1900 + t)
    bu, _ = make_weights(t, rows, cols, seed=1950 + t)
    dg, du = dense_of(bg, t, rows, cols, row_bytes(t, cols), 0), dense_of(bu, t, rows, cols, row_bytes(t, cols), 0)
    sg, su = slab_of(hl, dev, t, dg, rows, cols), slab_of(hl, dev, t, du, rows, cols)
    x = np.random.default_rng(1901 + n_vec).standard_normal((n_vec, cols)).astype(np.float32)
    out = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)
    hl.gate_up_swiglu(t, sg, su, to_dev(x, dev), out, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
    g = oracle.matmul(t, dg, rows, cols, x)
    u = oracle.matmul(t, du, rows, cols, x)
    ref = oracle.swiglu(g, u)
    tol = swiglu_tol(g, u, slab_gemv_tol(oracle, t, dg, rows, cols, x), slab_gemv_tol(oracle, t, du, rows, cols, x), ref,
                     fast=True)
    err = np.abs(host(out).astype(np.float64) - ref)
    print(f"    gate_up exact small-M {NAMES[t]} M={n_vec}: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


# ---- split-K failure path and the stream's workspace ------------------------------------------


def test_split_k_timeout_is_reported_and_the_workspace_recovers(hl, oracle, dev):
    """Forced from the host: every split-K reduction waits for a tag no partial carries (a
    bounded wait of 64 rounds), gives up, writes NaN and marks the status word. The kernels
    exit normally; halo_mi_stream_check reports a Device error once, and the next call on the
    stream is correct again."""
    import torch

    t, rows, cols = Q4_K, 576, 5120  # 9 slabs: split over K, every slab has a reducer
    say("split-K forced timeout", rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=1700)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.random.default_rng(1701).standard_normal((1, cols)).astype(np.float32)
    xd = to_dev(x, dev)
    y = torch.full((1, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.stream_check()  # clean before
    try:
        hl.force_splitk_timeout(64, True)
        hl.gemv(t, slab, xd, y, rows, cols, 1, variant=hl.Variant.SLAB_GEMV)
    finally:
        hl.force_splitk_timeout(0, False)
    with pytest.raises(hl.HaloError) as e:
        hl.stream_check()
    assert e.value.code == hl.ErrorCode.Device
    assert np.all(np.isnan(host(y))), "a reduction that gave up must not write a plausible value"
    hl.stream_check()  # reported once
    hl.gemv(t, slab, xd, y, rows, cols, 1, variant=hl.Variant.SLAB_GEMV)
    hl.stream_check()
    ref = oracle.matmul(t, dense, rows, cols, x)
    assert np.all(np.abs(host(y).astype(np.float64) - ref) <= slab_gemv_tol(oracle, t, dense, rows, cols, x))


def test_fused_norm_split_k_timeout_is_reported_and_recovers(hl, oracle, dev):
    """The one-vector fused norm inside the GEMV (every workgroup computes 1 / rms itself) under a
    forced split-K timeout (the reductions wait for a tag no partial carries, 64 rounds): they
    give up, leave NaN and mark the status word; the kernels exit normally, halo_mi_stream_check
    reports a Device error once, and the next calls are bitwise the unfused RMS_NORM then GEMV."""
    import torch

    t, rows, cols = Q4_K, 1024, 5120  # 16 slabs x 8 K chunks: 128 workgroups
    say("fused norm forced timeout", rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=1750)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    rng = np.random.default_rng(1751)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    y = torch.full((1, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.stream_check()
    try:
        hl.force_splitk_timeout(64, True)
        hl.gemv(t, slab, xd, y, rows, cols, 1, variant=hl.Variant.SLAB_GEMV, norm_w=wd)
    finally:
        hl.force_splitk_timeout(0, False)
    with pytest.raises(hl.HaloError) as e:
        hl.stream_check()
    assert e.value.code == hl.ErrorCode.Device
    assert not np.all(np.isfinite(host(y))), "a wait that gave up must not leave only plausible values"
    hl.stream_check()  # reported once
    for _ in range(2):  # the launch state moved on: later calls are correct, twice in a row
        hl.gemv(t, slab, xd, y, rows, cols, 1, variant=hl.Variant.SLAB_GEMV, norm_w=wd)
        hl.stream_check()
        xn = torch.empty((1, cols), dtype=torch.float32, device=dev)
        hl.rms_norm(xd, wd, xn, 1, cols)
        y2 = torch.full((1, rows), SENTINEL, dtype=torch.float32, device=dev)
        hl.gemv(t, slab, xn, y2, rows, cols, 1, variant=hl.Variant.SLAB_GEMV)
        assert isclose_bits(host(y), host(y2)), "after the timeout the fused norm is not bitwise rms_norm then the gemv"


def test_stream_release_frees_and_reallocates(hl, oracle, dev):
    import torch

    t, rows, cols = Q6_K, 640, 5120
    say("stream release", rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=1800)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    x = np.random.default_rng(1801).standard_normal((2, cols)).astype(np.float32)
    s = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(s):
        for _ in range(2):
            y = torch.full((2, rows), SENTINEL, dtype=torch.float32, device=dev)
            hl.gemv(t, slab, to_dev(x, dev), y, rows, cols, 2)
            hl.stream_check()
            outs.append(host(y))
            free_before = torch.cuda.mem_get_info()[0]
            hl.stream_release()
            assert torch.cuda.mem_get_info()[0] >= free_before + (100 << 20), "the workspace was not freed"
    hl.stream_release(s.cuda_stream)  # releasing a stream without a workspace is a no-op
    assert isclose_bits(outs[0], outs[1])
    ref = oracle.matmul(t, dense, rows, cols, x)
    assert np.all(np.abs(outs[0].astype(np.float64) - ref) <= slab_gemv_tol(oracle, t, dense, rows, cols, x))


def test_stream_read_reads_and_writes_nothing(hl, dev):
    """The read-floor helper: runs for every unroll, leaves its sink untouched, refuses misaligned
    operands."""
    import torch

    buf = torch.arange(1 << 20, dtype=torch.int32, device=dev)
    sink = torch.zeros(64 * 256, dtype=torch.int32, device=dev)
    for unroll in (2, 4, 8, 16):
        hl.stream_read(buf, buf.numel() * 4, 64, unroll, sink)
    assert int(host(sink).astype(np.int64).sum()) == 0
    with pytest.raises(hl.HaloError) as e:
        hl.stream_read(buf.data_ptr() + 4, 1024, 64, 4, sink)
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:
        hl.stream_read(buf, 1024, 64, 3, sink)
    assert e.value.code == hl.ErrorCode.Kernel
