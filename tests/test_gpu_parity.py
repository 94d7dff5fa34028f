"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Mirrors the reference's GEMV/GEMM tests (tests/unit/hip/test_hip_gemv.cpp:31-323): random
valid blocks with a subnormal fp16 scale in every row, an unaligned row stride and start,
strided x / y views with sentinels in the padding, and acceptance either bitwise (the
reference-order variant, and every dequantized weight) or within a derived bound.
"""
import sys

import numpy as np
import pytest

from helpers import (ALL_TYPES, BLOCK, BF16, GGUF_TYPES, PLAIN_TYPES, F16, F32, IQ4_XS, NAMES, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANT_TYPES, U, depth_cpu, gemm_emulated, gemm_tol,
                     gemv_mag, isclose_bits, make_weights, max_ratio, row_bytes, silu64, slab_gemv_tol, swiglu_tol)

pytestmark = pytest.mark.gpu

SENTINEL = 999.0


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def to_dev(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def dense_of(buf, t, rows, cols, stride, offset):
    rb = row_bytes(t, cols)
    return np.concatenate([buf[offset + r * stride: offset + r * stride + rb] for r in range(rows)])


def slab_of(hl, dev, t, dense, rows, cols):
    """SLAB image built on the device from dense GGUF rows."""
    import torch

    src = to_dev(dense, dev)
    dst = torch.empty(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device=dev)
    hl.repack_slab(t, src, rows, cols, dst)
    return dst


def strided_xy(dev, x, rows, x_pad, y_pad):
    import torch

    n_vec, cols = x.shape
    xs, ys = cols + x_pad, rows + y_pad
    xh = np.full((n_vec, xs), 12345.0, np.float32)
    xh[:, :cols] = x
    xd = to_dev(xh, dev)
    yd = torch.full((n_vec, ys), SENTINEL, dtype=torch.float32, device=dev)
    return xd, xs, yd, ys


CASES = [
    # (rows, cols, n_vec, stride_pad, offset, x_pad, y_pad): test_hip_gemv.cpp:213-230 shapes
    (37, 512, 1, 0, 0, 0, 0),
    (13, 5120, 3, 3, 1, 5, 3),
]


# ---- dequantization is bit-exact --------------------------------------------------------


def test_bf16_dequant_every_pattern(hl, oracle, dev):
    """All 65536 bf16 patterns as one BF16 row, bitwise the reference's widening (the pattern is
    the top half of the fp32 one, quant.cpp:72-74), NaN payloads included."""
    import torch

    pats = np.arange(65536, dtype=np.uint16)
    ref = oracle.dequantize_row(BF16, pats.view(np.uint8), 65536)
    out = torch.empty((1, 65536), dtype=torch.float32, device=dev)
    hl.dequant_rows(BF16, hl.Layout.GGUF, to_dev(pats.view(np.uint8), dev), 1, 65536, out)
    assert np.array_equal(host(out)[0].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("case", CASES)
def test_dequant_gguf_and_slab_bitwise(hl, oracle, dev, t, case):
    import torch

    rows, cols, _, pad, off, _, _ = case
    say("dequant", NAMES[t], rows, cols, pad, off)
    buf, stride = make_weights(t, rows, cols, seed=rows + cols + t, stride_pad=pad, offset=off)
    ref = oracle.dequantize_rows(t, buf[off:], rows, cols, stride)
    wd = to_dev(buf, dev)
    out = torch.empty((rows, cols), dtype=torch.float32, device=dev)
    hl.dequant_rows(t, hl.Layout.GGUF, wd.data_ptr() + off, rows, cols, out, w_stride=stride)
    assert isclose_bits(host(out), ref), "GGUF dequant differs from tensor::dequantize_row"
    slab = slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, off), rows, cols)
    out2 = torch.full((rows, cols), -1.0, dtype=torch.float32, device=dev)
    hl.dequant_rows(t, hl.Layout.SLAB, slab, rows, cols, out2)
    assert isclose_bits(host(out2), ref), "SLAB dequant differs from tensor::dequantize_row"
    # a row range in the middle of a slab
    if rows > 5:
        part = torch.empty((3, cols), dtype=torch.float32, device=dev)
        hl.dequant_rows(t, hl.Layout.SLAB, slab, rows, cols, part, first_row=2, n_rows=3)
        assert isclose_bits(host(part), ref[2:5])


# ---- repack / unpack / upload -------------------------------------------------------------


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("pad,off", [(5, 3), (0, 0)])  # unaligned rows (byte path); 16-byte aligned rows
def test_repack_device_equals_host_and_unpacks(hl, dev, t, pad, off):
    import torch

    rows, cols = 70, 768 if BLOCK[t][0] == 256 else 544
    say("repack", NAMES[t], rows, cols, pad, off)
    buf, stride = make_weights(t, rows, cols, seed=5 + t, stride_pad=pad, offset=off)
    dense = dense_of(buf, t, rows, cols, stride, off)
    host_slab = hl.repack_slab_host(t, dense, rows, cols)
    wd = to_dev(buf, dev)
    slab = torch.full((hl.slab_bytes(t, rows, cols),), 0xAB, dtype=torch.uint8, device=dev)
    hl.repack_slab(t, wd.data_ptr() + off, rows, cols, slab, src_stride=stride)
    assert np.array_equal(host(slab), host_slab)
    back = torch.zeros(rows * row_bytes(t, cols), dtype=torch.uint8, device=dev)
    hl.unpack_slab(t, slab, rows, cols, back)
    assert np.array_equal(host(back), dense)
    up = torch.zeros_like(slab)
    hl.upload_slab(t, buf[off:], rows, cols, up, src_stride=stride, chunk_bytes=row_bytes(t, cols) * 64)
    assert np.array_equal(host(up), host_slab)


# ---- GEMV -------------------------------------------------------------------------------


def run_gemv(hl, dev, t, w, layout, x, rows, cols, variant, x_pad=0, y_pad=0, w_stride=0):
    xd, xs, yd, ys = strided_xy(dev, x, rows, x_pad, y_pad)
    hl.gemv(t, w, xd, yd, rows, cols, x.shape[0], layout=layout, w_stride=w_stride, x_stride=xs, y_stride=ys,
            variant=variant)
    y = host(yd)
    assert np.all(y[:, rows:] == SENTINEL), "y padding overwritten"
    return y[:, :rows]


def matrix_case(t, case):
    """test_hip_gemv.cpp:219-227's two shapes for type t: plain types (F32, F16, BF16) take 100
    columns in the first (a dot tail of 100 % 8) and a 4-byte row stride pad and offset in the
    second; block types 512 columns, then a 3-byte pad and 1-byte offset."""
    rows, cols, n_vec, pad, off, xp, yp = case
    if t in PLAIN_TYPES:
        cols = 100 if rows == 37 else cols
        pad, off = (4, 4) if pad else (0, 0)
    return rows, cols, n_vec, pad, off, xp, yp


@pytest.mark.parametrize("t", GGUF_TYPES)
@pytest.mark.parametrize("case", CASES)
def test_dequant_gguf_type_matrix_bitwise(hl, oracle, dev, t, case):
    """GGUF-layout dequantization of every type of the reference's HIP test matrix, and of the
    rest of its dequantizer's dispatch (BF16, Q4_1, Q5_0, Q5_1, Q2_K), is bitwise
    tensor::dequantize_row, at an unaligned row stride and start."""
    import torch

    rows, cols, _, pad, off, _, _ = matrix_case(t, case)
    say("dequant gguf", NAMES[t], rows, cols, pad, off)
    buf, stride = make_weights(t, rows, cols, seed=300 + rows + t, stride_pad=pad, offset=off)
    ref = oracle.dequantize_rows(t, buf[off:], rows, cols, stride)
    wd = to_dev(buf, dev)
    out = torch.full((rows, cols), SENTINEL, dtype=torch.float32, device=dev)
    hl.dequant_rows(t, hl.Layout.GGUF, wd.data_ptr() + off, rows, cols, out, w_stride=stride)
    assert isclose_bits(host(out), ref), "GGUF dequant differs from tensor::dequantize_row"


@pytest.mark.parametrize("t", GGUF_TYPES)
@pytest.mark.parametrize("case", CASES)
def test_gemv_gguf_ref_bitwise(hl, oracle, dev, t, case):
    """The reference-order variant over GGUF rows is bitwise cpu::matmul for every type the
    reference dequantizes; on the GGUF layout the default variant is that kernel."""
    rows, cols, n_vec, pad, off, xp, yp = matrix_case(t, case)
    say("gemv_gguf_ref", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=100 + t + rows, stride_pad=pad, offset=off)
    x = np.random.default_rng(1000 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    ref = oracle.matmul(t, buf[off:], rows, cols, x, w_stride=stride)
    wd = to_dev(buf, dev)
    y = run_gemv(hl, dev, t, wd.data_ptr() + off, hl.Layout.GGUF, x, rows, cols, hl.Variant.GGUF_REF, xp, yp, stride)
    assert isclose_bits(y, ref), "reference-order gemv is not bitwise cpu::matmul"
    y0 = run_gemv(hl, dev, t, wd.data_ptr() + off, hl.Layout.GGUF, x, rows, cols, hl.Variant.DEFAULT, xp, yp, stride)
    assert isclose_bits(y0, ref), "the GGUF layout's default variant is not the reference-order kernel"


def test_f16_dequant_every_pattern(hl, oracle, dev):
    """All 65536 fp16 patterns as one F16 row: bitwise the reference's widening for every
    pattern that is not a NaN; a NaN stays a NaN of the same sign (the payload of a signalling
    NaN may be quieted differently by the device conversion)."""
    import torch

    pats = np.arange(65536, dtype=np.uint16)
    ref = oracle.dequantize_row(F16, pats.view(np.uint8), 65536)
    out = torch.empty((1, 65536), dtype=torch.float32, device=dev)
    hl.dequant_rows(F16, hl.Layout.GGUF, to_dev(pats.view(np.uint8), dev), 1, 65536, out)
    y = host(out)[0]
    nan = np.isnan(ref)
    assert np.array_equal(y[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(y[nan])) and np.array_equal(np.signbit(y[nan]), np.signbit(ref[nan]))
    print(f"    NaN patterns with the reference's exact bits: {int(np.sum(y[nan].view(np.uint32) == ref[nan].view(np.uint32)))}"
          f" of {int(nan.sum())}")


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("case", CASES + [(130, 1024, 4, 0, 0, 1, 2), (64, 256, 6, 0, 0, 0, 0)])
def test_gemv_slab_within_bound(hl, oracle, dev, t, case):
    rows, cols, n_vec, pad, off, xp, yp = case
    say("gemv_slab", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=200 + t + rows, stride_pad=pad, offset=off)
    dense = dense_of(buf, t, rows, cols, stride, off)
    x = np.random.default_rng(2000 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    ref = oracle.matmul(t, dense, rows, cols, x)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.SLAB_GEMV, xp, yp)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    slab gemv {NAMES[t]} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


def extreme_x(n_vec: int, cols: int, seed: int) -> np.ndarray:
    """x rows 2^-40, 1 and 2^40 times N(0, 1), each 256-column group scaled by its own 2^k
    (|k| <= 20), one whole group and a few scattered elements exactly zero: the slab GEMV scales
    each group's x by a power of two before its three-piece split, and rows of very different
    magnitude share one launch."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_vec, cols))
    x *= np.ldexp(1.0, np.array([-40, 0, 40, -20][:n_vec]))[:, None]
    ng = cols // 256
    x *= np.repeat(np.ldexp(1.0, rng.integers(-20, 21, (n_vec, ng))), 256, axis=1)
    x[:, 256 * (ng // 2): 256 * (ng // 2 + 1)] = 0.0
    x[rng.random((n_vec, cols)) < 0.01] = 0.0
    return x.astype(np.float32)


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("rows,cols", [(576, 5120), (17408, 5120)])
@pytest.mark.parametrize("variant", ["SLAB_GEMV", "SLAB_GEMM_EXACT_INVARIANT"])
def test_gemv_slab_extreme_magnitudes(hl, oracle, dev, t, rows, cols, variant):
    """The two batch-invariant kernels (the slab GEMV: the chunked split at 576 rows, the even
    split at 17408 except Q6_K; the exact GEMM with its fixed K split) with extreme_x's rows:
    within the slab GEMV's derived bound of cpu::matmul for every row, and every row of the
    three-vector call bitwise its one-vector call."""
    v = getattr(hl.Variant, variant)
    say("extreme x", variant, NAMES[t], rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=2600 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = extreme_x(3, cols, 2700 + t)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, v)
    ref = oracle.matmul(t, dense, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    extreme x {variant} {NAMES[t]} {rows}x{cols} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(np.isfinite(y)) and np.all(err <= tol)
    for i in range(3):
        y1 = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x[i:i + 1], rows, cols, v)
        assert isclose_bits(y1, y[i:i + 1]), f"row {i} depends on the batch"


INVARIANT_VARIANTS = ("SLAB_GEMV", "SLAB_GEMM_EXACT_INVARIANT")


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("rows,cols", [(130, 1024), (576, 5120)])
@pytest.mark.parametrize("variant", INVARIANT_VARIANTS)
def test_gemv_slab_rows_do_not_depend_on_the_batch(hl, oracle, dev, t, rows, cols, variant):
    """GemvArgs::allow_gemm == false (include/halo/backend/backend.h:298-302): every row of a
    batched call is bitwise the row of an n_vec == 1 call, whatever n_vec (the slab GEMV; the
    exact GEMM with its K split fixed by the shape, in passes of 8 past 8 vectors). Every row is
    within the slab GEMV's bound of cpu::matmul."""
    v = getattr(hl.Variant, variant)
    say("batch invariance", variant, NAMES[t], rows, cols)
    buf, stride = make_weights(t, rows, cols, seed=250 + t + rows)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    n = 12
    x = np.random.default_rng(2500 + t).standard_normal((n, cols)).astype(np.float32)
    singles = np.stack([run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x[i:i + 1], rows, cols, v, 0, 0)[0]
                        for i in range(n)])
    ref = oracle.matmul(t, dense, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, dense, rows, cols, x)
    err = np.abs(singles.astype(np.float64) - ref)
    print(f"    {variant} {NAMES[t]} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    for n_vec in (2, 3, 4, 5, 8, 9, 12):
        y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x[:n_vec], rows, cols, v, 1, 2)
        assert isclose_bits(y, singles[:n_vec]), f"n_vec={n_vec} changed a row"


@pytest.mark.parametrize("t,rows,cols,pair", [(Q4_K, 17408, 5120, False), (Q4_K, 17408, 5120, True),
                                               (Q6_K, 5120, 17408, False), (Q6_K, 151936, 5120, False)])
@pytest.mark.parametrize("variant", INVARIANT_VARIANTS)
def test_gemv_rows_do_not_depend_on_the_batch_at_baseline_shapes(hl, dev, t, rows, cols, pair, variant):
    """The same invariance at the BASELINE shapes, where the K split and the waves per chunk are
    largest (the gate/up pair streams two matrices; 151936 rows takes the multi-group kernel;
    there the exact GEMM's fixed split does not fit the workspace and variant 9 runs the slab
    GEMV, bitwise variant 2)."""
    import torch

    say("gemv batch invariance", variant, NAMES[t], rows, cols, "pair" if pair else "")
    v = getattr(hl.Variant, variant)
    if rows == 151936:
        _, slab = head_weights(hl, dev)
    else:
        slab = slab_of(hl, dev, t, synth(hl, t, rows, cols, 90 + rows), rows, cols)
    slab_u = slab_of(hl, dev, t, synth(hl, t, rows, cols, 91 + rows), rows, cols) if pair else None
    x = np.random.default_rng(9000 + rows).standard_normal((9, cols)).astype(np.float32)
    xd = to_dev(x, dev)

    def run(n0, n):
        y = torch.full((n, rows), SENTINEL, dtype=torch.float32, device=dev)
        xv = xd[n0:n0 + n]
        if pair:
            hl.gate_up_swiglu(t, slab, slab_u, xv, y, rows, cols, n, variant=v)
        else:
            hl.gemv(t, slab, xv, y, rows, cols, n, variant=v)
        return host(y)

    singles = np.concatenate([run(i, 1) for i in range(9)])
    for n_vec in (2, 3, 4, 5, 8, 9):
        assert isclose_bits(run(0, n_vec), singles[:n_vec]), f"n_vec={n_vec} changed a row"
    if rows == 151936 and v == hl.Variant.SLAB_GEMM_EXACT_INVARIANT:
        y2 = torch.full((2, rows), SENTINEL, dtype=torch.float32, device=dev)
        hl.gemv(t, slab, xd[:2], y2, rows, cols, 2, variant=hl.Variant.SLAB_GEMV)
        assert isclose_bits(host(y2), singles[:2]), "variant 9 on a shape past its split is not variant 2"


@pytest.mark.parametrize("t", (Q4_K, Q6_K))
def test_gemv_split_k_state_is_clean_between_calls(hl, oracle, dev, t):
    """Split-K calls of different shapes share the stream's workspace (arrival counters and
    partial words). A call after calls of other shapes (other chunk counts over the same
    counters and words) must give the same bits as the first call, within the bound."""
    shapes = [(576, 5120, 1), (640, 17408, 1), (576, 5120, 4), (130, 1024, 3), (576, 5120, 1)]
    mats = {}
    for rows, cols, _ in shapes:
        if (rows, cols) not in mats:
            buf, stride = make_weights(t, rows, cols, seed=700 + rows)
            dense = dense_of(buf, t, rows, cols, stride, 0)
            mats[(rows, cols)] = (dense, slab_of(hl, dev, t, dense, rows, cols))
    outs = []
    for i, (rows, cols, n_vec) in enumerate(shapes):
        say("gemv split-K state", NAMES[t], rows, cols, n_vec)
        dense, slab = mats[(rows, cols)]
        x = np.random.default_rng(7000 + cols + n_vec).standard_normal((n_vec, cols)).astype(np.float32)
        y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.SLAB_GEMV, 0, 0)
        ref = oracle.matmul(t, dense, rows, cols, x)
        assert np.all(np.abs(y.astype(np.float64) - ref) <= slab_gemv_tol(oracle, t, dense, rows, cols, x)), shapes[i]
        outs.append(y)
    assert isclose_bits(outs[0], outs[-1]), "a later call of the same shape gave different bits"


# ---- GEMM (bf16 MFMA) ---------------------------------------------------------------------


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("case", [(37, 5120, 17, 0, 0, 5, 3), (16, 256, 2, 0, 0, 0, 0), (33, 768, 40, 0, 0, 0, 0),
                                  (130, 1024, 130, 0, 0, 4, 1),
                                  (130, 1024, 300, 0, 0, 4, 1), (200, 768, 600, 0, 0, 0, 0)])
@pytest.mark.parametrize("variant", [3, 5])  # M tiles of 64..256 rows (k_gemm_pc) / 512 rows (k_gemm_lm)
def test_gemm_bf16_within_bounds(hl, oracle, dev, t, case, variant):
    rows, cols, n_vec, pad, off, xp, yp = case
    say("gemm_bf16", NAMES[t], rows, cols, n_vec, variant)
    buf, stride = make_weights(t, rows, cols, seed=300 + t + rows, stride_pad=pad, offset=off)
    dense = dense_of(buf, t, rows, cols, stride, off)
    x = np.random.default_rng(3000 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    ref = oracle.matmul(t, dense, rows, cols, x)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    if xp % 4:
        xp += 4 - xp % 4  # the MFMA path wants 16-byte aligned x rows
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, variant, xp, yp)
    err = np.abs(y.astype(np.float64) - ref)
    tol = gemm_tol(oracle, t, dense, rows, cols, x)
    print(f"    gemm vs cpu: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    emu, etol = gemm_emulated(oracle, t, dense, rows, cols, x)
    eerr = np.abs(y.astype(np.float64) - emu)
    print(f"    gemm vs bf16-exact products: worst |d|/bound = {max_ratio(eerr, etol):.4f}")
    assert np.all(eerr <= etol)


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("case", [(37, 5120, 17, 0, 0, 5, 3), (130, 1024, 9, 0, 0, 4, 1), (200, 768, 32, 0, 0, 0, 0),
                                  (64, 256, 12, 0, 0, 0, 0), (130, 1024, 40, 0, 0, 4, 1), (37, 768, 64, 0, 0, 0, 0)])
def test_gemm_small_m_within_bounds(hl, oracle, dev, t, case):
    """The auto variant at 9..32 x rows runs the small-M GEMM (k_gemm_sm: every wave dequantizes
    its own MFMA B fragments, no LDS; K chunks added in order by the reduce), at 40 and 64 rows
    the 64-row tiles of k_gemm_pc: the same bf16
    bounds as the other GEMM tile families, against the CPU and the bf16-exact products, and a
    second call is bitwise the first."""
    rows, cols, n_vec, pad, off, xp, yp = case
    say("gemm_small_m", NAMES[t], rows, cols, n_vec)
    buf, stride = make_weights(t, rows, cols, seed=320 + t + rows, stride_pad=pad, offset=off)
    dense = dense_of(buf, t, rows, cols, stride, off)
    x = np.random.default_rng(3200 + t + n_vec).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    ref = oracle.matmul(t, dense, rows, cols, x)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    if xp % 4:
        xp += 4 - xp % 4
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, 4, xp, yp)
    err = np.abs(y.astype(np.float64) - ref)
    tol = gemm_tol(oracle, t, dense, rows, cols, x)
    print(f"    gemm vs cpu: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    emu, etol = gemm_emulated(oracle, t, dense, rows, cols, x)
    eerr = np.abs(y.astype(np.float64) - emu)
    print(f"    gemm vs bf16-exact products: worst |d|/bound = {max_ratio(eerr, etol):.4f}")
    assert np.all(eerr <= etol)
    y2 = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, 4, xp, yp)
    assert isclose_bits(y2, y), "a second small-M GEMM call gave different bits"


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("pair", [False, True])
@pytest.mark.parametrize("kind", ["one", "many"])
def test_gemm_m512_partial_round(hl, oracle, dev, t, pair, kind):
    """512-row tiles that do not fill whole rounds of the GPU: the W units past the last whole
    round run as 128-row tiles split over K (k_gemm_lm with one x block per wave) whose partials
    are reduced in chunk order. one: one unit more than a round (300 x rows); many: 3000 x rows
    in 6 M tiles over 50 units (8 units remain). Checked against the oracle on the first rows
    and on the last 256 rows (the remaining units) for the plain GEMM and for the gate/up pair."""
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    cols = 512  # 16 slots: split tiles take two K chunks
    n_vec, units = (300, cus + 1) if kind == "one" else (3000, 50)
    rows = 64 * units * (1 if pair else 2)
    say("gemm m512 partial round", kind, NAMES[t], rows, cols, n_vec, "pair" if pair else "plain")
    rb = row_bytes(t, cols)
    x = np.random.default_rng(8000 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    xd = to_dev(x, dev)
    wa = synth(hl, t, rows, cols, 80 + t)
    sa = slab_of(hl, dev, t, wa, rows, cols)
    out = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    if pair:
        wb = synth(hl, t, rows, cols, 90 + t)
        sb = slab_of(hl, dev, t, wb, rows, cols)
        hl.gate_up_swiglu(t, sa, sb, xd, out, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMM_BF16_M512)
    else:
        hl.gemv(t, sa, xd, out, rows, cols, n_vec, variant=hl.Variant.SLAB_GEMM_BF16_M512)
    y = host(out)
    for r0, r1 in ((0, 128), (rows - 256, rows)):
        n = r1 - r0
        pa = wa[r0 * rb:r1 * rb]
        ga = oracle.matmul(t, pa, n, cols, x)
        ta = gemm_tol(oracle, t, pa, n, cols, x)
        ea, eta = gemm_emulated(oracle, t, pa, n, cols, x)
        if pair:
            pb = wb[r0 * rb:r1 * rb]
            ub = oracle.matmul(t, pb, n, cols, x)
            ref = oracle.gate_up_swiglu(t, pa, pb, n, cols, x)
            tol = swiglu_tol(ga, ub, ta, gemm_tol(oracle, t, pb, n, cols, x), ref, fast=True)
            eb, etb = gemm_emulated(oracle, t, pb, n, cols, x)
            refe = silu64(ea) * eb
            tole = swiglu_tol(ea, eb, eta, etb, refe, fast=True)
        else:
            ref, tol = ga, ta
            refe, tole = ea, eta
        err = np.abs(y[:, r0:r1].astype(np.float64) - ref)
        print(f"    rows [{r0}, {r1}): worst |d|/bound = {max_ratio(err, tol):.4f}")
        assert np.all(err <= tol)
        # the split tiles' K chunks and their reduce, held to the bf16-exact products' bound
        erre = np.abs(y[:, r0:r1].astype(np.float64) - refe)
        print(f"    rows [{r0}, {r1}) vs bf16-exact products: worst |d|/bound = {max_ratio(erre, tole):.4f}")
        assert np.all(erre <= tole)


# ---- fused gate/up + SwiGLU ---------------------------------------------------------------


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("n_vec,variant", [(1, 2), (2, 2), (4, 2), (5, 2), (8, 3), (17, 3), (300, 3), (17, 5), (300, 5),
                                           (600, 5), (5, 4), (8, 4), (17, 4), (32, 4), (48, 4), (64, 4)])
def test_gate_up_swiglu(hl, oracle, dev, t, n_vec, variant):
    import torch

    rows, cols = 96, 1024
    say("gate_up", NAMES[t], rows, cols, n_vec, variant)
    bg, sg = make_weights(t, rows, cols, seed=400 + t)
    bu, su = make_weights(t, rows, cols, seed=500 + t)
    dg, du = dense_of(bg, t, rows, cols, sg, 0), dense_of(bu, t, rows, cols, su, 0)
    x = np.random.default_rng(4000 + n_vec).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    ref = oracle.gate_up_swiglu(t, dg, du, rows, cols, x)
    g = oracle.matmul(t, dg, rows, cols, x)
    u = oracle.matmul(t, du, rows, cols, x)
    sgd, sud = slab_of(hl, dev, t, dg, rows, cols), slab_of(hl, dev, t, du, rows, cols)
    out = torch.full((n_vec, rows), SENTINEL, dtype=torch.float32, device=dev)
    hl.gate_up_swiglu(t, sgd, sud, to_dev(x, dev), out, rows, cols, n_vec, variant=variant)
    y = host(out)
    gemv = variant == hl.Variant.SLAB_GEMV
    if gemv:
        tg, tu = slab_gemv_tol(oracle, t, dg, rows, cols, x), slab_gemv_tol(oracle, t, du, rows, cols, x)
    else:
        tg, tu = gemm_tol(oracle, t, dg, rows, cols, x), gemm_tol(oracle, t, du, rows, cols, x)
    tol = swiglu_tol(g, u, tg, tu, ref, fast=not gemv)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    gate_up worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


# ---- host validation: error codes (test_hip_gemv.cpp:285-323) -------------------------------


def test_gemv_rejects_bad_arguments(hl, dev):
    import torch

    w = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    x = torch.zeros(128, dtype=torch.float32, device=dev)
    y = torch.zeros(64, dtype=torch.float32, device=dev)

    def code(**kw):
        args = dict(t=Q8_0, w=w, x=x, y=y, rows=2, cols=128, n_vec=1, layout=hl.Layout.GGUF, variant=0)
        args.update(kw)
        t = args.pop("t")
        try:
            hl.gemv(t, args.pop("w"), args.pop("x"), args.pop("y"), args.pop("rows"), args.pop("cols"),
                    args.pop("n_vec"), **args)
        except hl.HaloError as e:
            return e.code, str(e)
        return None, ""

    assert code()[0] is None  # valid baseline
    assert code(t=9)[0] == hl.ErrorCode.Unsupported  # Q8_1: no dequantizer in the reference either
    c, msg = code(cols=100)
    assert c == hl.ErrorCode.Kernel and "multiple of the block size 32" in msg
    c, msg = code(y=w.data_ptr() + 16)
    assert c == hl.ErrorCode.Kernel and "y overlaps w" in msg
    assert code(variant=10)[0] == hl.ErrorCode.Config  # past the last id
    assert code(variant=hl.Variant.SLAB_GEMV)[0] == hl.ErrorCode.Config  # GGUF bytes, SLAB kernel
    c, msg = code(t=F32, cols=64, w=w.data_ptr() + 2)
    assert c == hl.ErrorCode.Kernel and "4-byte aligned" in msg
    c, msg = code(layout=hl.Layout.SLAB, w_stride=300)
    assert c == hl.ErrorCode.Kernel
    c, msg = code(n_vec=2, x_stride=64)
    assert c == hl.ErrorCode.Kernel and "x row stride" in msg
    torch.cuda.synchronize()


# ---- BASELINE shapes (full size) ------------------------------------------------------------


def synth(hl, t, rows, cols, seed, outliers=0.0):
    from helpers import synth_matrix

    return synth_matrix(hl, t, rows, cols, seed, outlier_cols=outliers)


@pytest.mark.parametrize("t,rows,cols,seed,outliers", [
    (Q4_K, 17408, 5120, 2, 0.0),     # config 2: FFN gate/up shape
    (Q6_K, 5120, 17408, 3, 0.0),     # config 3: ffn_down
    (Q4_0, 4096, 4096, 0, 0.0),      # config 1
    (Q5_K, 17408, 5120, 6, 0.0),     # the UD pack's other formats at the gate/up shape
    (IQ4_XS, 17408, 5120, 7, 0.0),
])
@pytest.mark.parametrize("n_vec", [1, 4])
def test_baseline_shapes_gemv(hl, oracle, dev, t, rows, cols, seed, outliers, n_vec):
    say("baseline gemv", NAMES[t], rows, cols, n_vec)
    wq = synth(hl, t, rows, cols, seed, outliers)
    x = hl.fill_normal(seed + 1000, n_vec * cols).reshape(n_vec, cols)
    ref = oracle.matmul(t, wq, rows, cols, x)
    slab = slab_of(hl, dev, t, wq, rows, cols)
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.DEFAULT)
    tol = slab_gemv_tol(oracle, t, wq, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    {NAMES[t]} {rows}x{cols} M={n_vec}: worst |d|/bound = {max_ratio(err, tol):.4f}, "
          f"max rel err = {float(np.max(err / (np.abs(ref) + 1e-6))):.2e}")
    assert np.all(err <= tol)


_TWO_WAVE = {}


@pytest.mark.parametrize("n_vec", [1, 3])
@pytest.mark.parametrize("t", QUANT_TYPES)
def test_exact_small_m_two_wave_form(hl, oracle, dev, t, n_vec):
    """The exact small-M kernel's two-wave form (two waves per slab on alternate super-blocks,
    the odd wave's sums added to the even wave's through LDS). A plain 17408 x 5120 matrix at
    1-4 vectors runs as 68 workgroups (two units each) x 4 K chunks of 5 super-blocks, which
    takes it; every format, one and two vectors per lane half, within the slab GEMV's bound,
    and a second call bitwise the first."""
    rows, cols = 17408, 5120
    say("exact small-M two-wave form", NAMES[t], rows, cols, n_vec)
    if _TWO_WAVE.get("t") != t:  # one format's matrix serves both vector counts
        _TWO_WAVE.clear()
        wq = synth(hl, t, rows, cols, 40 + t)
        _TWO_WAVE.update(t=t, w=(wq, slab_of(hl, dev, t, wq, rows, cols)))
    wq, slab = _TWO_WAVE["w"]
    x = hl.fill_normal(4000 + n_vec, n_vec * cols).reshape(n_vec, cols)
    ref = oracle.matmul(t, wq, rows, cols, x)
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
    tol = slab_gemv_tol(oracle, t, wq, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    two-wave {NAMES[t]} M={n_vec}: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    y2 = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.SLAB_GEMM_EXACT_SMALL_M)
    assert isclose_bits(y2, y), "a second call gave different bits"


_HEAD = {}


def head_weights(hl, dev):
    """config 3b's head (151936 x 5120 Q6_K, 1% of the columns x8), quantized and uploaded once."""
    if "w" not in _HEAD:
        t, rows, cols = Q6_K, 151936, 5120
        wq = synth(hl, t, rows, cols, 3, 0.01)
        _HEAD["w"] = (wq, slab_of(hl, dev, t, wq, rows, cols))
    return _HEAD["w"]


@pytest.mark.parametrize("n_vec", [1, 2, 3, 4])
def test_baseline_q6_k_head(hl, oracle, dev, n_vec):
    """config 3b: 151936 x 5120 Q6_K with 1% of the columns scaled x8, M = 1..4, whole output."""
    t, rows, cols = Q6_K, 151936, 5120
    say("baseline head", rows, cols, n_vec)
    wq, slab = head_weights(hl, dev)
    x = hl.fill_normal(1003 + n_vec, n_vec * cols).reshape(n_vec, cols)
    ref = oracle.matmul(t, wq, rows, cols, x)
    y = run_gemv(hl, dev, t, slab, hl.Layout.SLAB, x, rows, cols, hl.Variant.DEFAULT)
    tol = slab_gemv_tol(oracle, t, wq, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    head M={n_vec} worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)


GATE_UP_GEMV_MAX = 2  # the gate/up auto choice: the GEMV pair up to 2 vectors, the exact small-M GEMM at 3..4
GATE_UP_EXACT_MAX = 4  # (kGateUpGemvMax), then the bf16 GEMM


@pytest.mark.parametrize("n_vec", [2, 3, 4, 8, 12, 20, 24, 64, 512])
def test_baseline_gate_up(hl, oracle, dev, n_vec):
    """config 4: fused gate/up pair over two 17408 x 5120 Q4_K matrices (and config 5's FFN pair
    at M = 4); the oracle checks every output. 12, 20 and 24 vectors take the small-M GEMM's
    12- and 24-row tiers, whose K chunks at this shape span several super-block groups."""
    import torch

    t, rows, cols = Q4_K, 17408, 5120
    say("baseline gate_up", n_vec)
    wg = synth(hl, t, rows, cols, 4)
    wu = synth(hl, t, rows, cols, 44)
    x = hl.fill_normal(1004, n_vec * cols).reshape(n_vec, cols)
    rb = row_bytes(t, cols)
    out = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)
    sg, su, xd = slab_of(hl, dev, t, wg, rows, cols), slab_of(hl, dev, t, wu, rows, cols), to_dev(x, dev)
    hl.gate_up_swiglu(t, sg, su, xd, out, rows, cols, n_vec)
    yall = host(out)
    # the split-K partial sums are added in a fixed order: a second call is bitwise identical
    hl.gate_up_swiglu(t, sg, su, xd, out, rows, cols, n_vec)
    assert isclose_bits(host(out), yall), "gate/up result changed between two identical calls"
    for c0, c1 in ((0, rows),):
        n = c1 - c0
        wg_c, wu_c = wg[c0 * rb:c1 * rb], wu[c0 * rb:c1 * rb]
        g = oracle.matmul(t, wg_c, n, cols, x)
        u = oracle.matmul(t, wu_c, n, cols, x)
        ref = oracle.swiglu(g, u)  # oracle.gate_up_swiglu's composition (pinned in test_oracle)
        y = yall[:, c0:c1]
        exact = n_vec <= GATE_UP_EXACT_MAX  # the GEMV pair or the exact small-M GEMM: the GEMV's bound
        if exact:
            tg = slab_gemv_tol(oracle, t, wg_c, n, cols, x)
            tu = slab_gemv_tol(oracle, t, wu_c, n, cols, x)
        else:
            tg = gemm_tol(oracle, t, wg_c, n, cols, x)
            tu = gemm_tol(oracle, t, wu_c, n, cols, x)
        # the GEMV pair's SiLU is the IEEE form, the GEMMs' the fast one
        tol = swiglu_tol(g, u, tg, tu, ref, fast=n_vec > GATE_UP_GEMV_MAX)
        err = np.abs(y.astype(np.float64) - ref)
        print(f"    gate_up M={n_vec} columns [{c0}, {c1}): worst |d|/bound = {max_ratio(err, tol):.4f}, "
              f"max |d| = {float(err.max()):.3e}, max |ref| = {float(np.abs(ref).max()):.3e}")
        assert np.all(err <= tol)
        if not exact:
            # the bf16 GEMM against the fp64 products of its own bf16-rounded operands: only the
            # fp32 accumulation's error is allowed ((K/32 + 42) u sum |x~||w~|), which a dropped
            # or repeated sub-block, a wrong tile or a lost K chunk would exceed many times over
            ge, gte = gemm_emulated(oracle, t, wg_c, n, cols, x)
            ue, ute = gemm_emulated(oracle, t, wu_c, n, cols, x)
            refe = silu64(ge) * ue
            tole = swiglu_tol(ge, ue, gte, ute, refe, fast=True)
            erre = np.abs(y.astype(np.float64) - refe)
            print(f"    gate_up M={n_vec} vs bf16-exact products: worst |d|/bound = {max_ratio(erre, tole):.4f}")
            assert np.all(erre <= tole)
    assert np.all(np.isfinite(host(out)))


# config 5: the hybrid layer's projections (the FFN pair is test_baseline_gate_up)
@pytest.mark.parametrize("name,t,rows,cols", [
    ("gdn_in", Q4_K, 12288, 5120), ("gdn_out", Q4_K, 5120, 6144), ("q", Q4_K, 6144, 5120),
    ("k", Q4_K, 1024, 5120), ("v", Q6_K, 1024, 5120), ("down", Q6_K, 5120, 17408)])
@pytest.mark.parametrize("n_vec", [1, 4, 512])
def test_baseline_hybrid_layer_shapes(hl, oracle, dev, name, t, rows, cols, n_vec):
    """Each projection of the config-5 layer at M = 1 and 4 (GEMV) and M = 512 (bf16 GEMM, the
    default for more than 8 vectors), every output checked."""
    import torch

    say("hybrid layer", name, NAMES[t], rows, cols, n_vec)
    wq = synth(hl, t, rows, cols, 500 + rows + cols)
    slab = slab_of(hl, dev, t, wq, rows, cols)
    x = hl.fill_normal(600 + n_vec, n_vec * cols).reshape(n_vec, cols)
    y = torch.empty((n_vec, rows), dtype=torch.float32, device=dev)
    hl.gemv(t, slab, to_dev(x, dev), y, rows, cols, n_vec)
    yh = host(y)
    ref = oracle.matmul(t, wq, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, wq, rows, cols, x) if n_vec <= 8 else gemm_tol(oracle, t, wq, rows, cols, x)
    err = np.abs(yh.astype(np.float64) - ref)
    print(f"    {name} M={n_vec}: worst |d|/bound = {max_ratio(err, tol):.4f}")
    assert np.all(err <= tol)
    if n_vec > 8:  # the bf16 GEMM: also against the fp64 products of its bf16-rounded operands
        emu, etol = gemm_emulated(oracle, t, wq, rows, cols, x)
        eerr = np.abs(yh.astype(np.float64) - emu)
        print(f"    {name} M={n_vec} vs bf16-exact products: worst |d|/bound = {max_ratio(eerr, etol):.4f}")
        assert np.all(eerr <= etol)
