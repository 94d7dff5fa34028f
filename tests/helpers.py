"""Shared test data builders and error bounds."""
from __future__ import annotations

import math

import numpy as np

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_XS, F32 = 2, 8, 12, 13, 14, 23, 0
F16, Q3_K, IQ4_NL, IQ3_S = 1, 11, 20, 21
Q4_1, Q5_0, Q5_1, Q2_K, BF16 = 3, 6, 7, 10, 30
QUANT_TYPES = (Q4_K, Q6_K, Q8_0, Q4_0, Q5_K, IQ4_XS)
SLAB_TYPES = QUANT_TYPES  # the types with a SLAB layout
# the reference's HIP GEMV test matrix, in its order (tests/unit/hip/test_hip_gemv.cpp:217-218)
ALL_TYPES = (Q4_K, Q5_K, Q6_K, Q8_0, F16, F32, IQ4_XS, IQ4_NL, Q3_K, IQ3_S, Q4_0)
# the rest of the reference dequantizer's dispatch (src/tensor/quant.cpp:386-407): GGUF layout only
GGUF_EXTRA_TYPES = (BF16, Q4_1, Q5_0, Q5_1, Q2_K)
GGUF_TYPES = ALL_TYPES + GGUF_EXTRA_TYPES
PLAIN_TYPES = (F32, F16, BF16)  # one element per block
NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K",
         IQ4_NL: "IQ4_NL", IQ3_S: "IQ3_S", IQ4_XS: "IQ4_XS", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1", Q2_K: "Q2_K",
         BF16: "BF16"}
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q3_K: (256, 110), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210), IQ4_NL: (32, 18), IQ3_S: (256, 110), IQ4_XS: (256, 136),
         Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q2_K: (256, 84), BF16: (1, 2)}
U = 2.0 ** -24  # fp32 unit roundoff


def row_bytes(t: int, cols: int) -> int:
    be, bb = BLOCK[t]
    assert cols % be == 0
    return cols // be * bb


def _put16(buf: np.ndarray, at: int, v: float) -> None:
    h = np.array([v], dtype=np.float16).view(np.uint16)[0]
    buf[at] = h & 0xFF
    buf[at + 1] = h >> 8


def make_weights(t: int, rows: int, cols: int, seed: int, stride_pad: int = 0, offset: int = 0):
    """Random valid weight bytes in the GGUF layout: random quants and finite fp16 scales, with
    one fp16-subnormal scale per row (the recipe of the reference's GEMV tests,
    tests/unit/hip/test_hip_gemv.cpp:43-104). Returns (buffer, row_stride)."""
    rng = np.random.default_rng(seed)
    rb = row_bytes(t, cols)
    stride = rb + stride_pad
    buf = rng.integers(0, 256, size=offset + (rows - 1) * stride + rb + 7, dtype=np.uint8)
    be, bb = BLOCK[t]
    for n in range(rows):
        row = offset + n * stride
        if t == F32:
            vals = rng.uniform(-1, 1, cols).astype(np.float32)
            vals[3 % cols] = np.float32(1e-40)  # one fp32 subnormal
            buf[row:row + 4 * cols] = vals.view(np.uint8)
            continue
        if t == F16:
            vals = rng.uniform(-1, 1, cols).astype(np.float16)
            vals[3 % cols] = np.float16(3e-7)  # one fp16 subnormal
            buf[row:row + 2 * cols] = vals.view(np.uint8)
            continue
        if t == BF16:
            vals = (rng.uniform(-1, 1, cols).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
            vals[3 % cols] = 0x0042  # one bf16 subnormal
            buf[row:row + 2 * cols] = vals.view(np.uint8)
            continue
        for b in range(cols // be):
            sc = 2e-6 if b == 0 else rng.uniform(-0.05, 0.05)
            if t in (Q4_0, Q8_0, IQ4_NL, IQ3_S, Q5_0):
                _put16(buf, row + bb * b, sc)
            elif t in (Q4_1, Q5_1):
                _put16(buf, row + bb * b, sc)
                _put16(buf, row + bb * b + 2, rng.uniform(-0.05, 0.05))
            elif t == Q2_K:
                _put16(buf, row + bb * b + 80, sc)
                _put16(buf, row + bb * b + 82, abs(rng.uniform(-0.05, 0.05)))
            elif t == Q3_K:
                _put16(buf, row + bb * b + 108, sc)
            elif t in (Q4_K, Q5_K):
                _put16(buf, row + bb * b, 4e-6 if b == 0 else sc)
                _put16(buf, row + bb * b + 2, abs(rng.uniform(-0.05, 0.05)))
            elif t == Q6_K:
                _put16(buf, row + bb * b + 208, 1e-6 if b == 0 else sc)
            elif t == IQ4_XS:
                _put16(buf, row + bb * b, 3e-6 if b == 0 else sc)
    return buf, stride


def dense_rows(buf: np.ndarray, t: int, rows: int, cols: int, stride: int, offset: int) -> np.ndarray:
    """The rows packed densely (row_bytes apart)."""
    rb = row_bytes(t, cols)
    return np.concatenate([buf[offset + r * stride: offset + r * stride + rb] for r in range(rows)])


def synth_matrix(hl, t: int, rows: int, cols: int, seed: int, std: float = 0.02, outlier_cols: float = 0.0):
    """BASELINE-style weights: N(0, std) from the portable generator, optionally with a fraction
    of columns scaled x8, quantized by this repo's quantizer. Returns GGUF bytes (numpy)."""
    w = hl.fill_normal(seed, rows * cols, 0.0, std).reshape(rows, cols)
    if outlier_cols:
        k = max(1, int(round(cols * outlier_cols)))
        cols_idx = np.random.default_rng(seed + 7).choice(cols, size=k, replace=False)
        w[:, cols_idx] *= 8.0
    return hl.quantize(t, w.reshape(-1))


def gemv_mag(oracle, t: int, wbytes: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    """sum_i |x_i| (|a_i| + |b_i| + 2 |off_i|) per output: the magnitude that bounds the rounding
    error of both the CPU dot and the SLAB kernels' factored sums (w = a - b; off = the offset
    the kernels take out of the quant, see oracle_dequant_terms)."""
    ax = np.abs(np.asarray(x, np.float64).reshape(-1, cols))
    if t == F32:
        w = wbytes.view(np.float32).reshape(rows, cols).astype(np.float64)
        return ax @ np.abs(w).T
    rb = row_bytes(t, cols)
    out = np.empty((ax.shape[0], rows), np.float64)
    step = 4096  # rows per chunk: bounds the host memory of the full-size cases
    for r0 in range(0, rows, step):
        n = min(step, rows - r0)
        a, b, off = oracle.dequant_terms(t, wbytes[r0 * rb:(r0 + n) * rb], n, cols)
        m = np.abs(a.astype(np.float64)) + np.abs(b.astype(np.float64)) + 2 * np.abs(off.astype(np.float64))
        out[:, r0:r0 + n] = ax @ m.T
    return out


def depth_cpu(cols: int) -> int:
    """Longest addition chain of cpu::detail::dot (backends/cpu/kernel_common.h:16-27)."""
    return cols // 8 + 3 + cols % 8 + 1


def depth_slab_gemv(cols: int) -> int:
    """Upper bound on the SLAB GEMV's longest chain: 16-term slot halves, the slot sums of one
    wave (at most cols/32), up to 16 wave partials, 16-term x half-sums, and the combines."""
    return cols // 32 + 16 + 16 + 16 + 16


def depth_gemm(cols: int) -> int:
    """MFMA accumulation: cols/32 steps of a 32-product dot each."""
    return cols // 32 + 32 + 8


def slab_gemv_tol(oracle, t, wbytes, rows, cols, x):
    mag = gemv_mag(oracle, t, wbytes, rows, cols, x)
    return (depth_cpu(cols) + depth_slab_gemv(cols) + 4) * U * mag * (1 + 1e-3) + 1e-30


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 to bf16 (nearest even), returned as fp32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def gemm_tol(oracle, t, wbytes, rows, cols, x):
    """bf16 GEMM vs the fp32 CPU reference: x and w each rounded to bf16 (relative error
    <= 2^-9 each, products exact in fp32), plus both summation errors."""
    w = oracle.dequantize_rows(t, wbytes, rows, cols).astype(np.float64)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w).T
    return (2.0 ** -8 + 2.0 ** -18 + (depth_cpu(cols) + depth_gemm(cols) + 2) * U) * mag * (1 + 1e-3) + 1e-30


def gemm_emulated(oracle, t, wbytes, rows, cols, x):
    """fp64 product of the bf16-rounded operands (the GEMM's exact-product reference), and the
    bound on the GEMM's own fp32 accumulation against it."""
    w = bf16_round(oracle.dequantize_rows(t, wbytes, rows, cols)).astype(np.float64)
    xb = bf16_round(x).astype(np.float64)
    ref = xb @ w.T
    tol = (depth_gemm(cols) + 2) * U * (np.abs(xb) @ np.abs(w).T) + 1e-30
    return ref, tol


def silu64(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def swiglu_tol(g, u, dg, du, out, fast=False):
    """|silu(g) u - silu(g') u'| for |g - g'| <= dg, |u - u'| <= du, plus the epilogue's own
    rounding (exp, divide, multiply; a few ulp). silu' is bounded by 1.1 everywhere.
    fast: the GEMM epilogues' SiLU on v_exp_f32 / v_rcp_f32, relative error at most
    (1.5 |g'| + 8) 2^-24 on silu(g'), taken at the worst g' within dg."""
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    tol = 1.1 * dg * (np.abs(u) + du) + (np.abs(silu64(g)) + 1.1 * dg) * du + 16 * U * np.abs(out) + 1e-30
    if fast:
        tol = tol + (1.5 * (np.abs(g) + dg) + 8) * U * (np.abs(silu64(g)) + 1.1 * dg) * (np.abs(u) + du)
    return tol


def max_ratio(err, tol) -> float:
    return float(np.max(np.asarray(err) / np.asarray(tol))) if np.size(err) else 0.0


def fmt_case(**kw) -> str:
    return " ".join(f"{k}={v}" for k, v in kw.items())


def isclose_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Bitwise equality of fp32 arrays (NaN payloads included)."""
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


__all__ = [n for n in dir() if not n.startswith("_")] + ["math"]
