"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path.

Every check here is independent of the oracle's own formulas: known-answer blocks from the
reference's tests, literal decodings of the block formats, a library routine (numpy's fp16
widening), closed forms, brute force in fp64, and invariants of cpu::matmul.
"""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

from helpers import F32, IQ4_XS, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, U, depth_cpu


def f16_bytes(v: float) -> bytes:
    return np.array([v], dtype=np.float16).tobytes()


# ---- fp16 -> fp32 (include/halo/tensor/fp16.h:19-37) -------------------------------------


def fp16_ldexp(h: int) -> float:
    """Independent definition (tests/unit/tensor/test_fp16.cpp:17-30 of the reference)."""
    sign = -1.0 if h >> 15 else 1.0
    exp = (h >> 10) & 0x1F
    mant = h & 0x3FF
    if exp == 0:
        return sign * math.ldexp(mant, -24)
    if exp == 31:
        return sign * math.inf if mant == 0 else math.nan
    return sign * math.ldexp(mant | 0x400, exp - 25)


def test_fp16_all_patterns_widen_exactly(oracle):
    lib = oracle.lib()
    got = np.array([lib.oracle_fp16_to_fp32(h) for h in range(65536)], dtype=np.float32)
    npy = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    for h in range(65536):
        ref = fp16_ldexp(h)
        if math.isnan(ref):
            assert math.isnan(got[h]) and (np.signbit(got[h]) == bool(h >> 15)), hex(h)
        else:
            assert float(got[h]) == ref and np.signbit(got[h]) == bool(h >> 15), hex(h)
    # numpy's widening is exact too: identical bits except NaN payload quieting
    nan = np.isnan(npy)
    assert np.array_equal(got[~nan].view(np.uint32), npy[~nan].view(np.uint32))
    # NaN: sign and payload kept, quiet bit set
    for h in (0x7C01, 0xFC01, 0x7E00, 0x7D55):
        bits = struct.unpack("<I", struct.pack("<f", got[h]))[0]
        assert bits == ((h & 0x8000) << 16) | 0x7F800000 | ((h & 0x3FF) << 13) | 0x400000


# ---- geometry (src/tensor/dtype.cpp:19-51, tests/unit/tensor/test_dequant.cpp:37-50) --------


def test_row_bytes_geometry_and_checks(oracle):
    assert oracle.row_bytes(F32, 5120) == 20480
    assert oracle.row_bytes(Q6_K, 5120) == 20 * 210
    assert oracle.row_bytes(Q4_0, 5120) == 160 * 18
    assert oracle.row_bytes(Q4_K, 5120) == 2880
    assert oracle.row_bytes(Q6_K, 17408) == 14280
    assert oracle.row_bytes(Q8_0, 0) == 0
    with pytest.raises(oracle.OracleError) as e:
        oracle.row_bytes(Q4_K, 100)
    assert e.value.code == oracle.EMODEL
    with pytest.raises(oracle.OracleError) as e:
        oracle.row_bytes(F32, -1)
    assert e.value.code == oracle.EMODEL
    with pytest.raises(oracle.OracleError) as e:
        oracle.row_bytes(5, 32)  # removed ggml id: refused, not a crash
    assert e.value.code == oracle.EUNSUPPORTED


# ---- known-answer blocks ----------------------------------------------------------------


def test_q8_0_hand_built_block(oracle):
    """tests/unit/tensor/test_dequant.cpp:52-59."""
    blk = f16_bytes(0.5) + bytes((j - 16) & 0xFF for j in range(32))
    y = oracle.dequantize_row(Q8_0, np.frombuffer(blk, np.uint8), 32)
    assert np.array_equal(y, np.array([0.5 * (j - 16) for j in range(32)], np.float32))


def test_q4_0_hand_built_block_nibble_order(oracle):
    """tests/unit/tensor/test_dequant.cpp:61-72: low nibbles -> 0..15, high -> 16..31."""
    blk = f16_bytes(2.0) + bytes(((15 - j) << 4) | j for j in range(16))
    y = oracle.dequantize_row(Q4_0, np.frombuffer(blk, np.uint8), 32)
    for j in range(16):
        assert y[j] == 2.0 * (j - 8)
        assert y[j + 16] == 2.0 * (7 - j)


# Literal 6-bit (scale, min) decodings of one 12-byte Q4_K scales field, worked out by hand
# from the ggml packing (bytes 0-3: sc[0..3] + top bits of sc[4..7]; bytes 4-7: m[0..3] + top
# bits of m[4..7]; bytes 8-11: low nibbles of sc[4..7] | m[4..7]).
Q4K_SCALES = bytes([0x41, 0x02, 0x83, 0xC4, 0x05, 0x46, 0x87, 0xC8, 0x9A, 0xBC, 0xDE, 0xF1])
Q4K_SC_M = [(1, 5), (2, 6), (3, 7), (4, 8), (26, 9), (12, 27), (46, 45), (49, 63)]


def q4k_block(d: float, dmin: float, scales: bytes, qs: bytes) -> np.ndarray:
    assert len(scales) == 12 and len(qs) == 128
    return np.frombuffer(f16_bytes(d) + f16_bytes(dmin) + scales + qs, np.uint8)


def test_q4_k_literal_scale_min_table(oracle):
    # quant bytes: group g byte l holds q_lo = l % 16 and q_hi = 15 - l % 16
    qs = bytes(((15 - l % 16) << 4) | (l % 16) for g in range(4) for l in range(32))
    y = oracle.dequantize_row(Q4_K, q4k_block(1.0, 0.5, Q4K_SCALES, qs), 256)
    for e in range(256):
        g, hi, l = e // 64, (e % 64) // 32, e % 32
        sc, m = Q4K_SC_M[2 * g + hi]
        q = (15 - l % 16) if hi else (l % 16)
        assert y[e] == np.float32(sc * q - 0.5 * m), e


@pytest.mark.parametrize("j", range(8))
def test_q4_k_single_subblock_scale(oracle, j):
    """Only sub-block j has sc = 1 (d = 1, dmin = 0, all quants 15): exactly its 32 elements
    are 15, every other element is 0."""
    s = bytearray(12)
    if j < 4:
        s[j] = 1
    else:
        s[j + 4] = 1
    y = oracle.dequantize_row(Q4_K, q4k_block(1.0, 0.0, bytes(s), bytes([0xFF] * 128)), 256)
    exp = np.zeros(256, np.float32)
    exp[32 * j: 32 * j + 32] = 15.0
    assert np.array_equal(y, exp)


@pytest.mark.parametrize("j", range(8))
def test_q4_k_single_subblock_min_high_bits(oracle, j):
    """m[j] = 63 (for j >= 4 its top two bits live in byte j), d = 0, dmin = 1: sub-block j is
    -63, the rest 0."""
    s = bytearray(12)
    if j < 4:
        s[j + 4] = 63
    else:
        s[j] = 0xC0  # top bits of m[j] -> byte j (= j - 4 + 4)
        s[j + 4] = 0xF0  # low nibble of m[j] in the high half of byte j + 4
    y = oracle.dequantize_row(Q4_K, q4k_block(0.0, 1.0, bytes(s), bytes(128)), 256)
    exp = np.zeros(256, np.float32)
    exp[32 * j: 32 * j + 32] = -63.0
    assert np.array_equal(y, -np.abs(y)) and np.array_equal(y, exp)


def q6k_block(ql: bytes, qh: bytes, sc: bytes, d: float) -> np.ndarray:
    return np.frombuffer(ql + qh + sc + f16_bytes(d), np.uint8)


def test_q6_k_extremes(oracle):
    ones = bytes([1] * 16)
    y = oracle.dequantize_row(Q6_K, q6k_block(bytes(128), bytes(64), ones, 1.0), 256)
    assert np.all(y == -32.0)  # q = 0 -> -32
    y = oracle.dequantize_row(Q6_K, q6k_block(bytes([0xFF] * 128), bytes([0xFF] * 64), ones, 1.0), 256)
    assert np.all(y == 31.0)  # q = 63 -> +31


def test_q6_k_high_bit_quarters_and_nibble_halves(oracle):
    """qh byte 0b11100100 gives quarter k the top bits k; ql low nibble 5 serves quarters 0-1,
    high nibble 9 quarters 2-3: element value 16 k + nibble - 32 (d = 1, all scales 1)."""
    ones = bytes([1] * 16)
    y = oracle.dequantize_row(Q6_K, q6k_block(bytes([0x95] * 128), bytes([0b11100100] * 64), ones, 1.0), 256)
    for e in range(256):
        k = (e % 128) // 32
        nib = 5 if k < 2 else 9
        assert y[e] == 16 * k + nib - 32, e


def test_q6_k_scale_index_map(oracle):
    """Scales sc[i] = i + 1; q = 33 everywhere (value sc * 1): element e of half n, quarter k,
    lane l uses scale 8 n + l // 16 + 2 k (16 weights per scale, in the order of the format)."""
    sc = bytes(range(1, 17))
    # q = 33 = 0b100001: low nibble 1, top bits 2
    y = oracle.dequantize_row(Q6_K, q6k_block(bytes([0x11] * 128), bytes([0b10101010] * 64), sc, 1.0), 256)
    expect = []
    for n in range(2):
        for k in range(4):
            for l in range(32):
                expect.append(8 * n + l // 16 + 2 * k + 1)
    assert np.array_equal(y, np.array(expect, np.float32))


def test_q6_k_negative_scale_and_fp16_subnormal_d(oracle):
    d = 2.0 ** -20  # fp16 subnormal
    sc = bytes([0x80] * 16)  # int8 -128
    y = oracle.dequantize_row(Q6_K, q6k_block(bytes([0xFF] * 128), bytes([0xFF] * 64), sc, d), 256)
    assert np.all(y == np.float32(d * -128 * 31))


def q5k_block(d: float, dmin: float, scales: bytes, qh: bytes, qs: bytes) -> np.ndarray:
    assert len(scales) == 12 and len(qh) == 32 and len(qs) == 128
    return np.frombuffer(f16_bytes(d) + f16_bytes(dmin) + scales + qh + qs, np.uint8)


def test_q5_k_geometry(oracle):
    """block_q5_K {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} = 176 bytes per 256."""
    assert oracle.row_bytes(Q5_K, 5120) == 20 * (2 + 2 + 12 + 32 + 128)
    assert oracle.row_bytes(IQ4_XS, 5120) == 20 * (2 + 2 + 4 + 128)


def test_q5_k_literal_scale_min_table_without_high_bits(oracle):
    """qh = 0: Q5_K is Q4_K with its quants 48 bytes in (same 12-byte scales field)."""
    qs = bytes(((15 - l % 16) << 4) | (l % 16) for g in range(4) for l in range(32))
    y = oracle.dequantize_row(Q5_K, q5k_block(1.0, 0.5, Q4K_SCALES, bytes(32), qs), 256)
    for e in range(256):
        g, hi, l = e // 64, (e % 64) // 32, e % 32
        sc, m = Q4K_SC_M[2 * g + hi]
        q = (15 - l % 16) if hi else (l % 16)
        assert y[e] == np.float32(sc * q - 0.5 * m), e


@pytest.mark.parametrize("bit", range(8))
def test_q5_k_high_bit_selects_one_subblock(oracle, bit):
    """Only bit `bit` of every qh byte set, all nibbles 0, d = 1, dmin = 0, every sc = 1: the
    32 elements of sub-block `bit` (group bit // 2, nibble half bit % 2) are 16, the rest 0."""
    ones = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])  # sc[0..7] = 1, m[0..7] = 0
    y = oracle.dequantize_row(Q5_K, q5k_block(1.0, 0.0, ones, bytes([1 << bit] * 32), bytes(128)), 256)
    exp = np.zeros(256, np.float32)
    exp[32 * bit: 32 * bit + 32] = 16.0
    assert np.array_equal(y, exp)


def test_q5_k_high_bit_per_lane(oracle):
    """qh[l] = 0xFF for even l only, all nibbles 15, sc = 1, m = 1, d = 2, dmin = 0.25: element
    (sub-block j, lane l) is 2 (15 + 16 [l even]) - 0.25."""
    ones = bytes([1, 1, 1, 1, 1, 1, 1, 1, 0x11, 0x11, 0x11, 0x11])
    qh = bytes(0xFF if l % 2 == 0 else 0 for l in range(32))
    y = oracle.dequantize_row(Q5_K, q5k_block(2.0, 0.25, ones, qh, bytes([0xFF] * 128)), 256)
    for e in range(256):
        l = e % 32
        assert y[e] == np.float32(2 * (15 + (16 if l % 2 == 0 else 0)) - 0.25), e


IQ4NL = json.loads((Path(__file__).resolve().parent / "golden" / "iq4nl_table.json").read_text())["kvalues_iq4nl"]


def iq4xs_block(d: float, scales_h: int, scales_l: bytes, qs: bytes) -> np.ndarray:
    assert len(scales_l) == 4 and len(qs) == 128
    return np.frombuffer(f16_bytes(d) + struct.pack("<H", scales_h) + scales_l + qs, np.uint8)


def test_iq4_xs_table_and_nibble_order(oracle):
    """ls = 33 everywhere (low nibble 1, high bits 2 -> 1 + 32), d = 1: dl = 1, element j of a
    sub-block is table[low nibble of qs[j]], element j + 16 table[high nibble]; the table is the
    reference's kvalues_iq4nl (golden fixture)."""
    qs = bytes(((15 - j) << 4) | j for ib in range(8) for j in range(16))
    y = oracle.dequantize_row(IQ4_XS, iq4xs_block(1.0, 0xAAAA, bytes([0x11] * 4), qs), 256)
    for ib in range(8):
        for j in range(16):
            assert y[32 * ib + j] == IQ4NL[j]
            assert y[32 * ib + j + 16] == IQ4NL[15 - j]


def test_iq4_xs_six_bit_scales(oracle):
    """Sub-block ib has ls = (nibble ib of scales_l) | (bits 2ib..2ib+1 of scales_h) << 4 and
    multiplier d (ls - 32); every code 8 (table value 1): element value d (ls - 32)."""
    ls = [0, 63, 32, 17, 48, 5, 60, 33]
    sl = bytes((ls[2 * i] & 15) | ((ls[2 * i + 1] & 15) << 4) for i in range(4))
    sh = sum((v >> 4) << (2 * ib) for ib, v in enumerate(ls))
    y = oracle.dequantize_row(IQ4_XS, iq4xs_block(0.5, sh, sl, bytes([0x88] * 128)), 256)
    for ib in range(8):
        assert np.all(y[32 * ib: 32 * ib + 32] == np.float32(0.5 * (ls[ib] - 32) * IQ4NL[8])), ib


def test_q5_k_and_iq4_xs_dequant_terms(oracle):
    """a - b reproduces the dequantized weight bit for bit; Q5_K has no offset (its codes are
    non-negative), IQ4_XS's is 128 dl with dl the sub-block multiplier d (ls - 32)."""
    rng = np.random.default_rng(5)
    for t, bb in ((Q5_K, 176), (IQ4_XS, 136)):
        w = rng.integers(0, 256, size=4 * bb, dtype=np.uint8)
        for b in range(4):
            w[bb * b: bb * b + 2] = np.frombuffer(f16_bytes(rng.uniform(-0.05, 0.05)), np.uint8)
            if t == Q5_K:
                w[bb * b + 2: bb * b + 4] = np.frombuffer(f16_bytes(rng.uniform(0, 0.05)), np.uint8)
        a, b_, off = oracle.dequant_terms(t, w, 1, 1024)
        y = oracle.dequantize_row(t, w, 1024)
        assert np.array_equal((a - b_).astype(np.float32)[0], y)
        if t == Q5_K:
            assert np.all(off == 0)
            continue
        assert np.all(b_ == 0)
        for b in range(4):
            blk = w[bb * b: bb * (b + 1)]
            d = np.float32(np.frombuffer(blk[0:2].tobytes(), np.float16)[0])
            sh = int(blk[2]) | int(blk[3]) << 8
            for ib in range(8):
                ls = ((int(blk[4 + ib // 2]) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
                dl = np.float32(d * np.float32(ls - 32))
                seg = slice(256 * b + 32 * ib, 256 * b + 32 * ib + 32)
                assert np.all(off[0, seg] == np.float32(128) * dl)


def _f16(blk, i):
    return np.float32(np.frombuffer(bytes(blk[i:i + 2]), np.float16)[0])


def _random_blocks(rng, t, bb, n):
    """n blocks of random bytes with finite fp16 scales (the d / dmin words)."""
    w = rng.integers(0, 256, size=n * bb, dtype=np.uint8)
    for b in range(n):
        base = bb * b + (208 if t == Q6_K else 0)
        w[base: base + 2] = np.frombuffer(f16_bytes(rng.uniform(-0.05, 0.05)), np.uint8)
        if t in (Q4_K, Q5_K):
            w[bb * b + 2: bb * b + 4] = np.frombuffer(f16_bytes(rng.uniform(0, 0.05)), np.uint8)
    # an fp16-subnormal scale in the first block
    w[(208 if t == Q6_K else 0): (208 if t == Q6_K else 0) + 2] = np.frombuffer(bytes([0x07, 0x00]), np.uint8)
    return w


@pytest.mark.parametrize("t,bb,be", [(Q4_0, 18, 32), (Q8_0, 34, 32)])
def test_q4_0_q8_0_dequant_terms(oracle, t, bb, be):
    """Q4_0: w = q d - 8 d, so off = 8 d (quant.cpp:79-90); Q8_0: codes are read as unsigned
    bytes by the kernels, so off = 128 d (quant.cpp:143-151). a is the dequantized weight,
    b = 0. With every code at its lowest value (nibble 0 / int8 -128), w = -off exactly."""
    rng = np.random.default_rng(11)
    n = 8
    w = _random_blocks(rng, t, bb, n)
    a, b_, off = oracle.dequant_terms(t, w, 1, n * be)
    y = oracle.dequantize_row(t, w, n * be)
    assert np.array_equal((a - b_).astype(np.float32)[0], y)
    assert np.all(b_ == 0)
    k = 8 if t == Q4_0 else 128
    for b in range(n):
        d = _f16(w[bb * b: bb * (b + 1)], 0)
        assert np.all(off[0, be * b: be * (b + 1)] == np.float32(k) * d), b
    low = w.copy()
    for b in range(n):
        low[bb * b + 2: bb * (b + 1)] = 0x00 if t == Q4_0 else 0x80
    a2, b2, off2 = oracle.dequant_terms(t, low, 1, n * be)
    y2 = oracle.dequantize_row(t, low, n * be)
    assert isbits(off2[0], -y2) and isbits(a2[0], y2)


def _k4_scale_min(s: bytes, j: int):
    """ggml's get_scale_min_k4 written from the 12-byte layout: 6-bit (sc, m) pairs, the first
    four whole in bytes 0..3 / 4..7, the last four split into low nibbles of bytes 8..11 and
    the top two bits of bytes 0..7."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def test_q4_k_dequant_terms(oracle):
    """Q4_K: a = (d sc) q, b = dmin m, off = 0 (quant.cpp:247-269); recomputed here from the
    block bytes with an independent reading of the scale/min table."""
    rng = np.random.default_rng(12)
    n = 6
    w = _random_blocks(rng, Q4_K, 144, n)
    a, b_, off = oracle.dequant_terms(Q4_K, w, 1, n * 256)
    y = oracle.dequantize_row(Q4_K, w, n * 256)
    assert np.array_equal((a - b_).astype(np.float32)[0], y)
    assert np.all(off == 0)
    for b in range(n):
        blk = bytes(w[144 * b: 144 * (b + 1)])
        d, dmin = _f16(blk, 0), _f16(blk, 2)
        for e in range(256):
            g, hi, l = e // 64, (e % 64) // 32, e % 32
            sc, m = _k4_scale_min(blk[4:16], 2 * g + hi)
            byte = blk[16 + 32 * g + l]
            q = (byte >> 4) if hi else (byte & 15)
            assert a[0, 256 * b + e] == np.float32(np.float32(d * np.float32(sc)) * np.float32(q)), (b, e)
            assert b_[0, 256 * b + e] == np.float32(dmin * np.float32(m)), (b, e)


def test_q6_k_dequant_terms(oracle):
    """Q6_K: a is the dequantized weight, b = 0, off = 32 (d sc) with sc the int8 scale of the
    element's 16-weight sub-block (quant.cpp:302-327). Every code 0 gives w = -32 (d sc), so
    off = -w exactly there; on random blocks off is constant over each 16-weight run and is 32
    times one of the block's 16 products d sc."""
    rng = np.random.default_rng(13)
    n = 5
    w = _random_blocks(rng, Q6_K, 210, n)
    a, b_, off = oracle.dequant_terms(Q6_K, w, 1, n * 256)
    y = oracle.dequantize_row(Q6_K, w, n * 256)
    assert np.array_equal((a - b_).astype(np.float32)[0], y)
    assert np.all(b_ == 0)
    for b in range(n):
        blk = w[210 * b: 210 * (b + 1)]
        d = _f16(blk, 208)
        allowed = {float(np.float32(32) * np.float32(d * np.float32(s))) for s in blk[192:208].view(np.int8)}
        ob = off[0, 256 * b: 256 * (b + 1)].reshape(16, 16)
        assert np.all(ob == ob[:, :1])
        assert {float(v) for v in ob[:, 0]} <= allowed
    zero = w.copy()
    for b in range(n):
        zero[210 * b: 210 * b + 192] = 0
    a2, _, off2 = oracle.dequant_terms(Q6_K, zero, 1, n * 256)
    y2 = oracle.dequantize_row(Q6_K, zero, n * 256)
    assert isbits(off2[0], -y2) and isbits(a2[0], y2)
    # one scale per sub-block: scale s_j alone non-zero moves exactly the 16 weights of run j
    for j in range(16):
        one = zero[:210].copy()
        one[192:208] = 0
        one[192 + j] = 3
        _, _, o1 = oracle.dequant_terms(Q6_K, one, 1, 256)
        nz = np.nonzero(o1[0])[0]
        y1 = oracle.dequantize_row(Q6_K, one, 256)
        assert np.array_equal(nz, np.nonzero(y1)[0]) and len(nz) == 16, j


def isbits(a, b) -> bool:
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32),
                          np.ascontiguousarray(b, np.float32).view(np.uint32))


# ---- the canonical pack's remaining types: F16, IQ4_NL, Q3_K, IQ3_S ---------------------------
# (quant.cpp:68-70, :154-165, :196-233, :350-384; the reference's HIP test matrix,
# tests/unit/hip/test_hip_gemv.cpp:217-218)

F16, Q3_K, IQ4_NL, IQ3_S = 1, 11, 20, 21
_TABLES = json.loads((Path(__file__).resolve().parent / "golden" / "iq3s_tables.json").read_text())
IQ3S_GRID = _TABLES["iq3s_grid"]
KMASK = _TABLES["kmask_iq2xs"]
_INC = Path(__file__).resolve().parents[1] / "halo_amd" / "csrc" / "iq3s_grid.inc"


def test_iq3s_codebook_include_is_the_reference_table():
    """The one codebook source of the device decoder and the oracle equals the reference's
    iq3s_grid entry for entry (fixture read from src/tensor/ggml_tables.h as data), and the sign
    masks are the single bits 1 << j."""
    import re

    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]{8})u", _INC.read_text())]
    assert vals == IQ3S_GRID
    assert KMASK == [1 << j for j in range(8)]


def test_new_type_geometry(oracle):
    """dtype.cpp:20, :29, :39-40 and test_dequant.cpp:41's literal."""
    assert oracle.row_bytes(IQ4_NL, 17408) == 544 * 18
    assert oracle.row_bytes(F16, 100) == 200  # one element per block: any length
    assert oracle.row_bytes(Q3_K, 5120) == 20 * 110
    assert oracle.row_bytes(IQ3_S, 5120) == 20 * 110
    for t, n in ((Q3_K, 100), (IQ3_S, 128), (IQ4_NL, 16)):
        with pytest.raises(oracle.OracleError) as e:
            oracle.row_bytes(t, n)
        assert e.value.code == oracle.EMODEL


def test_f16_rows_widen_every_pattern(oracle):
    """An F16 row is its elements widened one by one (quant.cpp:68-70): every one of the 65536
    patterns equals the pinned fp16 widening bitwise (NaN included)."""
    pats = np.arange(65536, dtype=np.uint16)
    y = oracle.dequantize_row(F16, pats.view(np.uint8), 65536)
    lib = oracle.lib()
    want = np.array([lib.oracle_fp16_to_fp32(int(h)) for h in pats], np.float32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def iq4nl_block(d_bits: int, qs: bytes) -> np.ndarray:
    return np.frombuffer(struct.pack("<H", d_bits) + qs, np.uint8)


def test_iq4_nl_table_nibble_order_and_subnormal_scale(oracle):
    """Element j < 16 is table[low nibble of qs[j]], j + 16 table[high nibble], times d; d = 2
    and d = 2^-24 (the smallest fp16 subnormal, 0x0001) give exact multiples of the table."""
    qs = bytes(((15 - j) << 4) | j for j in range(16))
    for d_bits, d in ((0x4000, 2.0), (0x0001, 2.0 ** -24)):
        y = oracle.dequantize_row(IQ4_NL, iq4nl_block(d_bits, qs), 32)
        for j in range(16):
            assert y[j] == np.float32(d * IQ4NL[j])
            assert y[j + 16] == np.float32(d * IQ4NL[15 - j])


def q3k_block(hmask: bytes, qs: bytes, scales: bytes, d: float) -> np.ndarray:
    assert len(hmask) == 32 and len(qs) == 64 and len(scales) == 12
    return np.frombuffer(hmask + qs + scales + f16_bytes(d), np.uint8)


def test_q3_k_literal_six_bit_scales(oracle):
    """Bytes 0..7 of the scales = 0x21 (low nibble 1, high 2), bytes 8..11 = 0xE4 (2-bit fields
    0, 1, 2, 3): the 16 scales are 1, 1, 1, 1, 17, 17, 17, 17, 34, 34, 34, 34, 50, 50, 50, 50.
    With every 2-bit code 1 and every high bit set (q = 1), element e's value is d (sc - 32) for
    the scale of its 16-element run e // 16."""
    sc = [1] * 4 + [17] * 4 + [34] * 4 + [50] * 4
    y = oracle.dequantize_row(Q3_K, q3k_block(b"\xff" * 32, b"\x55" * 64, b"\x21" * 8 + b"\xe4" * 4, 0.5), 256)
    # runs of 16 in element order take scales 0, 1, ..., 15 (is++ in quant.cpp:219-224)
    for e in range(256):
        assert y[e] == np.float32(0.5 * (sc[e // 16] - 32)), e


def test_q3_k_codes_and_high_bit(oracle):
    """Scale bytes 0..7 = 0x11 and 8..11 = 0xAA (every 2-bit field 2): all 16 scales are
    1 | 32 = 33, so dl = d. qs bytes 0xE4 hold the codes 0, 1, 2, 3 at shifts 0, 2, 4, 6, so
    element 128 n + 32 j + l has code j; with its hmask bit clear the value drops by 4. Only
    hmask[5]'s bit 6 is set: half 1, shift pair 2, lane 5 (element 128 + 64 + 5)."""
    hm = bytearray(32)
    hm[5] = 1 << 6
    y = oracle.dequantize_row(Q3_K, q3k_block(bytes(hm), b"\xe4" * 64, bytes([0x11] * 8 + [0xAA] * 4), 1.0), 256)
    for e in range(256):
        j = (e % 128) // 32
        code = j - (0 if e == 128 + 64 + 5 else 4)
        assert y[e] == np.float32(code), e


def _q3k_walk(blk: bytes) -> np.ndarray:
    """quant.cpp:196-233's loops walked literally: the 32-bit aux shuffle with kmask1/kmask2,
    then 2 halves x 4 shifts x 2 runs of 16, moving q by 32 per half and the hmask bit per
    shift."""
    d = float(np.frombuffer(blk[108:110], np.float16)[0])
    aux = list(struct.unpack("<3I", blk[96:108])) + [0]
    km1, km2 = 0x03030303, 0x0F0F0F0F
    tmp = aux[2]
    aux[2] = ((aux[0] >> 4) & km2) | (((tmp >> 4) & km1) << 4)
    aux[3] = ((aux[1] >> 4) & km2) | (((tmp >> 6) & km1) << 4)
    aux[0] = (aux[0] & km2) | (((tmp >> 0) & km1) << 4)
    aux[1] = (aux[1] & km2) | (((tmp >> 2) & km1) << 4)
    scales = np.frombuffer(struct.pack("<4I", *aux), np.int8)
    out, q, m, is_ = [], 32, 1, 0
    for _ in range(2):
        shift = 0
        for _ in range(4):
            for half in (0, 16):
                dl = np.float32(d) * np.float32(int(scales[is_]) - 32)
                is_ += 1
                for l in range(16):
                    v = ((blk[q + l + half] >> shift) & 3) - (0 if blk[l + half] & m else 4)
                    out.append(np.float32(dl * np.float32(v)))
            shift += 2
            m <<= 1
        q += 32
    return np.array(out, np.float32)


def _iq3s_walk(blk: bytes) -> np.ndarray:
    """quant.cpp:350-384's loops walked literally: pairs of sub-blocks, each half moving qs by
    8 and signs by 4, qh by 2 per pair, the 9th index bit taken from h << (8 - 2 l) and
    h << (7 - 2 l)."""
    d = np.float32(np.frombuffer(blk[0:2], np.float16)[0])
    qs, qh, signs, scales = 2, 66, 74, 106
    out = []
    for ib32 in range(0, 8, 2):
        db1 = d * np.float32(1 + 2 * (blk[scales + ib32 // 2] & 0xF))
        db2 = d * np.float32(1 + 2 * (blk[scales + ib32 // 2] >> 4))
        for half in range(2):
            db = db1 if half == 0 else db2
            h = blk[qh + half]
            for l in range(4):
                g1 = blk[qs + 2 * l] | ((h << (8 - 2 * l)) & 256)
                g2 = blk[qs + 2 * l + 1] | ((h << (7 - 2 * l)) & 256)
                vals = [0.0] * 8
                for j in range(4):
                    s1 = np.float32(-1) if blk[signs + l] & KMASK[j] else np.float32(1)
                    s2 = np.float32(-1) if blk[signs + l] & KMASK[j + 4] else np.float32(1)
                    vals[j] = db * np.float32((IQ3S_GRID[g1] >> (8 * j)) & 0xFF) * s1
                    vals[j + 4] = db * np.float32((IQ3S_GRID[g2] >> (8 * j)) & 0xFF) * s2
                out.extend(vals)
            qs += 8
            signs += 4
        qh += 2
    return np.array(out, np.float32)


def _blocks_with_scale(rng, n, bb, d_at):
    w = rng.integers(0, 256, size=n * bb, dtype=np.uint8)
    for b in range(n):
        w[bb * b + d_at: bb * b + d_at + 2] = np.frombuffer(f16_bytes(rng.uniform(-0.05, 0.05)), np.uint8)
    w[d_at: d_at + 2] = (0x07, 0x00)  # an fp16-subnormal d in the first block
    return w


@pytest.mark.parametrize("t,walk,d_at", [(Q3_K, _q3k_walk, 108), (IQ3_S, _iq3s_walk, 0)])
def test_q3_k_iq3_s_equal_the_literal_loop_walk(oracle, t, walk, d_at):
    """On random blocks the oracle's per-element index form equals a literal walk of the
    reference's loops bitwise (signed zeros included)."""
    rng = np.random.default_rng(21 + t)
    w = _blocks_with_scale(rng, 24, 110, d_at)
    y = oracle.dequantize_row(t, w, 24 * 256)
    want = np.concatenate([walk(bytes(w[110 * b: 110 * (b + 1)])) for b in range(24)])
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def iq3s_block(d: float, qs: bytes, qh: bytes, signs: bytes, scales: bytes) -> np.ndarray:
    assert len(qs) == 64 and len(qh) == 8 and len(signs) == 32 and len(scales) == 4
    return np.frombuffer(f16_bytes(d) + qs + qh + signs + scales, np.uint8)


def test_iq3_s_known_answers(oracle):
    """All-zero fields, d = 0.25: codebook entry 0 (0x01010101), scale 1, no signs -> 0.25
    everywhere. Then sub-block 3, group 5 takes entry 0x1FF (qs[29] = 0xFF, bit 5 of qh[3]),
    element 3 * 32 + 5 * 4 + 1 is negated (bit 5 of signs[14]), and sub-block 3's scale
    nibble (the high one of scales[1]) is 2 (multiplier 5)."""
    z = iq3s_block(0.25, bytes(64), bytes(8), bytes(32), bytes(4))
    assert np.all(oracle.dequantize_row(IQ3_S, z, 256) == np.float32(0.25))
    qs, qh, signs, scales = bytearray(64), bytearray(8), bytearray(32), bytearray(4)
    qs[3 * 8 + 5] = 0xFF
    qh[3] = 1 << 5
    signs[3 * 4 + 2] = 1 << 5  # elements 3*32 + 16 .. +23: the 6th one, i.e. 3*32 + 21
    scales[1] = 0x20
    y = oracle.dequantize_row(IQ3_S, iq3s_block(0.25, bytes(qs), bytes(qh), bytes(signs), bytes(scales)), 256)
    g = IQ3S_GRID[0x1FF]
    want = np.full(256, 0.25, np.float32)
    want[96:128] = 0.25 * 5  # sub-block 3's multiplier
    for k in range(4):
        want[96 + 20 + k] = 0.25 * 5 * ((g >> (8 * k)) & 0xFF)
    want[96 + 21] = -want[96 + 21]
    assert np.array_equal(y, want)


@pytest.mark.parametrize("t,bb,be,d_at", [(IQ4_NL, 18, 32, 0), (Q3_K, 110, 256, 108), (IQ3_S, 110, 256, 0)])
def test_new_type_dequant_terms(oracle, t, bb, be, d_at):
    """a is the dequantized weight bitwise, b = 0, and off is the multiplier times the code
    bias the kernels add (IQ4_NL 128 d; Q3_K 4 d (sc - 32) per 16-element run; IQ3_S 16 db per
    32-element sub-block), recomputed here from the block bytes."""
    rng = np.random.default_rng(40 + t)
    n = 6
    w = _blocks_with_scale(rng, n, bb, d_at)
    a, b_, off = oracle.dequant_terms(t, w, 1, n * be)
    y = oracle.dequantize_row(t, w, n * be)
    assert np.array_equal(a[0].view(np.uint32), y.view(np.uint32)) and np.all(b_ == 0)
    for b in range(n):
        blk = bytes(w[bb * b: bb * (b + 1)])
        d = _f16(blk, d_at)
        if t == IQ4_NL:
            want = np.full(32, np.float32(128) * d, np.float32)
        elif t == Q3_K:
            s = [((blk[96 + i % 8] >> (4 * (i // 8))) & 15) | (((blk[104 + i % 4] >> (2 * (i // 4))) & 3) << 4)
                 for i in range(16)]
            want = np.repeat([np.float32(4) * np.float32(d * np.float32(v - 32)) for v in s], 16).astype(np.float32)
        else:
            s = [(blk[106 + i // 2] >> (4 * (i % 2))) & 15 for i in range(8)]
            want = np.repeat([np.float32(16) * np.float32(d * np.float32(1 + 2 * v)) for v in s], 32).astype(np.float32)
        assert np.array_equal(off[0, be * b: be * (b + 1)], want), b


# ---- the rest of the dequantizer's dispatch: BF16, Q4_1, Q5_0, Q5_1, Q2_K ---------------------
# (quant.cpp:72-74, :93-140, :168-193; dispatch :386-407; geometry dtype.cpp:26-30, :33, :53)

Q4_1, Q5_0, Q5_1, Q2_K, BF16 = 3, 6, 7, 10, 30


def test_extra_type_geometry(oracle):
    """dtype.cpp's table rows 3, 6, 7, 10 and 30 (block elements, block bytes)."""
    for t, be, bb in ((Q4_1, 32, 20), (Q5_0, 32, 22), (Q5_1, 32, 24), (Q2_K, 256, 84), (BF16, 1, 2)):
        assert oracle.row_bytes(t, 17408 if be > 1 else 7) == (17408 // be * bb if be > 1 else 14)
    for t, n in ((Q4_1, 16), (Q5_0, 48), (Q5_1, 1), (Q2_K, 128)):
        with pytest.raises(oracle.OracleError) as e:
            oracle.row_bytes(t, n)
        assert e.value.code == oracle.EMODEL
    for t in (4, 5, 9, 15, 16, 24, 29):  # unassigned ids and types without a dequantizer
        with pytest.raises(oracle.OracleError) as e:
            oracle.row_bytes(t, 256)
        assert e.value.code == oracle.EUNSUPPORTED


def test_bf16_rows_are_the_top_half_of_fp32(oracle):
    """Every one of the 65536 bf16 patterns widens to the fp32 pattern with the same top 16 bits
    and zero below (fp16.h:61-63): a closed form, NaN payloads and signed zeros included."""
    pats = np.arange(65536, dtype=np.uint16)
    y = oracle.dequantize_row(BF16, pats.view(np.uint8), 65536)
    assert np.array_equal(y.view(np.uint32), pats.astype(np.uint32) << 16)


def _walk_q4_1_q5(blk: bytes, t: int) -> np.ndarray:
    """quant.cpp:93-140's loops walked literally: j over 16 bytes writing y[j] and y[j + 16], the
    fifth bits xh_0 = ((qh >> j) << 4) & 0x10 and xh_1 = (qh >> (j + 12)) & 0x10."""
    d = np.float32(np.frombuffer(blk[0:2], np.float16)[0])
    m = np.float32(np.frombuffer(blk[2:4], np.float16)[0]) if t in (Q4_1, Q5_1) else None
    qh = struct.unpack("<I", blk[{Q5_0: 2, Q5_1: 4}[t]: {Q5_0: 2, Q5_1: 4}[t] + 4])[0] if t != Q4_1 else 0
    qs = blk[{Q4_1: 4, Q5_0: 6, Q5_1: 8}[t]:]
    y = [np.float32(0)] * 32
    for j in range(16):
        xh_0 = ((qh >> j) << 4) & 0x10
        xh_1 = (qh >> (j + 12)) & 0x10
        x0, x1 = (qs[j] & 0x0F) | xh_0, (qs[j] >> 4) | xh_1
        if t == Q5_0:
            y[j], y[j + 16] = np.float32(x0 - 16) * d, np.float32(x1 - 16) * d
        else:
            y[j], y[j + 16] = np.float32(x0) * d + m, np.float32(x1) * d + m
    return np.array(y, np.float32)


def _walk_q2_k(blk: bytes) -> np.ndarray:
    """quant.cpp:168-193's loops walked literally: two halves moving q by 32, four shifts, two
    runs of 16 per shift, each run taking the next scale byte (is++)."""
    d = np.float32(np.frombuffer(blk[80:82], np.float16)[0])
    dmin = np.float32(np.frombuffer(blk[82:84], np.float16)[0])
    out, q, is_ = [], 16, 0
    for _ in range(2):
        shift = 0
        for _ in range(4):
            for half in (0, 16):
                sc = blk[is_]
                is_ += 1
                dl, ml = d * np.float32(sc & 0xF), dmin * np.float32(sc >> 4)
                for l in range(16):
                    out.append(dl * np.float32((blk[q + half + l] >> shift) & 3) - ml)
            shift += 2
        q += 32
    return np.array(out, np.float32)


@pytest.mark.parametrize("t,bb,be", [(Q4_1, 20, 32), (Q5_0, 22, 32), (Q5_1, 24, 32), (Q2_K, 84, 256)])
def test_extra_types_equal_the_literal_loop_walk(oracle, t, bb, be):
    """On random blocks (finite scales, one fp16-subnormal d) the oracle's per-element index form
    equals a literal walk of the reference's loops bitwise."""
    rng = np.random.default_rng(60 + t)
    n = 40
    w = rng.integers(0, 256, size=n * bb, dtype=np.uint8)
    hdr = (80, 82) if t == Q2_K else ((0, 2) if t in (Q4_1, Q5_1) else (0,))
    for b in range(n):
        for k, at in enumerate(hdr):
            v = rng.uniform(-0.05, 0.05) if k == 0 else rng.uniform(-0.5, 0.5)
            w[bb * b + at: bb * b + at + 2] = np.frombuffer(f16_bytes(v), np.uint8)
    w[hdr[0]: hdr[0] + 2] = (0x03, 0x00)  # an fp16-subnormal d in the first block
    y = oracle.dequantize_row(t, w, n * be)
    walk = _walk_q2_k if t == Q2_K else (lambda blk: _walk_q4_1_q5(blk, t))
    want = np.concatenate([walk(bytes(w[bb * b: bb * (b + 1)])) for b in range(n)])
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def test_q4_1_known_answers(oracle):
    """qs[j] = (15 - j) << 4 | j: element j < 16 has code j, j + 16 code 15 - j. d = 1, m = 0
    gives the codes; d = 0.5, m = -4 gives q / 2 - 4 exactly; m = 65504 with the smallest
    subnormal d (2^-24) gives 65504 for every code (q d is below half an ulp of m)."""
    qs = bytes(((15 - j) << 4) | j for j in range(16))
    codes = np.array(list(range(16)) + [15 - j for j in range(16)], np.float32)

    def blk(d_bits, m):
        return np.frombuffer(struct.pack("<H", d_bits) + f16_bytes(m) + qs, np.uint8)

    assert np.array_equal(oracle.dequantize_row(Q4_1, blk(0x3C00, 0.0), 32), codes)
    assert np.array_equal(oracle.dequantize_row(Q4_1, blk(0x3800, -4.0), 32), codes / 2 - 4)
    assert np.all(oracle.dequantize_row(Q4_1, blk(0x0001, 65504.0), 32) == np.float32(65504))


@pytest.mark.parametrize("t", [Q5_0, Q5_1])
def test_q5_fifth_bit_is_bit_e_of_qh(oracle, t):
    """Every nibble 8 (qs bytes 0x88) and only bits 3 and 20 of qh set: elements 3 and 20 have
    code 24, every other element code 8. With d = 0.5 (and m = 1 for Q5_1) the values are
    Q5_0: (code - 16) / 2, Q5_1: code / 2 + 1. (Bit e for e >= 16 comes from xh_1's shift by
    j + 12: reading bit e - 16 instead would move element 20's bit to element 4.)"""
    qh = struct.pack("<I", (1 << 3) | (1 << 20))
    hdr = f16_bytes(0.5) + (f16_bytes(1.0) if t == Q5_1 else b"")
    y = oracle.dequantize_row(t, np.frombuffer(hdr + qh + b"\x88" * 16, np.uint8), 32)
    code = np.full(32, 8.0, np.float32)
    code[[3, 20]] = 24.0
    want = (code - 16) / 2 if t == Q5_0 else code / 2 + 1
    assert np.array_equal(y, want.astype(np.float32))


def test_q2_k_known_answers(oracle):
    """qs bytes 0xE4 hold codes 0, 1, 2, 3 at shifts 0, 2, 4, 6, so element 128 n + 32 j + l has
    code j. Scale bytes 0x21 (scale 1, min 2) with d = 0.5, dmin = 0.25: value j / 2 - 0.5.
    Then scale byte 11 alone = 0x53 (scale 3, min 5): the 16-element run 11 in element order
    (elements 176 .. 191: half 1, shift pair 1, second run; code 1) becomes 3 / 2 - 5 / 4."""
    def blk(scales):
        return np.frombuffer(bytes(scales) + b"\xe4" * 64 + f16_bytes(0.5) + f16_bytes(0.25), np.uint8)

    j = (np.arange(256) % 128) // 32
    want = (j * 0.5 - 0.5).astype(np.float32)
    assert np.array_equal(oracle.dequantize_row(Q2_K, blk([0x21] * 16), 256), want)
    sc = [0x21] * 16
    sc[11] = 0x53
    want[176:192] = np.float32(1.5 - 1.25)
    assert np.array_equal(oracle.dequantize_row(Q2_K, blk(sc), 256), want)


@pytest.mark.parametrize("t,bb,be", [(Q4_1, 20, 32), (Q5_0, 22, 32), (Q5_1, 24, 32), (Q2_K, 84, 256), (BF16, 2, 1)])
def test_extra_type_dequant_terms(oracle, t, bb, be):
    """a - b is the dequantized weight bitwise (b = -m for Q4_1 / Q5_1, ml for Q2_K, else 0), and
    no kernel takes a code bias out (off = 0)."""
    rng = np.random.default_rng(80 + t)
    n = 8 if be > 1 else 256
    w = rng.integers(0, 256, size=n * bb, dtype=np.uint8)
    w[1::2] &= 0xBF  # every fp16 / bf16 field finite
    a, b_, off = oracle.dequant_terms(t, w, 1, n * be)
    y = oracle.dequantize_row(t, w, n * be)
    assert np.array_equal((a[0] - b_[0]).view(np.uint32), y.view(np.uint32)) and np.all(off == 0)
    if t in (Q5_0, BF16):
        assert np.all(b_ == 0)


# ---- rms_norm (backends/cpu/ops_basic.cpp:18-33) ------------------------------------------


def test_rms_norm_sum_of_squares_in_the_dot_order(oracle):
    """x[0] = 4096 and x[1 + 8 j] = 1 for j < 8 (64 columns, eps = 0, w = 1). In the dot's 8-lane
    order the eight ones share lane 1 (p1 = 8) and 2^24 + 8 is exact: the sum is 16777224. Added
    one at a time to 2^24, each 1 rounds away (ties to even): 16777216. The two orders give
    different outputs, and the oracle must give the first."""
    x = np.zeros(64, np.float32)
    x[0] = 4096.0
    x[1::8] = 1.0
    f = np.float32

    def expected(ss):
        inv = f(1.0) / np.sqrt(f(ss) / f(64))
        return (x * inv) * f(1.0)

    good, seq = expected(16777224.0), expected(16777216.0)
    assert not np.array_equal(good, seq)
    y = oracle.rms_norm(x, np.ones(64, np.float32), eps=0.0)
    assert np.array_equal(y, good)


def test_rms_norm_closed_forms(oracle):
    w = np.random.default_rng(3).standard_normal(64).astype(np.float32)
    # x = 0.5 everywhere, eps = 0: mean 0.25, inv 2, x * inv = 1 exactly: out = w bitwise
    assert np.array_equal(oracle.rms_norm(np.full(64, 0.5, np.float32), w, eps=0.0), w)
    # a zero row: inv = 1 / sqrt(eps), out = 0 (with eps = 0, 0 * inf = NaN, as on the CPU)
    assert np.array_equal(oracle.rms_norm(np.zeros(64, np.float32), w, eps=1e-6), np.zeros(64, np.float32) * w)
    assert np.all(np.isnan(oracle.rms_norm(np.zeros(64, np.float32), w, eps=0.0)))


@pytest.mark.parametrize("cols", [5, 8, 100, 5120])
def test_rms_norm_within_fp64_bound_rows_independent(oracle, cols):
    """Against fp64: the sum of squares has relative error <= (cols/8 + 4) u (positive terms,
    longest chain), which moves inv by half of that; mean, +eps, sqrt, 1/ and the two products
    add at most 6 u."""
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    y = oracle.rms_norm(x, w, eps=1e-6)
    x64 = x.astype(np.float64)
    inv = 1.0 / np.sqrt((x64 * x64).sum(axis=1, keepdims=True) / cols + np.float64(np.float32(1e-6)))
    ref = x64 * inv * w.astype(np.float64)
    tol = (0.5 * (cols / 8 + 4) + 8) * U * np.abs(ref) + 1e-300
    assert np.all(np.abs(y - ref) <= tol)
    # each row on its own gives the same bits (no state across rows)
    for r in range(3):
        assert np.array_equal(oracle.rms_norm(x[r], w, eps=1e-6), y[r])


def test_dequant_rejects_bad_arguments(oracle):
    """tests/unit/tensor/test_dequant.cpp:74-87."""
    src = np.zeros(210, np.uint8)
    dst = np.zeros(256, np.float32)
    lib = oracle.lib()
    assert lib.oracle_dequantize_row(Q6_K, src.ctypes.data, dst.ctypes.data, 255) == oracle.EMODEL
    assert lib.oracle_dequantize_row(Q6_K, src.ctypes.data, dst.ctypes.data, -256) == oracle.EMODEL
    assert lib.oracle_dequantize_row(16, src.ctypes.data, dst.ctypes.data, 256) == oracle.EUNSUPPORTED
    assert lib.oracle_dequantize_row(Q6_K, src.ctypes.data, dst.ctypes.data, 256) == oracle.OK
    assert oracle.dequantize_row(Q6_K, src, 0).size == 0


# ---- dot order, vec_dot_row, matmul ----------------------------------------------------------


def test_dot_fixed_8_lane_order_known_answer(oracle):
    """cpu::detail::dot: partial j sums i = j mod 8, combined ((p0+p4)+(p1+p5))+((p2+p6)+(p3+p7)),
    then the tail. With a = [2^24, 1 x 7], b = 1: p0 + p4 = 2^24 + 1 rounds (ties to even) to
    2^24, p1 + p5 = 2, right half = 4, total 2^24 + 6. A sequential sum would give 2^24."""
    a = np.array([2.0 ** 24] + [1.0] * 7, np.float32)
    assert oracle.dot(a, np.ones(8, np.float32)) == 16777222.0
    # tail (n % 8 elements) is summed separately and added last: 2^24 + 6 + 1 -> 2^24 + 8
    a9 = np.append(a, np.float32(1.0))
    assert oracle.dot(a9, np.ones(9, np.float32)) == 16777224.0
    # a sequential reduction would lose every 1: the order is really being pinned
    s = np.float32(0)
    for v in a:
        s = np.float32(s + v)
    assert s == 16777216.0


def test_vec_dot_row_matches_sequential_double(oracle):
    """tests/unit/tensor/test_dequant.cpp:90-112."""
    rng = np.random.default_rng(7)
    n = 1024
    for t in (F32, 1, 30, Q4_0, Q8_0, Q4_K, Q6_K, 20, 21):  # F16, BF16, IQ4_NL, IQ3_S by id
        row = rng.integers(0, 256, size=oracle.row_bytes(t, n), dtype=np.uint8)
        row[1::2] &= 0xBF  # cap exponents: every fp16 field stays finite
        x = ((rng.integers(0, 2001, n) - 1000) / 1000.0).astype(np.float32)
        w = oracle.dequantize_row(t, row, n)
        ref = 0.0
        for i in range(n):
            ref += float(w[i]) * float(x[i])
        assert oracle.vec_dot_row(t, row, x) == np.float32(ref), t


def brute_force_fp64(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    return x.astype(np.float64) @ w.astype(np.float64).T


@pytest.mark.parametrize("t,k,n", [(1, 5120, 67), (7, 512, 37), (3, 256, 1)])
def test_matmul_within_derived_bound_of_fp64(oracle, t, k, n):
    """y within d_cpu * u * sum|x w| of the exact fp64 product (cf. test_ops.cpp:446-471)."""
    rng = np.random.default_rng(10 + k)
    for wt in (Q4_K, Q6_K, Q4_0, Q8_0):
        row = rng.integers(0, 256, size=n * oracle.row_bytes(wt, k), dtype=np.uint8)
        row[1::2] &= 0xBF
        x = rng.standard_normal((t, k)).astype(np.float32)
        y = oracle.matmul(wt, row, n, k, x)
        w = oracle.dequantize_rows(wt, row, n, k)
        ref = brute_force_fp64(w, x)
        mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
        tol = (depth_cpu(k) + 1) * U * mag + 1e-38
        assert np.all(np.abs(y - ref) <= tol), wt
        # and each output is exactly the fixed-order dot of its dequantized row
        for ti in range(t):
            for ni in range(0, n, max(1, n // 5)):
                assert y[ti, ni] == oracle.dot(x[ti], w[ni])


def test_matmul_dense_equals_dequantized_bitwise(oracle):
    rng = np.random.default_rng(3)
    k, n = 512, 45
    wq = rng.integers(0, 256, size=n * oracle.row_bytes(Q4_K, k), dtype=np.uint8)
    wq[1::2] &= 0xBF
    w = oracle.dequantize_rows(Q4_K, wq, n, k)
    x = rng.standard_normal((4, k)).astype(np.float32)
    assert np.array_equal(oracle.matmul(Q4_K, wq, n, k, x).view(np.uint32),
                          oracle.matmul(F32, w.view(np.uint8), n, k, x).view(np.uint32))


def test_matmul_padded_stride_equals_dense(oracle):
    rng = np.random.default_rng(4)
    k, n, pad = 512, 21, 3
    rb = oracle.row_bytes(Q6_K, k)
    wq = rng.integers(0, 256, size=n * rb, dtype=np.uint8)
    wq[1::2] &= 0xBF
    padded = np.zeros(n * (rb + pad), np.uint8)
    for r in range(n):
        padded[r * (rb + pad): r * (rb + pad) + rb] = wq[r * rb:(r + 1) * rb]
    x = rng.standard_normal((2, k)).astype(np.float32)
    assert np.array_equal(oracle.matmul(Q6_K, wq, n, k, x), oracle.matmul(Q6_K, padded, n, k, x, w_stride=rb + pad))


def test_matmul_thread_count_invariance(oracle):
    """Bitwise identical for any thread count (thread_pool.h:8-10; test_ops.cpp:517-565)."""
    rng = np.random.default_rng(12)
    k, n = 768 // 256 * 256, 150
    wq = rng.integers(0, 256, size=n * oracle.row_bytes(Q4_K, k), dtype=np.uint8)
    wq[1::2] &= 0xBF
    x = rng.standard_normal((9, k)).astype(np.float32)
    base = oracle.matmul(Q4_K, wq, n, k, x, threads=1)
    for th in (2, 3, 7, 16, 64):
        assert np.array_equal(oracle.matmul(Q4_K, wq, n, k, x, threads=th).view(np.uint32), base.view(np.uint32)), th


def test_partition_range_literal(oracle):
    import ctypes

    lib = oracle.lib()
    got = []
    for i in range(3):
        b, e = ctypes.c_size_t(), ctypes.c_size_t()
        lib.oracle_partition_range(10, 3, i, ctypes.byref(b), ctypes.byref(e))
        got.append((b.value, e.value))
    assert got == [(0, 4), (4, 7), (7, 10)]


def test_swiglu_closed_forms(oracle):
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 88.0, -100.0], np.float32)
    u = np.array([5.0, 2.0, 3.0, 1.0, 1.0, 0.5, 7.0], np.float32)
    out = oracle.swiglu(g, u)
    assert out[0] == 0.0
    assert out[3] == np.float32(30.0)  # sigmoid(30) rounds to 1 in fp32
    ref = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u
    # fp32 overflow of exp(100) makes silu(-100) exactly -0: an absolute floor covers it
    assert np.all(np.abs(out - ref) <= 8 * U * np.abs(ref) + 1e-37)


def test_gate_up_composition_equals_parts(oracle):
    rng = np.random.default_rng(5)
    k, n = 512, 40
    wg = rng.integers(0, 256, size=n * oracle.row_bytes(Q4_K, k), dtype=np.uint8)
    wu = rng.integers(0, 256, size=n * oracle.row_bytes(Q4_K, k), dtype=np.uint8)
    wg[1::2] &= 0xBF
    wu[1::2] &= 0xBF
    x = rng.standard_normal((3, k)).astype(np.float32)
    out = oracle.gate_up_swiglu(Q4_K, wg, wu, n, k, x)
    g = oracle.matmul(Q4_K, wg, n, k, x)
    u = oracle.matmul(Q4_K, wu, n, k, x)
    assert np.array_equal(out, oracle.swiglu(g, u))


# ---- LM head: matmul + fused argmax (src/backend/cpu_backend.cpp:669-770) ------------------

QNAN_BITS = 0x7FC00000  # std::numeric_limits<float>::quiet_NaN()
NO_INDEX = 0xFFFFFFFF   # index -1 as the u32 result word


def _f32_head(logit_cols):
    """F32 head weights whose logits are chosen directly: W[:, 0] = logits, x = e_0 (every
    other product is an exact 0, so the fp32 dot returns the logit bitwise)."""
    logits = np.asarray(logit_cols, np.float32)
    w = np.zeros((logits.size, 8), np.float32)
    w[:, 0] = logits
    return w.view(np.uint8).ravel(), logits.size, 8


def _bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def test_lm_head_ties_go_to_the_lowest_index(oracle):
    w, rows, cols = _f32_head([1, 5, 5, -2, 3, 5, 0, 4, 1, 2])
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 1
    res, logits = oracle.lm_head(F32, w, rows, cols, x)
    assert logits[0].tolist() == [1, 5, 5, -2, 3, 5, 0, 4, 1, 2]
    assert res[0].tolist() == [int(np.argmax(logits[0])), _bits(5.0), 0] == [1, _bits(5.0), 0]


def test_lm_head_zero_ties_and_infinities(oracle):
    # equal zeros: the lower index wins (the dot starts from +0, so a -0 weight gives a +0
    # logit); +inf beats every finite value; -inf loses to everything
    w, rows, cols = _f32_head([-np.inf, -0.0, 0.0, -1.0])
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 1
    res, logits = oracle.lm_head(F32, w, rows, cols, x)
    assert logits[0, 1] == logits[0, 2] == 0.0
    assert res[0].tolist() == [1, int(logits[0, 1].view(np.uint32)), 0]
    w, rows, cols = _f32_head([3.0, np.inf, 7.0, np.inf])
    res, _ = oracle.lm_head(F32, w, rows, cols, x)
    assert res[0].tolist() == [1, _bits(np.inf), 0]


def test_lm_head_nan_poisons_only_its_vector(oracle):
    w, rows, cols = _f32_head([1, 9, 3])
    x = np.zeros((3, cols), np.float32)
    x[:, 0] = 1
    x[1, 5] = np.nan  # every logit of vector 1 is NaN
    res, _ = oracle.lm_head(F32, w, rows, cols, x)
    assert res[0].tolist() == [1, _bits(9.0), 0]
    assert res[1].tolist() == [NO_INDEX, QNAN_BITS, 1]
    assert res[2].tolist() == [1, _bits(9.0), 0]


def test_lm_head_valid_rows_clamps_the_argmax_not_the_logits(oracle):
    w, rows, cols = _f32_head([1, 2, 3, 10, 20])
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 1
    res, logits = oracle.lm_head(F32, w, rows, cols, x, valid_rows=3)
    assert res[0].tolist() == [2, _bits(3.0), 0]
    assert logits[0].tolist() == [1, 2, 3, 10, 20]
    # valid_rows past the end is the whole matrix; 0 is the whole matrix
    for vr in (0, 5, 99):
        res, _ = oracle.lm_head(F32, w, rows, cols, x, valid_rows=vr)
        assert res[0].tolist() == [4, _bits(20.0), 0]


def test_lm_head_nan_past_valid_rows_still_poisons(oracle):
    # cpu_backend.cpp:734-739: the NaN test comes before the valid_rows clamp
    w, rows, cols = _f32_head([1, 2, np.nan])
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 1
    res, _ = oracle.lm_head(F32, w, rows, cols, x, valid_rows=2)
    assert res[0].tolist() == [NO_INDEX, QNAN_BITS, 1]


def test_lm_head_across_8192_row_slabs(oracle):
    # the maximum in the second slab, and a tie across the slab boundary
    vals = np.zeros(8192 + 100, np.float32)
    vals[8192 + 50] = 4.0
    vals[7000] = 4.0
    w, rows, cols = _f32_head(vals)
    x = np.zeros((1, cols), np.float32)
    x[0, 0] = 1
    res, _ = oracle.lm_head(F32, w, rows, cols, x)
    assert res[0].tolist() == [7000, _bits(4.0), 0]
    vals[7000] = 3.0
    w, rows, cols = _f32_head(vals)
    res, _ = oracle.lm_head(F32, w, rows, cols, x)
    assert res[0].tolist() == [8242, _bits(4.0), 0]


def test_lm_head_q6_k_logits_are_matmul_and_index_is_first_argmax(oracle):
    rng = np.random.default_rng(11)
    rows, cols = 300, 512
    w = rng.integers(0, 256, size=rows * oracle.row_bytes(Q6_K, cols), dtype=np.uint8)
    w[208::210] = 0x00  # keep every d finite: fp16 d with a small exponent
    w[209::210] &= 0x0F
    x = rng.standard_normal((4, cols)).astype(np.float32)
    res, logits = oracle.lm_head(Q6_K, w, rows, cols, x)
    assert np.array_equal(logits, oracle.matmul(Q6_K, w, rows, cols, x))
    for i in range(4):
        assert res[i, 0] == np.argmax(logits[i]) and res[i, 1] == logits[i].max().view(np.uint32) and res[i, 2] == 0


# ---- argmax (backends/cpu/matmul.cpp:61-72) -------------------------------------------------


def test_argmax_words_first_maximum_and_poison(oracle):
    """The index is numpy's first maximum (ties to the lowest index), the value its bits; a row
    with a NaN anywhere gives the poisoned words {0xFFFFFFFF, NaN, 1}."""
    rng = np.random.default_rng(21)
    lg = rng.standard_normal((6, 777)).astype(np.float32)
    lg[0, [3, 500]] = 7.0                      # tie
    lg[1, :] = -np.inf                         # all -inf: index 0
    lg[2, 0] = np.nan                          # NaN first
    lg[3, 776] = np.nan                        # NaN last
    lg[4, :] = 0.0
    lg[4, 9] = -0.0                            # -0 == +0: the first zero stays
    res = oracle.argmax_words(lg)
    for i in range(6):
        if np.isnan(lg[i]).any():
            assert res[i, 0] == 0xFFFFFFFF and res[i, 2] == 1 and np.isnan(res[i, 1:2].view(np.float32)[0]), i
            continue
        j = int(np.argmax(lg[i]))
        assert res[i, 0] == j and res[i, 2] == 0, i
        assert res[i, 1] == lg[i, j:j + 1].view(np.uint32)[0], i
    assert res[0, 0] == 3 and res[1, 0] == 0 and res[4, 0] == 0
