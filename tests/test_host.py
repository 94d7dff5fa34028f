"""CPU-side tests of the product library: the C ABI loads and exports every declared symbol,
the host SLAB repack is a bijection with the documented byte placement, and the synthetic
input generators (normal fill, quantizers) are deterministic and sane. No GPU calls."""
import re
from pathlib import Path

import numpy as np
import pytest

from helpers import BLOCK, IQ4_XS, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0, QUANT_TYPES, make_weights, row_bytes

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "halo_mi355x.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(halo_mi_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(hl):
    import ctypes

    names = declared_functions()
    assert len(names) >= 13
    so = ctypes.CDLL(str(ROOT / "halo_amd" / "libhalo_mi355x.so"))
    for n in names:
        assert hasattr(so, n), n
    from halo_amd._lib import SIGNATURES

    assert sorted(SIGNATURES) == names  # every declared function is bound, nothing else


def test_geometry(hl):
    assert hl.row_bytes(Q4_K, 5120) == 2880
    assert hl.row_bytes(Q6_K, 17408) == 14280
    assert hl.row_bytes(Q4_K, 100) == 0
    assert hl.slab_bytes(Q4_K, 17408, 5120) == 17408 * 2880
    assert hl.slab_bytes(Q6_K, 65, 512) == 128 * 2 * 210  # rows rounded up to 64
    assert hl.slab_bytes(Q5_K, 65, 512) == 128 * 2 * 176
    assert hl.slab_bytes(IQ4_XS, 64, 256) == 64 * 136
    assert hl.slab_bytes(11, 64, 256) == 0  # Q3_K: not on this path


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("rows", [1, 64, 70, 130])
def test_host_repack_is_a_bijection(hl, t, rows):
    cols = 512
    buf, stride = make_weights(t, rows, cols, seed=rows + t)
    rb = row_bytes(t, cols)
    dense = np.concatenate([buf[r * stride: r * stride + rb] for r in range(rows)])
    slab = hl.repack_slab_host(t, dense, rows, cols)
    assert slab.size == (rows + 63) // 64 * 64 * rb
    back = hl.unpack_slab_host(t, slab, rows, cols)
    assert np.array_equal(back, dense)
    # a permutation of the bits plus zero padding rows: the number of set bits is kept
    assert int(np.unpackbits(slab).sum()) == int(np.unpackbits(dense).sum())


def test_host_repack_strided_source(hl):
    t, rows, cols = Q6_K, 13, 512
    buf, stride = make_weights(t, rows, cols, seed=9, stride_pad=3, offset=1)
    rb = row_bytes(t, cols)
    dense = np.concatenate([buf[1 + r * stride: 1 + r * stride + rb] for r in range(rows)])
    a = hl.repack_slab_host(t, dense, rows, cols)
    b = hl.repack_slab_host(t, buf[1:], rows, cols, src_stride=stride)
    assert np.array_equal(a, b)


def test_slab_byte_placement_q4_k(hl):
    """Slot j of super-block b, row r: 16 B at (8 b + j) * 64 * 16 + r * 16; byte t holds the
    sub-block's element t (low nibble) and t + 16 (high nibble). Headers follow the quants."""
    rows, cols = 3, 512
    rng = np.random.default_rng(1)
    w = rng.integers(0, 256, size=rows * row_bytes(Q4_K, cols), dtype=np.uint8)
    slab = hl.repack_slab_host(Q4_K, w, rows, cols)
    nb, S = cols // 256, cols // 32
    for r in range(rows):
        for b in range(nb):
            blk = w[r * 288 + b * 144: r * 288 + (b + 1) * 144]
            hdr = slab[S * 64 * 16 + (b * 64 + r) * 16:][:16]
            assert np.array_equal(hdr, blk[:16])
            for j in range(8):
                g, hi = j // 2, j % 2
                q = blk[16 + 32 * g: 16 + 32 * g + 32]
                vals = (q >> 4) if hi else (q & 15)  # sub-block j's 32 quants in element order
                rec = slab[((8 * b + j) * 64 + r) * 16:][:16]
                assert np.array_equal(rec & 15, vals[:16]) and np.array_equal(rec >> 4, vals[16:])


def test_slab_byte_placement_q6_k(hl):
    """Q6_K slot records rebuild every 6-bit quant: low nibbles as in the 4-bit record, top
    bits per the qh record layout (bits 5:4 / 7:6 / 1:0 / 3:2)."""
    rows, cols = 2, 256
    rng = np.random.default_rng(2)
    w = rng.integers(0, 256, size=rows * 210, dtype=np.uint8)
    slab = hl.repack_slab_host(Q6_K, w, rows, cols)
    S = 8
    for r in range(rows):
        blk = w[r * 210:(r + 1) * 210]
        # the 256 unsigned 6-bit quants in element order, from the GGUF block
        q = np.zeros(256, np.int64)
        for e in range(256):
            n, rr = e // 128, e % 128
            k, l = rr // 32, rr % 32
            lb = blk[64 * n + l + 32 * (k & 1)]
            q[e] = ((lb & 15) if k < 2 else (lb >> 4)) | (((blk[128 + 32 * n + l] >> (2 * k)) & 3) << 4)
        for j in range(S):
            ql = slab[(j * 64 + r) * 16:][:16]
            qh = slab[S * 64 * 16 + (j * 64 + r) * 8:][:8]
            for e in range(32):
                lo4 = (ql[e] & 15) if e < 16 else (ql[e - 16] >> 4)
                base, up = e % 16, e // 16
                w_, rem = base // 8, base % 8
                byte = qh[4 * w_ + rem % 4]
                shift = (2 if up else 0) if rem >= 4 else (6 if up else 4)
                assert lo4 | (((byte >> shift) & 3) << 4) == q[32 * j + e]
        sc = slab[S * 64 * 24 + r * 16:][:16]
        d = slab[S * 64 * 24 + 64 * 16 + r * 2:][:2]
        assert np.array_equal(sc, blk[192:208]) and np.array_equal(d, blk[208:210])


def test_slab_byte_placement_q5_k(hl):
    """Q5_K: 4-bit records as Q4_K (quants at byte 48), a 4-byte word per (slot, row) holding
    the fifth bits (element e's at bit i + 8 b for e = 4 i + b < 16, at bit 4 + i + 8 b for
    e = 16 + 4 i + b), then the 16 header bytes per (block, row)."""
    rows, cols = 3, 512
    rng = np.random.default_rng(3)
    w = rng.integers(0, 256, size=rows * row_bytes(Q5_K, cols), dtype=np.uint8)
    slab = hl.repack_slab_host(Q5_K, w, rows, cols)
    nb, S = cols // 256, cols // 32
    for r in range(rows):
        for b in range(nb):
            blk = w[r * 352 + b * 176: r * 352 + (b + 1) * 176]
            hdr = slab[S * 64 * 16 + S * 64 * 4 + (b * 64 + r) * 16:][:16]
            assert np.array_equal(hdr, blk[:16])
            for j in range(8):
                g, hi = j // 2, j % 2
                q = blk[48 + 32 * g: 48 + 32 * g + 32]
                vals = (q >> 4) if hi else (q & 15)
                top = (blk[16:48] >> j) & 1  # fifth bit of element l of sub-block j
                rec = slab[((8 * b + j) * 64 + r) * 16:][:16]
                assert np.array_equal(rec & 15, vals[:16]) and np.array_equal(rec >> 4, vals[16:])
                word = int.from_bytes(slab[S * 64 * 16 + ((8 * b + j) * 64 + r) * 4:][:4].tobytes(), "little")
                for e in range(32):
                    i, bb = (e % 16) // 4, e % 4
                    bit = (i if e < 16 else 4 + i) + 8 * bb
                    assert (word >> bit) & 1 == top[e], (r, b, j, e)


def test_slab_byte_placement_iq4_xs(hl):
    """IQ4_XS: the block's 16-byte sub-block records are already slot records (element t low,
    t + 16 high); the 8 header bytes (d, scales_h, scales_l) per (block, row) follow."""
    rows, cols = 2, 512
    rng = np.random.default_rng(4)
    w = rng.integers(0, 256, size=rows * row_bytes(IQ4_XS, cols), dtype=np.uint8)
    slab = hl.repack_slab_host(IQ4_XS, w, rows, cols)
    nb, S = cols // 256, cols // 32
    for r in range(rows):
        for b in range(nb):
            blk = w[r * 272 + b * 136: r * 272 + (b + 1) * 136]
            assert np.array_equal(slab[S * 64 * 16 + (b * 64 + r) * 8:][:8], blk[:8])
            for j in range(8):
                assert np.array_equal(slab[((8 * b + j) * 64 + r) * 16:][:16], blk[8 + 16 * j: 24 + 16 * j])


def test_fill_normal_deterministic_and_normal(hl):
    a = hl.fill_normal(0, 1_000_001)
    b = hl.fill_normal(0, 1_000_001)
    assert np.array_equal(a, b)
    assert not np.array_equal(a[:1000], hl.fill_normal(1, 1000))
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    # seekable: a prefix is the prefix of a longer fill
    assert np.array_equal(hl.fill_normal(0, 10), a[:10])
    s = hl.fill_normal(3, 4000, 0.0, 0.02)
    assert abs(float(s.std()) - 0.02) < 2e-3


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_quantizer_round_trip_and_determinism(hl, oracle, t):
    """The repo's own quantizer (the reference ships none: parity unpinned): deterministic for
    any thread count, finite scales, and small round-trip error against the oracle's dequant."""
    be, bb = BLOCK[t]
    n = 256 * 64
    x = hl.fill_normal(11, n, 0.0, 0.02)
    q1 = hl.quantize(t, x, threads=1)
    q7 = hl.quantize(t, x, threads=7)
    assert q1.size == n // be * bb and np.array_equal(q1, q7)
    y = oracle.dequantize_row(t, q1, n)
    assert np.all(np.isfinite(y))
    err = y.astype(np.float64) - x
    rel_rms = float(np.sqrt(np.mean(err ** 2)) / np.std(x))
    limit = {Q8_0: 0.01, Q6_K: 0.04, Q5_K: 0.06, Q4_K: 0.12, IQ4_XS: 0.12, Q4_0: 0.15}[t]
    assert rel_rms < limit, rel_rms


def test_quantizer_rejects(hl):
    for t in (11, 16):  # Q3_K, IQ2_XXS: formats the quantizer does not write
        with pytest.raises(hl.HaloError) as e:
            hl.quantize(t, np.zeros(256, np.float32))
        assert e.value.code == hl.ErrorCode.Unsupported
    with pytest.raises(hl.HaloError) as e:
        hl.quantize(Q4_K, np.zeros(100, np.float32))
    assert e.value.code == hl.ErrorCode.Kernel


def test_host_repack_rejects(hl):
    with pytest.raises(hl.HaloError) as e:
        hl.repack_slab_host(11, np.zeros(110, np.uint8), 1, 256)  # Q3_K
    assert e.value.code == hl.ErrorCode.Unsupported
    with pytest.raises(hl.HaloError) as e:
        hl.repack_slab_host(Q4_K, np.zeros(144, np.uint8), 1, 100)
    assert e.value.code == hl.ErrorCode.Kernel


def test_single_hip_runtime_in_process(hl):
    """Regression: loading the library before torch used to map /opt/rocm's HIP runtime next to
    torch's bundled copy, so torch's streams reached the wrong runtime."""
    import torch  # noqa: F401

    assert len(hl._lib.hip_runtimes()) == 1
