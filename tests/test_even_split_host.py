"""The even split's integer divisions (halo_amd/csrc/gemv_device.h: udiv_inv, even_wg), restated
in numpy float32 and checked against exact integer division over every operand the host admits.

The kernel divides with a float reciprocal the host computes (1.0f / d) and corrects the quotient
by one step; that is exact only if the float quotient is within one of x / d. pick_even admits a
launch when G = slabs x matrices x slot groups lies in [4096, 8192] (at least kEvenMinGroups, and
at most 16 units per share of 512 workgroups), so the kernel's operands are:
  - seg_of(u) = u / ngrp for u < G, ngrp <= G (and the publishing workgroup's (i + 1) G / 512 < G);
  - even_wg(u) = ((u + 1) 512 - 1) / G for u < G.
Both are checked here for every d and every x in those ranges (no GPU).
"""
from __future__ import annotations

import numpy as np

K_EVEN_W = 512
G_MIN, G_MAX = 4096, 8192


def udiv_inv(x: np.ndarray, d: int, inv: np.float32) -> np.ndarray:
    """gemv_device.h udiv_inv: q = (uint32)((float)x * inv), then one correction step."""
    xf = x.astype(np.float32)
    q = (xf * inv).astype(np.uint32)  # v_cvt_f32_u32 (RNE), v_mul_f32, v_cvt_u32_f32 (truncation)
    r = x.astype(np.int64) - q.astype(np.int64) * d
    return np.where(r < 0, q - 1, np.where(r >= d, q + 1, q)).astype(np.uint32)


def host_inv(d: int) -> np.float32:
    """k_gemv.hip: 1.0f / (float)d on the host (correctly rounded float division)."""
    return np.float32(1.0) / np.float32(d)


def test_segment_division_every_divisor():
    x = np.arange(G_MAX, dtype=np.uint32)
    for d in range(1, G_MAX + 1):
        got = udiv_inv(x, d, host_inv(d))
        assert np.array_equal(got, x // d), f"u / {d}"


def test_workgroup_of_unit_every_launch_size():
    u = np.arange(G_MAX, dtype=np.uint64)
    for g in range(G_MIN, G_MAX + 1):
        x = ((u[:g] + 1) * K_EVEN_W - 1).astype(np.uint32)
        got = udiv_inv(x, g, host_inv(g))
        assert np.array_equal(got, x // g), f"even_wg over G = {g}"
        # the shares [b G / W, (b + 1) G / W) hold every unit once, in order
        assert got[0] == 0 and got[-1] == K_EVEN_W - 1 and np.all(np.diff(got.astype(np.int64)) >= 0)


def test_correction_is_needed():
    """The uncorrected float quotient is off by one for some admitted operands (so the
    correction step is what makes the division exact, and a restatement without it would fail)."""
    misses = 0
    x = np.arange(G_MAX, dtype=np.uint32)
    for d in range(1, G_MAX + 1):
        q = (x.astype(np.float32) * host_inv(d)).astype(np.uint32)
        misses += int(np.count_nonzero(q != x // d))
    assert misses > 0
