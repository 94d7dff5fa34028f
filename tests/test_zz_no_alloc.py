"""halo_mi_gemv_noalloc (the slab GEMV over the library's device-resident scratch) against
halo_mi_gemv, through the C ABI: bitwise equal outputs on two calls in a row, the second on a
smaller input, with nothing allocated on the device by the calls; shapes and variants past the
scratch are refused.

Runs in a fresh process on its own and after the other tests (it makes its own stream, so the
other tests' workspaces do not matter).
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import NAMES, Q4_K, Q6_K, isclose_bits, make_weights
from test_gpu_parity import SENTINEL, dense_of, host, say, slab_of, to_dev

pytestmark = pytest.mark.gpu


def _case(hl, dev, t, rows, cols, seed):
    buf, stride = make_weights(t, rows, cols, seed=seed)
    return slab_of(hl, dev, t, dense_of(buf, t, rows, cols, stride, 0), rows, cols)


def test_noalloc_matches_gemv_bitwise_and_allocates_nothing(hl, dev):
    import torch

    # first call: 17408 x 5120 Q4_K (272 slabs over the even split's 512 workgroups), 3 vectors
    # with the fused norm; then
    # smaller inputs on the same scratch: the auto ids 4 and 0 where their choice is the slab
    # GEMV (Q6_K at 4 and 3 vectors; a Q4_K matrix of 96 slabs at 4), and a single vector
    calls = [(Q4_K, 17408, 5120, 3, True, 2), (Q6_K, 5120, 6144, 4, False, 4), (Q4_K, 6144, 5120, 4, True, 0),
             (Q6_K, 5120, 6144, 3, False, 0), (Q6_K, 5120, 6144, 1, False, 0)]
    mats = {(t, rows, cols): _case(hl, dev, t, rows, cols, 2100 + rows) for t, rows, cols, _, _, _ in calls}
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):  # the runtime's own lazy set-up of a new stream (first launch, first copy)
        torch.zeros(1, device=dev).add_(1).cpu()
    torch.cuda.synchronize()
    for i, (t, rows, cols, n_vec, norm, variant) in enumerate(calls):
        say("gemv_noalloc", i, NAMES[t], rows, cols, n_vec, "norm" if norm else "")
        rng = np.random.default_rng(2200 + i)
        x = to_dev((rng.standard_normal((n_vec, cols)) * 2).astype(np.float32), dev)
        nw = to_dev(rng.uniform(0.5, 1.5, cols).astype(np.float32), dev) if norm else None
        w = mats[(t, rows, cols)]
        y = torch.full((n_vec, rows + 1), SENTINEL, dtype=torch.float32, device=dev)
        ref = torch.full((n_vec, rows + 1), SENTINEL, dtype=torch.float32, device=dev)
        # the existing entry point first, on the default stream: it also has the runtime load the
        # library's GEMV code object (its code and the scratch array), which is no allocation of
        # the call under test
        hl.gemv(t, w, x, ref, rows, cols, n_vec, y_stride=rows + 1, variant=variant, norm_w=nw)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        with torch.cuda.stream(s):
            hl.gemv_noalloc(t, w, x, y, rows, cols, n_vec, y_stride=rows + 1, variant=variant, norm_w=nw)
            s.synchronize()
            free1 = torch.cuda.mem_get_info()[0]
            hl.stream_check()
        # halo_mi_gemv's first call on a stream allocates its ~116 MiB workspace
        assert free0 - free1 < (2 << 20), f"the no-alloc call took {(free0 - free1) >> 20} MiB of device memory"
        yh, rh = host(y), host(ref)
        assert np.all(yh[:, rows:] == SENTINEL), "y padding written"
        assert isclose_bits(yh, rh), f"call {i}: halo_mi_gemv_noalloc differs from halo_mi_gemv"
        assert np.all(np.isfinite(yh[:, :rows]))


def test_noalloc_refuses_what_does_not_fit(hl, dev):
    import torch

    t, rows, cols = Q4_K, 64, 256
    w = _case(hl, dev, t, rows, cols, 2300)
    x = to_dev(np.ones((16, cols), np.float32), dev)
    y = torch.zeros((16, rows), dtype=torch.float32, device=dev)
    for variant, n_vec in ((hl.Variant.SLAB_GEMM_BF16, 1), (hl.Variant.DEFAULT, 16), (hl.Variant.SLAB_GEMM_BF16_M512, 2),
                           (hl.Variant.SLAB_GEMM_EXACT_INVARIANT, 1)):
        with pytest.raises(hl.HaloError) as e:  # the GEMM's staging does not fit the scratch
            hl.gemv_noalloc(t, w, x, y, rows, cols, n_vec, variant=variant)
        assert e.value.code == hl.ErrorCode.Unsupported
    # the auto ids where halo_mi_gemv's choice is the exact small-M GEMM (17408 x 5120 Q4_K at
    # 3..8 vectors): refused, since that kernel's partials do not fit the scratch and the slab
    # GEMV would not be bitwise what halo_mi_gemv returns
    big = _case(hl, dev, t, 17408, 5120, 2301)
    xs = to_dev(np.ones((8, 5120), np.float32), dev)
    ys = torch.full((8, 17408), SENTINEL, dtype=torch.float32, device=dev)
    for variant in (hl.Variant.DEFAULT, hl.Variant.SLAB_AUTO):
        for n_vec in (3, 5, 8):
            with pytest.raises(hl.HaloError) as e:
                hl.gemv_noalloc(t, big, xs, ys, 17408, 5120, n_vec, variant=variant)
            assert e.value.code == hl.ErrorCode.Unsupported
    assert np.all(host(ys) == SENTINEL), "a refused call wrote its output"
    with pytest.raises(hl.HaloError) as e:  # y overlapping x: the same checks as halo_mi_gemv
        hl.gemv_noalloc(t, w, x, x, rows, cols, 1)
    assert e.value.code == hl.ErrorCode.Kernel
    # 1000 slabs at K = 8448 split into 5 K chunks: 1000 * 5 * 4 * 64 words, past the scratch's
    # 2^20 (halo_mi_gemv takes it). Real buffers of that size (zero blocks), so nothing out of
    # bounds could be read even if the call were not refused.
    big_rows, big_cols = 64000, 8448
    wb = torch.zeros(hl.slab_bytes(t, big_rows, big_cols), dtype=torch.uint8, device=dev)
    xb = torch.ones((1, big_cols), dtype=torch.float32, device=dev)
    yb = torch.full((1, big_rows), SENTINEL, dtype=torch.float32, device=dev)
    with pytest.raises(hl.HaloError) as e:
        hl.gemv_noalloc(t, wb, xb, yb, big_rows, big_cols, 1, variant=hl.Variant.SLAB_GEMV)
    assert e.value.code == hl.ErrorCode.Unsupported
    assert np.all(host(yb) == SENTINEL), "a refused call wrote its output"
    hl.gemv(t, wb, xb, yb, big_rows, big_cols, 1, variant=hl.Variant.SLAB_GEMV)
    assert np.all(host(yb) == 0.0)
