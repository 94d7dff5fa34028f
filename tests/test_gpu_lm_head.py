"""GPU parity of the LM head (halo_mi_lm_head): the gemv over the vocabulary and the fused argmax,
against the oracle's restatement of CpuBackend::lm_head (src/backend/cpu_backend.cpp:669-770).

The argmax is taken over exactly the values the GPU's gemv produces, so the GPU result must be
the first maximum of its own logits bitwise; against the CPU, the index must agree wherever the
CPU's top-2 gap exceeds twice the gemv's error bound (the reference's own criterion,
tests/unit/backend/test_hip_backend.cpp:603-636), and the value lies within that bound.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from helpers import F32, NAMES, Q4_0, Q4_K, Q6_K, Q8_0, QUANT_TYPES, gemm_tol, make_weights, row_bytes, slab_gemv_tol, synth_matrix
from test_gpu_parity import dense_of, host, say, slab_of, to_dev

pytestmark = pytest.mark.gpu

NO_INDEX = 0xFFFFFFFF
QNAN_BITS = 0x7FC00000


def _bits(v) -> int:
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def run_head(hl, dev, t, w, x, rows, cols, *, layout=None, variant=0, logits=True, valid_rows=0, ids=False,
             slots=None, scatter_len=0, w_stride=0):
    import torch

    n_vec = x.shape[0]
    res = torch.full((n_vec, 3), 0xABCD, dtype=torch.int32, device=dev)
    y = torch.full((n_vec, rows), 999.0, dtype=torch.float32, device=dev) if logits else None
    idt = torch.full((n_vec,), -7, dtype=torch.int32, device=dev) if ids else None
    sl = to_dev(np.asarray(slots, np.uint32).view(np.int32), dev) if slots is not None else None
    sc = torch.full((max(scatter_len, 1),), -7, dtype=torch.int32, device=dev) if slots is not None else None
    hl.lm_head(t, w, to_dev(x, dev), res, rows, cols, n_vec, logits=y, valid_rows=valid_rows, ids=idt, ids_slots=sl,
               ids_scatter=sc, ids_scatter_len=scatter_len, layout=hl.Layout.SLAB if layout is None else layout,
               w_stride=w_stride, variant=variant)
    out = host(res).view(np.uint32)
    return (out, host(y) if logits else None, host(idt) if ids else None, host(sc) if slots is not None else None)


def first_max(row, limit=None):
    r = row if limit is None else row[:limit]
    return int(np.argmax(r)), _bits(r.max())


@pytest.mark.parametrize("t", QUANT_TYPES)
@pytest.mark.parametrize("variant", [0, 2, 3, 5])
def test_lm_head_matches_its_logits_and_the_cpu(hl, oracle, dev, t, variant):
    rows, cols, n_vec = 1000, 512, 3
    say("lm_head", NAMES[t], rows, cols, n_vec, variant)
    buf, stride = make_weights(t, rows, cols, seed=600 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = np.random.default_rng(6000 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    res, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols, variant=variant)
    cpu, cpu_logits = oracle.lm_head(t, dense, rows, cols, x)
    gemm = variant in (3, 5)
    tol = gemm_tol(oracle, t, dense, rows, cols, x) if gemm else slab_gemv_tol(oracle, t, dense, rows, cols, x)
    assert np.all(np.abs(y.astype(np.float64) - cpu_logits) <= tol)
    for v in range(n_vec):
        idx, vbits = first_max(y[v])
        assert res[v].tolist() == [idx, vbits, 0], f"vector {v}: not the first maximum of the GPU's own logits"
        top2 = np.sort(cpu_logits[v].astype(np.float64))[-2:]
        if top2[1] - top2[0] > 2 * tol[v].max():
            assert res[v, 0] == cpu[v, 0], f"vector {v}: decisive gap but a different index"
        assert abs(float(y[v, res[v, 0]]) - float(cpu_logits[v, cpu[v, 0]])) <= 2 * tol[v].max()


@pytest.mark.parametrize("t", (Q4_K, Q6_K))
def test_lm_head_without_logits_equals_with(hl, oracle, dev, t):
    rows, cols, n_vec = 700, 1024, 6  # 6 vectors: two passes of the slab gemv
    buf, stride = make_weights(t, rows, cols, seed=610 + t)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = np.random.default_rng(6100 + t).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    with_y, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols)
    without, _, _, _ = run_head(hl, dev, t, slab, x, rows, cols, logits=False)
    assert np.array_equal(with_y, without)
    for v in range(n_vec):
        assert with_y[v].tolist() == [*first_max(y[v]), 0]


def test_lm_head_ties_on_the_slab_path_go_to_the_lowest_index(hl, oracle, dev):
    """The winning row duplicated further down (identical bytes give identical logits): the
    lower copy's index wins, in the same slab and across slabs."""
    t, rows, cols = Q6_K, 900, 512
    buf, stride = make_weights(t, rows, cols, seed=620)
    dense = dense_of(buf, t, rows, cols, stride, 0).copy()
    x = np.random.default_rng(6200).uniform(-1, 1, (1, cols)).astype(np.float32)
    _, logits = oracle.lm_head(t, dense, rows, cols, x)
    best = int(np.argmax(logits[0]))
    rb = row_bytes(t, cols)
    for dup in (best - best % 64 + (best % 64 + 7) % 64, rows - 1):  # same slab, last slab
        if dup <= best:
            continue
        d = dense.copy()
        d[dup * rb:(dup + 1) * rb] = dense[best * rb:(best + 1) * rb]
        slab = slab_of(hl, dev, t, d, rows, cols)
        res, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols)
        assert y[0, dup] == y[0, best]
        assert res[0, 0] == min(best, int(np.argmax(y[0]))) and res[0, 0] == int(np.argmax(y[0]))


def test_lm_head_gguf_reference_variant_is_bitwise_the_cpu(hl, oracle, dev):
    """Variant 1 (GGUF layout, the CPU's dot order) gives the CPU's logits bitwise, so the result
    words equal the oracle's exactly, including crafted ties, infinities and valid_rows."""
    vals = np.array([1, 5, 5, -2, np.inf, 7, np.inf, 4, 1, 2] * 30, np.float32)
    rows, cols = vals.size, 8
    w = np.zeros((rows, cols), np.float32)
    w[:, 0] = vals
    x = np.zeros((2, cols), np.float32)
    x[:, 0] = 1
    x[1, 0] = -1
    wd = to_dev(w.view(np.uint8).ravel(), dev)
    for vr in (0, 4, 6, 297):
        res, _, _, _ = run_head(hl, dev, F32, wd, x, rows, cols, layout=hl.Layout.GGUF, variant=1, valid_rows=vr)
        cpu, _ = oracle.lm_head(F32, w.view(np.uint8).ravel(), rows, cols, x, valid_rows=vr)
        assert np.array_equal(res, cpu), f"valid_rows={vr}: {res.tolist()} vs {cpu.tolist()}"
    t = Q4_K
    buf, stride = make_weights(t, 333, 256, seed=630, stride_pad=5, offset=3)
    xq = np.random.default_rng(6300).uniform(-1, 1, (4, 256)).astype(np.float32)
    dense = dense_of(buf, t, 333, 256, stride, 3)
    # padded GGUF rows (stride = row bytes + 5), starting 3 bytes into the buffer
    res, _, _, _ = run_head(hl, dev, t, to_dev(np.ascontiguousarray(buf[3:]), dev), xq, 333, 256,
                            layout=hl.Layout.GGUF, variant=1, w_stride=stride)
    assert np.array_equal(res, oracle.lm_head(t, dense, 333, 256, xq)[0])


@pytest.mark.parametrize("variant", [0, 3])
def test_lm_head_nan_poisons_only_its_vector(hl, oracle, dev, variant):
    t, rows, cols, n_vec = Q4_K, 400, 512, 4
    buf, stride = make_weights(t, rows, cols, seed=640)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = np.random.default_rng(6400).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    x[2, 100] = np.nan
    slab = slab_of(hl, dev, t, dense, rows, cols)
    res, y, ids, _ = run_head(hl, dev, t, slab, x, rows, cols, variant=variant, ids=True)
    assert res[2].tolist() == [NO_INDEX, QNAN_BITS, 1]
    assert ids[2] == 0
    for v in (0, 1, 3):
        assert res[v].tolist() == [*first_max(y[v]), 0]
        assert ids[v] == res[v, 0]


@pytest.mark.parametrize("variant", [0, 5])
def test_lm_head_valid_rows_clamps_the_argmax_not_the_logits(hl, oracle, dev, variant):
    t, rows, cols, n_vec = Q6_K, 1000, 512, 2
    buf, stride = make_weights(t, rows, cols, seed=650)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = np.random.default_rng(6500).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    slab = slab_of(hl, dev, t, dense, rows, cols)
    _, y_all, _, _ = run_head(hl, dev, t, slab, x, rows, cols, variant=variant)
    for vr in (1, 37, 64, 65, 999, 1000, 5000):
        res, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols, variant=variant, valid_rows=vr)
        assert np.array_equal(y, y_all), "valid_rows changed the logits"
        for v in range(n_vec):
            assert res[v].tolist() == [*first_max(y[v], min(vr, rows)), 0], f"valid_rows={vr}"


def test_lm_head_ids_and_scattered_ids(hl, oracle, dev):
    t, rows, cols, n_vec = Q4_0, 300, 256, 3
    buf, stride = make_weights(t, rows, cols, seed=660)
    dense = dense_of(buf, t, rows, cols, stride, 0)
    x = np.random.default_rng(6600).uniform(-1, 1, (n_vec, cols)).astype(np.float32)
    x[1, 0] = np.nan
    slab = slab_of(hl, dev, t, dense, rows, cols)
    res, _, ids, sc = run_head(hl, dev, t, slab, x, rows, cols, ids=True, slots=[4, 0, 9], scatter_len=6)
    assert ids.tolist() == [int(res[0, 0]), 0, int(res[2, 0])]
    # slot 4 <- vector 0, slot 0 <- vector 1 (poisoned: 0), slot 9 is past the 6 elements: dropped
    assert sc.tolist() == [0, -7, -7, -7, int(res[0, 0]), -7]


def test_lm_head_rejects_bad_arguments(hl, dev):
    import torch

    t, rows, cols = Q4_K, 64, 256
    slab = torch.zeros(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device=dev)
    x = torch.zeros((1, cols), dtype=torch.float32, device=dev)
    res = torch.zeros((1, 3), dtype=torch.int32, device=dev)
    ids = torch.zeros(1, dtype=torch.int32, device=dev)

    def code(**kw):
        args = dict(logits=None, variant=0)
        args.update(kw)
        try:
            hl.lm_head(t, slab, x, res, rows, cols, 1, **args)
        except hl.HaloError as e:
            return e.code
        return 0

    assert code() == 0
    assert code(variant=3) == hl.ErrorCode.Kernel  # the GEMM ranks the logits: y needed
    assert code(variant=10) == hl.ErrorCode.Config  # past the last id
    assert code(ids_slots=ids, ids_scatter=ids, ids_scatter_len=1) == hl.ErrorCode.Kernel  # without ids
    assert code(ids=res) == hl.ErrorCode.Kernel  # ids overlaps result
    with pytest.raises(hl.HaloError):
        hl.lm_head(t, slab, x, None, rows, cols, 1)


def test_baseline_q6_k_lm_head(hl, oracle, dev):
    """BASELINE config 3b: the 151936 x 5120 Q6_K head (1% of columns x8) at M = 1, fused
    argmax without keeping the logits; the index agrees with the CPU where the top-2 gap is
    decisive, and always with the first maximum of the GPU's logits."""
    t, rows, cols = Q6_K, 151936, 5120
    say("baseline lm_head", rows, cols)
    wq = synth_matrix(hl, t, rows, cols, 3, outlier_cols=0.01)
    x = hl.fill_normal(1003, cols).reshape(1, cols)
    slab = slab_of(hl, dev, t, wq, rows, cols)
    res_fused, _, _, _ = run_head(hl, dev, t, slab, x, rows, cols, logits=False)
    res, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols)
    assert np.array_equal(res_fused, res)
    assert res[0].tolist() == [*first_max(y[0]), 0]
    cpu, cpu_logits = oracle.lm_head(t, wq, rows, cols, x)
    top = np.argsort(cpu_logits[0])[-2:]
    rb = row_bytes(t, cols)
    cand = np.unique(np.concatenate([top, [res[0, 0]]]))
    tol = np.concatenate([slab_gemv_tol(oracle, t, wq[r * rb:(r + 1) * rb], 1, cols, x)[0] for r in cand])
    gap = float(cpu_logits[0, top[1]]) - float(cpu_logits[0, top[0]])
    print(f"    head: gpu {res[0, 0]} cpu {cpu[0, 0]} top-2 gap {gap:.3e} bound {tol.max():.3e}")
    if gap > 2 * tol.max():
        assert res[0, 0] == cpu[0, 0]
    assert abs(float(y[0, res[0, 0]]) - float(cpu_logits[0, cpu[0, 0]])) <= 2 * tol.max()


@pytest.mark.parametrize("n_vec", [1, 4])
def test_real_vocab_q6_k_lm_head(hl, oracle, dev, n_vec):
    """The model's own vocabulary: the 248320 x 5120 Q6_K head (1.04 GB; process.md:662 of the
    reference) at M = 1 and 4. Every logit against the CPU within the gemv bound; the fused
    argmax without logits equals the one with them, and is the first maximum of the GPU's own
    logits; the index agrees with the CPU's wherever the CPU's top-2 gap is decisive."""
    import torch

    t, rows, cols = Q6_K, 248320, 5120
    say("real-vocabulary lm_head", rows, cols, n_vec)
    key = ("real_vocab",)
    if key not in _REAL:
        wq = synth_matrix(hl, t, rows, cols, 8, outlier_cols=0.01)
        _REAL.clear()
        _REAL[key] = (wq, slab_of(hl, dev, t, wq, rows, cols))
    wq, slab = _REAL[key]
    x = hl.fill_normal(1800 + n_vec, n_vec * cols).reshape(n_vec, cols)
    res_fused, _, _, _ = run_head(hl, dev, t, slab, x, rows, cols, logits=False)
    res, y, _, _ = run_head(hl, dev, t, slab, x, rows, cols)
    assert np.array_equal(res_fused, res), "the argmax changed with the logits kept"
    ref = oracle.matmul(t, wq, rows, cols, x)
    tol = slab_gemv_tol(oracle, t, wq, rows, cols, x)
    err = np.abs(y.astype(np.float64) - ref)
    print(f"    real-vocabulary head M={n_vec}: worst |d|/bound = {float(np.max(err / tol)):.4f}")
    assert np.all(err <= tol)
    for v in range(n_vec):
        assert res[v].tolist() == [*first_max(y[v]), 0], f"vector {v}: not the first maximum of its own logits"
        top2 = np.sort(ref[v])[-2:]
        if top2[1] - top2[0] > 2 * tol[v].max():
            assert res[v, 0] == int(np.argmax(ref[v])), f"vector {v}: decisive gap but a different index"
    if n_vec == 4:
        _REAL.clear()
        torch.cuda.empty_cache()


_REAL = {}
