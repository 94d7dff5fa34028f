"""GPU parity of the model-scale upload (halo_mi_upload_tensors): host GGUF rows -> SLAB images
through the pinned / copy / repack pipeline, with row-fused projections (the rows of several
parts concatenated, as try_make_fused does, src/models/qwen35.cpp:253-288). Acceptance is
bitwise: every image equals the host repack of the concatenated rows, and unpacking it gives
those bytes back.
"""
from __future__ import annotations

import numpy as np
import pytest

from helpers import IQ4_XS, NAMES, Q4_0, Q4_K, Q6_K, Q8_0, make_weights, row_bytes
from test_gpu_parity import host, say, to_dev

pytestmark = pytest.mark.gpu


def dense_rows(buf, t, rows, cols, stride, off):
    rb = row_bytes(t, cols)
    return np.concatenate([buf[off + r * stride: off + r * stride + rb] for r in range(rows)])


@pytest.mark.parametrize("chunk_slabs,threads", [(1, 1), (1, 3), (2, 0), (0, 0)])
def test_upload_tensors_fused_parts_bitwise(hl, dev, chunk_slabs, threads):
    import torch

    cols = 512
    specs = [  # (type, [(rows, stride_pad, offset), ...])
        (Q4_K, [(130, 0, 0)]),
        (Q6_K, [(70, 5, 1), (64, 0, 0), (1, 3, 2)]),  # a row-fused projection: ragged, strided parts
        (IQ4_XS, [(200, 0, 0)]),
        (Q8_0, [(33, 0, 0), (31, 7, 0)]),
        (Q4_0, [(5, 0, 0)]),
    ]
    tensors, expect, dsts, keep = [], [], [], []
    for k, (t, parts) in enumerate(specs):
        rb = row_bytes(t, cols)
        plist, dense = [], []
        for p, (rows, pad, off) in enumerate(parts):
            buf, stride = make_weights(t, rows, cols, seed=100 * k + p, stride_pad=pad, offset=off)
            keep.append(buf)
            plist.append((buf.ctypes.data + off, rows, stride))
            dense.append(dense_rows(buf, t, rows, cols, stride, off))
        total = sum(r for r, _, _ in parts)
        dense = np.concatenate(dense)
        dst = torch.full((hl.slab_bytes(t, total, cols),), 0xCD, dtype=torch.uint8, device=dev)
        tensors.append((t, cols, plist, dst))
        expect.append((t, total, dense, hl.repack_slab_host(t, dense, total, cols)))
        dsts.append(dst)
    rb_max = max(row_bytes(t, cols) for t, _ in specs)
    chunk = chunk_slabs * 64 * rb_max
    say("upload_tensors", chunk, threads)
    hl.upload_tensors(tensors, chunk_bytes=chunk, host_threads=threads)
    for (t, total, dense, slab), dst in zip(expect, dsts):
        assert np.array_equal(host(dst), slab), f"{NAMES[t]}: the uploaded image differs from the host repack"
        back = torch.zeros(total * row_bytes(t, cols), dtype=torch.uint8, device=dev)
        hl.unpack_slab(t, dst, total, cols, back)
        assert np.array_equal(host(back), dense), f"{NAMES[t]}: unpacking does not give the concatenated rows"


def test_upload_tensors_large_default_chunks(hl, dev):
    """17408 x 5120 Q4_K (50 MB) in 64 MiB chunks, compared with the device repack."""
    import torch

    t, rows, cols = Q4_K, 17408, 5120
    say("upload_tensors large", rows, cols)
    w = np.random.default_rng(5).integers(0, 256, size=rows * row_bytes(t, cols), dtype=np.uint8)
    dst = torch.zeros(hl.slab_bytes(t, rows, cols), dtype=torch.uint8, device=dev)
    hl.upload_tensors([(t, cols, [(w, rows)], dst)])
    ref = torch.zeros_like(dst)
    hl.repack_slab(t, to_dev(w, dev), rows, cols, ref)
    assert torch.equal(dst, ref)


def test_upload_tensors_rejects(hl, dev):
    import torch

    t, cols = Q4_K, 256
    w = np.zeros(64 * row_bytes(t, cols), np.uint8)
    dst = torch.zeros(hl.slab_bytes(t, 64, cols), dtype=torch.uint8, device=dev)
    with pytest.raises(hl.HaloError) as e:  # two destinations overlapping
        hl.upload_tensors([(t, cols, [(w, 64)], dst), (t, cols, [(w, 64)], dst.data_ptr() + 256)])
    assert e.value.code == hl.ErrorCode.Kernel
    with pytest.raises(hl.HaloError) as e:
        hl.upload_tensors([(11, cols, [(w, 64)], dst)])
    assert e.value.code == hl.ErrorCode.Unsupported
    with pytest.raises(hl.HaloError) as e:  # a strided part whose stride is below the row size
        hl.upload_tensors([(t, cols, [(w, 2, 10)], dst)])
    assert e.value.code == hl.ErrorCode.Kernel
