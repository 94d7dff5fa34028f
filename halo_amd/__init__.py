"""halo_amd: MI355X-native quantized matrix-multiply backend (GGUF Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K /
IQ4_XS).

The compute path is hand-written HIP for gfx950 in ``libhalo_mi355x.so``, reached through the
C ABI declared in ``include/halo_mi355x.h``. This package loads that library with ctypes and
mirrors the reference's operator interface for the path (``Backend::gemv`` over
``GemvArgs``; include/halo/backend/backend.h:283-314, :562). There is no CPU fallback: if the
library is missing every entry point raises.
"""
from __future__ import annotations

from ._lib import (  # noqa: F401
    DType,
    ErrorCode,
    HaloError,
    Layout,
    Variant,
    ARGMAX_RESULT_BYTES,
    SLAB_ROWS,
    STATUS_BAD_INDEX,
    STATUS_SPLITK_TIMEOUT,
    argmax,
    block_bytes,
    block_elems,
    dequant_rows,
    fill_normal,
    force_splitk_timeout,
    gate_up_swiglu,
    gemv,
    gemm_group,
    gemv_group,
    gemv_noalloc,
    get_rows,
    lib,
    lm_head,
    quantize,
    repack_slab,
    repack_slab_host,
    rms_norm,
    row_bytes,
    slab_bytes,
    stream_check,
    stream_read,
    stream_release,
    swiglu,
    unpack_slab,
    unpack_slab_host,
    upload_slab,
    upload_tensors,
)
