"""ctypes bindings of libhalo_mi355x.so (the C ABI in include/halo_mi355x.h).

Pointer arguments are plain integers (device addresses, e.g. ``tensor.data_ptr()``) and
``stream`` is a hipStream_t as an integer (0 = null stream). Functions taking torch tensors
validate dtype/device and pass ``torch.cuda.current_stream()`` unless a stream is given.
"""
from __future__ import annotations

import ctypes
import enum
import functools
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_LIB_PATH = _PKG / "libhalo_mi355x.so"

SLAB_ROWS = 64


class DType(enum.IntEnum):
    """ggml type ids (include/halo/tensor/dtype.h:18-49 of the reference)."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ4_NL = 20
    IQ3_S = 21
    IQ4_XS = 23
    BF16 = 30


class Layout(enum.IntEnum):
    GGUF = 0
    SLAB = 1


class Variant(enum.IntEnum):
    DEFAULT = 0
    GGUF_REF = 1
    SLAB_GEMV = 2
    SLAB_GEMM_BF16 = 3
    SLAB_AUTO = 4
    SLAB_GEMM_BF16_M512 = 5
    SLAB_GEMV_VALU = 6
    SLAB_GEMM_BF16_SMALL_M = 7
    SLAB_GEMM_EXACT_SMALL_M = 8
    SLAB_GEMM_EXACT_INVARIANT = 9


class ErrorCode(enum.IntEnum):
    """Status codes; names follow halo::ErrorCode (include/halo/core/error.h:13-24)."""

    Ok = 0
    Kernel = 1
    Unsupported = 2
    Config = 3
    Memory = 4
    Device = 5


class HaloError(RuntimeError):
    def __init__(self, code: int, message: str):
        self.code = ErrorCode(code)
        super().__init__(f"{self.code.name.upper()}_ERROR: {message}")


_BLOCK = {DType.F32: (1, 4), DType.F16: (1, 2), DType.BF16: (1, 2), DType.Q4_0: (32, 18), DType.Q4_1: (32, 20),
          DType.Q5_0: (32, 22), DType.Q5_1: (32, 24), DType.Q8_0: (32, 34), DType.Q2_K: (256, 84),
          DType.Q3_K: (256, 110), DType.Q4_K: (256, 144), DType.Q5_K: (256, 176), DType.Q6_K: (256, 210),
          DType.IQ4_NL: (32, 18), DType.IQ3_S: (256, 110), DType.IQ4_XS: (256, 136)}


def block_elems(t: int) -> int:
    """Weights per block; 0 for a type this backend does not handle."""
    return _BLOCK.get(int(t), (0, 0))[0]


def block_bytes(t: int) -> int:
    return _BLOCK.get(int(t), (0, 0))[1]


class _GemvParams(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_uint32),
        ("layout", ctypes.c_uint32),
        ("w", ctypes.c_void_p),
        ("w_stride", ctypes.c_uint64),
        ("x", ctypes.c_void_p),
        ("x_stride", ctypes.c_uint64),
        ("y", ctypes.c_void_p),
        ("y_stride", ctypes.c_uint64),
        ("rows", ctypes.c_uint32),
        ("cols", ctypes.c_uint32),
        ("n_vec", ctypes.c_uint32),
        ("variant", ctypes.c_uint32),
        ("norm_w", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
    ]


class _GateUpParams(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_uint32),
        ("layout", ctypes.c_uint32),
        ("w_gate", ctypes.c_void_p),
        ("w_up", ctypes.c_void_p),
        ("x", ctypes.c_void_p),
        ("x_stride", ctypes.c_uint64),
        ("out", ctypes.c_void_p),
        ("out_stride", ctypes.c_uint64),
        ("rows", ctypes.c_uint32),
        ("cols", ctypes.c_uint32),
        ("n_vec", ctypes.c_uint32),
        ("variant", ctypes.c_uint32),
        ("norm_w", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
    ]


class _GemvSegment(ctypes.Structure):
    _fields_ = [("type", ctypes.c_uint32), ("w", ctypes.c_void_p), ("rows", ctypes.c_uint32), ("y", ctypes.c_void_p),
                ("y_stride", ctypes.c_uint64)]


class _GemvGroupParams(ctypes.Structure):
    _fields_ = [
        ("segs", ctypes.POINTER(_GemvSegment)),
        ("n_segs", ctypes.c_uint32),
        ("x", ctypes.c_void_p),
        ("x_stride", ctypes.c_uint64),
        ("cols", ctypes.c_uint32),
        ("n_vec", ctypes.c_uint32),
        ("norm_w", ctypes.c_void_p),
        ("norm_eps", ctypes.c_float),
    ]


class _LmHeadParams(ctypes.Structure):
    _fields_ = [
        ("gemv", _GemvParams),
        ("result", ctypes.c_void_p),
        ("valid_rows", ctypes.c_uint32),
        ("ids", ctypes.c_void_p),
        ("ids_slots", ctypes.c_void_p),
        ("ids_scatter", ctypes.c_void_p),
        ("ids_scatter_len", ctypes.c_uint64),
    ]


class _UploadPart(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("src_stride", ctypes.c_uint64), ("rows", ctypes.c_uint32)]


class _UploadTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_uint32),
        ("cols", ctypes.c_uint32),
        ("parts", ctypes.POINTER(_UploadPart)),
        ("n_parts", ctypes.c_uint32),
        ("dst", ctypes.c_void_p),
    ]


class _GetRowsParams(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_uint32),
        ("layout", ctypes.c_uint32),
        ("table", ctypes.c_void_p),
        ("table_stride", ctypes.c_uint64),
        ("n_rows", ctypes.c_uint32),
        ("cols", ctypes.c_uint32),
        ("ids", ctypes.c_void_p),
        ("n_ids", ctypes.c_uint32),
        ("out", ctypes.c_void_p),
        ("out_stride", ctypes.c_uint64),
        ("status", ctypes.c_void_p),
        ("status_keep", ctypes.c_uint32),
    ]


ARGMAX_RESULT_BYTES = 12  # HALO_MI_ARGMAX_RESULT_BYTES: {index, value bits, poisoned} per vector
STATUS_BAD_INDEX = 8  # HALO_MI_STATUS_BAD_INDEX: a GET_ROWS id outside the table
STATUS_SPLITK_TIMEOUT = 0x100  # HALO_MI_STATUS_SPLITK_TIMEOUT: a split-K reduction gave up waiting


# Every symbol include/halo_mi355x.h declares, with its ctypes signature.
_U32, _U64, _VP, _INT = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_int
SIGNATURES = {
    "halo_mi_last_error": (ctypes.c_char_p, []),
    "halo_mi_gemv": (_INT, [ctypes.POINTER(_GemvParams), _VP]),
    "halo_mi_gemv_noalloc": (_INT, [ctypes.POINTER(_GemvParams), _VP]),
    "halo_mi_gemv_group": (_INT, [ctypes.POINTER(_GemvGroupParams), _VP]),
    "halo_mi_gemm_group": (_INT, [ctypes.POINTER(_GemvGroupParams), _VP]),
    "halo_mi_gate_up_swiglu": (_INT, [ctypes.POINTER(_GateUpParams), _VP]),
    "halo_mi_lm_head": (_INT, [ctypes.POINTER(_LmHeadParams), _VP]),
    "halo_mi_argmax": (_INT, [_VP, _U64, _U32, _U32, _VP, _VP]),
    "halo_mi_swiglu": (_INT, [_VP, _U64, _VP, _U64, _VP, _U64, _U32, _U32, _VP]),
    "halo_mi_dequant_rows": (_INT, [_U32, _U32, _VP, _U64, _U32, _U32, _U32, _U32, _VP, _U64, _VP]),
    "halo_mi_get_rows": (_INT, [ctypes.POINTER(_GetRowsParams), _VP]),
    "halo_mi_rms_norm": (_INT, [_VP, _U64, _VP, _VP, _U64, _U32, _U32, ctypes.c_float, _VP]),
    "halo_mi_stream_read": (_INT, [_VP, _U64, _U32, _U32, _VP, _VP]),
    "halo_mi_stream_check": (_INT, [_VP]),
    "halo_mi_stream_release": (_INT, [_VP]),
    "halo_mi_test_splitk_timeout": (_INT, [_U32, _INT]),
    "halo_mi_row_bytes": (_U64, [_U32, _U32]),
    "halo_mi_slab_bytes": (_U64, [_U32, _U32, _U32]),
    "halo_mi_repack_slab": (_INT, [_U32, _VP, _U64, _U32, _U32, _VP, _VP]),
    "halo_mi_unpack_slab": (_INT, [_U32, _VP, _U32, _U32, _VP, _U64, _VP]),
    "halo_mi_repack_slab_host": (_INT, [_U32, _VP, _U64, _U32, _U32, _VP]),
    "halo_mi_unpack_slab_host": (_INT, [_U32, _VP, _U32, _U32, _VP, _U64]),
    "halo_mi_upload_slab": (_INT, [_U32, _VP, _U64, _U32, _U32, _VP, _U64, _VP]),
    "halo_mi_upload_tensors": (_INT, [ctypes.POINTER(_UploadTensor), _U32, _U64, _U32, _VP]),
    "halo_mi_fill_normal": (None, [_U64, _VP, _U64, ctypes.c_float, ctypes.c_float]),
    "halo_mi_quantize": (_INT, [_U32, _VP, _U64, _VP, _U32]),
}


def hip_runtimes() -> list[str]:
    """Paths of the HIP runtime libraries mapped into this process."""
    with open("/proc/self/maps") as f:
        return sorted({line.split()[-1] for line in f if "libamdhip64" in line})


@functools.lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    """The loaded library. Raises (never falls back) when it has not been built.

    The process must hold exactly one HIP runtime. torch bundles its own libamdhip64 (soname
    libamdhip64.so.7, but its own libraries ask for it as "libamdhip64.so"), so if this library
    were loaded first it would pull in /opt/rocm's copy and a later torch import would load a
    second one: torch's streams and allocations would then reach the wrong runtime. Importing
    torch first makes this library bind to torch's runtime by soname.
    """
    if not _LIB_PATH.exists():
        raise RuntimeError(f"{_LIB_PATH} is missing: build it with `python -m halo_amd.build` (hipcc, gfx950)")
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    so = ctypes.CDLL(str(_LIB_PATH))
    runtimes = hip_runtimes()
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes are loaded in this process: {runtimes}")
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    return so


def _check(rc: int) -> None:
    if rc != 0:
        raise HaloError(rc, lib().halo_mi_last_error().decode())


def _ptr(t) -> int:
    if t is None:
        return 0
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int:
    if stream is not None:
        return int(stream)
    import torch

    return torch.cuda.current_stream().cuda_stream


# ---- geometry ---------------------------------------------------------------------------


def row_bytes(t: int, cols: int) -> int:
    return int(lib().halo_mi_row_bytes(int(t), int(cols)))


def slab_bytes(t: int, rows: int, cols: int) -> int:
    return int(lib().halo_mi_slab_bytes(int(t), int(rows), int(cols)))


# ---- host utilities ---------------------------------------------------------------------


def fill_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0):
    """SplitMix64 + Box-Muller normal fill (portable, seed-determined), as a float32 numpy array."""
    import numpy as np

    out = np.empty(int(n), dtype=np.float32)
    lib().halo_mi_fill_normal(int(seed), out.ctypes.data, int(n), float(mean), float(std))
    return out


def quantize(t: int, src, threads: int = 0):
    """fp32 numpy array (size a multiple of the block) -> GGUF block bytes (numpy uint8)."""
    import numpy as np

    src = np.ascontiguousarray(src, dtype=np.float32)
    be, bb = block_elems(t), block_bytes(t)
    out = np.empty(src.size // be * bb if be and src.size % be == 0 else 1, dtype=np.uint8)
    _check(lib().halo_mi_quantize(int(t), src.ctypes.data, src.size, out.ctypes.data, int(threads)))
    return out


def repack_slab_host(t: int, src, rows: int, cols: int, src_stride: int = 0):
    import numpy as np

    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(slab_bytes(t, rows, cols), dtype=np.uint8)
    _check(lib().halo_mi_repack_slab_host(int(t), src.ctypes.data, int(src_stride), int(rows), int(cols), out.ctypes.data))
    return out


def unpack_slab_host(t: int, src, rows: int, cols: int):
    import numpy as np

    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * row_bytes(t, cols), dtype=np.uint8)
    _check(lib().halo_mi_unpack_slab_host(int(t), src.ctypes.data, int(rows), int(cols), out.ctypes.data, 0))
    return out


# ---- device entry points (torch tensors or raw device addresses) -------------------------


def gemv(t: int, w, x, y, rows: int, cols: int, n_vec: int, *, layout: int = Layout.SLAB, w_stride: int = 0,
         x_stride: int = 0, y_stride: int = 0, variant: int = Variant.DEFAULT, norm_w=None, norm_eps: float = 1e-6,
         stream=None) -> None:
    """y = W x (halo_mi_gemv); with norm_w, y = W (rms_norm(x) * norm_w), eps = norm_eps."""
    p = _GemvParams(int(t), int(layout), _ptr(w), int(w_stride), _ptr(x), int(x_stride), _ptr(y), int(y_stride),
                    int(rows), int(cols), int(n_vec), int(variant), _ptr(norm_w), float(norm_eps))
    _check(lib().halo_mi_gemv(ctypes.byref(p), _stream(stream)))


def gemv_noalloc(t: int, w, x, y, rows: int, cols: int, n_vec: int, *, x_stride: int = 0, y_stride: int = 0,
                 variant: int = Variant.DEFAULT, norm_w=None, norm_eps: float = 1e-6, stream=None) -> None:
    """halo_mi_gemv_noalloc: the SLAB GEMV over the library's device-resident scratch (no allocation)."""
    p = _GemvParams(int(t), int(Layout.SLAB), _ptr(w), 0, _ptr(x), int(x_stride), _ptr(y), int(y_stride), int(rows),
                    int(cols), int(n_vec), int(variant), _ptr(norm_w), float(norm_eps))
    _check(lib().halo_mi_gemv_noalloc(ctypes.byref(p), _stream(stream)))


def _group_params(segs, x, cols, n_vec, x_stride, norm_w, norm_eps):
    arr = (_GemvSegment * len(segs))()
    for i, seg in enumerate(segs):
        t, w, rows, y = seg[:4]
        arr[i] = _GemvSegment(int(t), _ptr(w), int(rows), _ptr(y), int(seg[4]) if len(seg) > 4 else 0)
    # the segment array is kept alive with the params (ctypes keeps the reference)
    return _GemvGroupParams(arr, len(segs), _ptr(x), int(x_stride), int(cols), int(n_vec), _ptr(norm_w), float(norm_eps))


def gemv_group(segs, x, cols: int, n_vec: int, *, x_stride: int = 0, norm_w=None, norm_eps: float = 1e-6,
               stream=None) -> None:
    """Grouped GEMV (halo_mi_gemv_group): segs is a list of (type, w, rows, y) or (type, w, rows, y,
    y_stride), SLAB matrices that share x; one launch per pair of weight types."""
    p = _group_params(segs, x, cols, n_vec, x_stride, norm_w, norm_eps)
    _check(lib().halo_mi_gemv_group(ctypes.byref(p), _stream(stream)))


def gemm_group(segs, x, cols: int, n_vec: int, *, x_stride: int = 0, norm_w=None, norm_eps: float = 1e-6,
               stream=None) -> None:
    """Grouped bf16 GEMM (halo_mi_gemm_group): the segments of gemv_group on the bf16 MFMA GEMM,
    x staged once, one launch per pair of weight types."""
    p = _group_params(segs, x, cols, n_vec, x_stride, norm_w, norm_eps)
    _check(lib().halo_mi_gemm_group(ctypes.byref(p), _stream(stream)))


def gate_up_swiglu(t: int, w_gate, w_up, x, out, rows: int, cols: int, n_vec: int, *, layout: int = Layout.SLAB,
                   x_stride: int = 0, out_stride: int = 0, variant: int = Variant.DEFAULT, norm_w=None,
                   norm_eps: float = 1e-6, stream=None) -> None:
    p = _GateUpParams(int(t), int(layout), _ptr(w_gate), _ptr(w_up), _ptr(x), int(x_stride), _ptr(out), int(out_stride),
                      int(rows), int(cols), int(n_vec), int(variant), _ptr(norm_w), float(norm_eps))
    _check(lib().halo_mi_gate_up_swiglu(ctypes.byref(p), _stream(stream)))


def lm_head(t: int, w, x, result, rows: int, cols: int, n_vec: int, *, logits=None, valid_rows: int = 0, ids=None,
            ids_slots=None, ids_scatter=None, ids_scatter_len: int = 0, layout: int = Layout.SLAB, w_stride: int = 0,
            x_stride: int = 0, y_stride: int = 0, variant: int = Variant.DEFAULT, norm_w=None, norm_eps: float = 1e-6,
            stream=None) -> None:
    """The gemv over the vocabulary and the fused argmax (halo_mi_lm_head): result receives
    n_vec triples {index, value bits, poisoned} as uint32; logits (optional) every row."""
    g = _GemvParams(int(t), int(layout), _ptr(w), int(w_stride), _ptr(x), int(x_stride), _ptr(logits), int(y_stride),
                    int(rows), int(cols), int(n_vec), int(variant), _ptr(norm_w), float(norm_eps))
    p = _LmHeadParams(g, _ptr(result), int(valid_rows), _ptr(ids), _ptr(ids_slots), _ptr(ids_scatter),
                      int(ids_scatter_len))
    _check(lib().halo_mi_lm_head(ctypes.byref(p), _stream(stream)))


def argmax(logits, result, n: int, n_vec: int, *, logits_stride: int = 0, stream=None) -> None:
    """ARGMAX (halo_mi_argmax): result receives n_vec triples {index, value bits, poisoned}."""
    _check(lib().halo_mi_argmax(_ptr(logits), int(logits_stride), int(n), int(n_vec), _ptr(result), _stream(stream)))


def swiglu(gate, up, out, rows: int, cols: int, *, gate_stride: int = 0, up_stride: int = 0, out_stride: int = 0,
           stream=None) -> None:
    _check(lib().halo_mi_swiglu(_ptr(gate), int(gate_stride), _ptr(up), int(up_stride), _ptr(out), int(out_stride),
                                int(rows), int(cols), _stream(stream)))


def dequant_rows(t: int, layout: int, w, rows: int, cols: int, out, *, first_row: int = 0, n_rows: int | None = None,
                 w_stride: int = 0, out_stride: int = 0, stream=None) -> None:
    n = rows - first_row if n_rows is None else n_rows
    _check(lib().halo_mi_dequant_rows(int(t), int(layout), _ptr(w), int(w_stride), int(rows), int(cols), int(first_row),
                                      int(n), _ptr(out), int(out_stride), _stream(stream)))


def get_rows(t: int, layout: int, table, n_rows: int, cols: int, ids, n_ids: int, out, *, table_stride: int = 0,
             out_stride: int = 0, status=None, status_keep: bool = False, stream=None) -> None:
    """GET_ROWS (halo_mi_get_rows): out[i] = dequant(table row ids[i]); ids int32 on the device."""
    p = _GetRowsParams(int(t), int(layout), _ptr(table), int(table_stride), int(n_rows), int(cols), _ptr(ids), int(n_ids),
                       _ptr(out), int(out_stride), _ptr(status), 1 if status_keep else 0)
    _check(lib().halo_mi_get_rows(ctypes.byref(p), _stream(stream)))


def rms_norm(x, w, out, rows: int, cols: int, *, eps: float = 1e-6, x_stride: int = 0, out_stride: int = 0,
             stream=None) -> None:
    """RMS_NORM (halo_mi_rms_norm), bitwise cpu::rms_norm."""
    _check(lib().halo_mi_rms_norm(_ptr(x), int(x_stride), _ptr(w), _ptr(out), int(out_stride), int(rows), int(cols),
                                  float(eps), _stream(stream)))


def stream_read(p, nbytes: int, workgroups: int, unroll: int, sink, stream=None) -> None:
    """One read-only stream over nbytes at p (halo_mi_stream_read): the read floor's kernel."""
    _check(lib().halo_mi_stream_read(_ptr(p), int(nbytes), int(workgroups), int(unroll), _ptr(sink), _stream(stream)))


def stream_check(stream=None) -> None:
    """Synchronizes the stream and raises HaloError(Device) when a kernel marked its status word
    (a split-K reduction that gave up waiting) since the last check (halo_mi_stream_check)."""
    _check(lib().halo_mi_stream_check(_stream(stream)))


def stream_release(stream=None) -> None:
    """Frees the stream's workspace on the current device (halo_mi_stream_release)."""
    _check(lib().halo_mi_stream_release(_stream(stream)))


def force_splitk_timeout(spin_limit: int, force: bool) -> None:
    """Failure-path test hook (halo_mi_test_splitk_timeout): force every split-K reduction to give
    up after spin_limit rounds; force=False restores normal operation."""
    _check(lib().halo_mi_test_splitk_timeout(int(spin_limit), 1 if force else 0))


def repack_slab(t: int, src, rows: int, cols: int, dst, *, src_stride: int = 0, stream=None) -> None:
    _check(lib().halo_mi_repack_slab(int(t), _ptr(src), int(src_stride), int(rows), int(cols), _ptr(dst), _stream(stream)))


def unpack_slab(t: int, src, rows: int, cols: int, dst, *, dst_stride: int = 0, stream=None) -> None:
    _check(lib().halo_mi_unpack_slab(int(t), _ptr(src), int(rows), int(cols), _ptr(dst), int(dst_stride), _stream(stream)))


def upload_tensors(tensors, *, chunk_bytes: int = 0, host_threads: int = 0, stream=None) -> None:
    """Model-scale upload (halo_mi_upload_tensors). tensors: a list of (type, cols, parts, dst)
    with parts a list of (host rows, rows) or (host rows, rows, src_stride); host rows are numpy
    uint8 arrays (e.g. memmaps of the GGUF tensors) or host addresses. The parts' rows are
    concatenated into one SLAB matrix at dst (a row-fused projection when there are several)."""
    keep = []
    arr = (_UploadTensor * len(tensors))()
    for i, (t, cols, parts, dst) in enumerate(tensors):
        pa = (_UploadPart * len(parts))()
        for j, part in enumerate(parts):
            src, rows = part[0], part[1]
            stride = part[2] if len(part) > 2 else 0
            pa[j] = _UploadPart(src if isinstance(src, int) else src.ctypes.data, int(stride), int(rows))
        keep.append(pa)
        arr[i] = _UploadTensor(int(t), int(cols), pa, len(parts), _ptr(dst))
    _check(lib().halo_mi_upload_tensors(arr, len(tensors), int(chunk_bytes), int(host_threads), _stream(stream)))


def upload_slab(t: int, host_src, rows: int, cols: int, dst, *, src_stride: int = 0, chunk_bytes: int = 0,
                stream=None) -> None:
    """host_src: a numpy uint8 array (e.g. a memmap of the GGUF tensor) or a host address."""
    addr = host_src if isinstance(host_src, int) else host_src.ctypes.data
    _check(lib().halo_mi_upload_slab(int(t), addr, int(src_stride), int(rows), int(cols), _ptr(dst), int(chunk_bytes),
                                     _stream(stream)))
