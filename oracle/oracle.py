"""ctypes wrapper of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this module, as the
checker of the HIP path. See oracle.h for the reference lines each function restates.
"""
from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_SO = _DIR / "liboracle.so"

OK, EMODEL, EUNSUPPORTED, EKERNEL = 0, 1, 2, 3


class OracleError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"oracle error {code} in {what}")


@functools.lru_cache(maxsize=None)
def lib() -> ctypes.CDLL:
    if not _SO.exists():
        raise RuntimeError(f"{_SO} is missing: run `make -C oracle`")
    so = ctypes.CDLL(str(_SO))
    U32, U64, I64, VP, INT = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
    sig = {
        "oracle_fp16_to_fp32": (ctypes.c_float, [ctypes.c_uint16]),
        "oracle_block_elems": (U32, [U32]),
        "oracle_block_bytes": (U32, [U32]),
        "oracle_row_bytes": (U64, [U32, I64, ctypes.POINTER(INT)]),
        "oracle_dequantize_row": (INT, [U32, VP, VP, I64]),
        "oracle_dequant_terms": (INT, [U32, VP, VP, VP, VP, I64]),
        "oracle_dot": (ctypes.c_float, [VP, VP, ctypes.c_size_t]),
        "oracle_vec_dot_row": (INT, [U32, VP, VP, I64, ctypes.POINTER(ctypes.c_float)]),
        "oracle_matmul": (INT, [U32, VP, U64, U32, U32, VP, U64, U32, VP, U64, U32]),
        "oracle_swiglu": (None, [VP, VP, VP, ctypes.c_size_t]),
        "oracle_rms_norm": (None, [VP, U64, VP, VP, U64, U32, U32, ctypes.c_float]),
        "oracle_gate_up_swiglu": (INT, [U32, VP, VP, U64, U32, U32, VP, U32, VP, U32]),
        "oracle_lm_head": (INT, [U32, VP, U64, U32, U32, VP, U32, U32, VP, VP, U32]),
        "oracle_argmax_words": (None, [VP, U32, U32, VP]),
        "oracle_partition_range": (None, [ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                          ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
        "oracle_default_threads": (U32, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(so, name)
        fn.restype = res
        fn.argtypes = args
    return so


def _chk(rc: int, what: str) -> None:
    if rc != OK:
        raise OracleError(rc, what)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fp16_to_fp32(h: int) -> float:
    return lib().oracle_fp16_to_fp32(int(h))


def row_bytes(t: int, n: int) -> int:
    err = ctypes.c_int(0)
    v = lib().oracle_row_bytes(int(t), int(n), ctypes.byref(err))
    _chk(err.value, "row_bytes")
    return int(v)


def dequantize_row(t: int, src, n: int) -> np.ndarray:
    src = _u8(src)
    out = np.empty(int(n), dtype=np.float32)
    _chk(lib().oracle_dequantize_row(int(t), src.ctypes.data, out.ctypes.data, int(n)), "dequantize_row")
    return out


def dequantize_rows(t: int, w, rows: int, cols: int, stride: int = 0) -> np.ndarray:
    """rows x cols fp32 from GGUF rows `stride` bytes apart (0 = dense)."""
    w = _u8(w)
    rb = row_bytes(t, cols)
    stride = stride or rb
    out = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        row = w[r * stride: r * stride + rb]
        _chk(lib().oracle_dequantize_row(int(t), row.ctypes.data, out[r].ctypes.data, int(cols)), "dequantize_row")
    return out


def dequant_terms(t: int, w, rows: int, cols: int):
    """(a, b, off) per weight, with w = fl(a - b); see oracle.h."""
    w = _u8(w)
    rb = row_bytes(t, cols)
    a = np.empty((rows, cols), np.float32)
    b = np.empty_like(a)
    off = np.empty_like(a)
    for r in range(rows):
        row = w[r * rb: (r + 1) * rb]
        _chk(lib().oracle_dequant_terms(int(t), row.ctypes.data, a[r].ctypes.data, b[r].ctypes.data,
                                        off[r].ctypes.data, int(cols)), "dequant_terms")
    return a, b, off


def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return lib().oracle_dot(a.ctypes.data, b.ctypes.data, a.size)


def vec_dot_row(t: int, row, x) -> float:
    row, x = _u8(row), _f32(x)
    out = ctypes.c_float()
    _chk(lib().oracle_vec_dot_row(int(t), row.ctypes.data, x.ctypes.data, x.size, ctypes.byref(out)), "vec_dot_row")
    return out.value


def matmul(t: int, w, rows: int, cols: int, x, *, w_stride: int = 0, threads: int = 0) -> np.ndarray:
    """y[n_vec, rows] = dequant(W) x (cpu::matmul semantics)."""
    w = _u8(w)
    x = _f32(x).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), dtype=np.float32)
    th = threads or lib().oracle_default_threads()
    _chk(lib().oracle_matmul(int(t), w.ctypes.data, int(w_stride), int(rows), int(cols), x.ctypes.data, int(cols),
                             x.shape[0], y.ctypes.data, int(rows), int(th)), "matmul")
    return y


def lm_head(t: int, w, rows: int, cols: int, x, *, valid_rows: int = 0, w_stride: int = 0, threads: int = 0):
    """(result words [n_vec, 3] uint32, logits [n_vec, rows]) of CpuBackend::lm_head."""
    w = _u8(w)
    x = _f32(x).reshape(-1, cols)
    n = x.shape[0]
    logits = np.empty((n, rows), dtype=np.float32)
    res = np.empty((n, 3), dtype=np.uint32)
    th = threads or lib().oracle_default_threads()
    _chk(lib().oracle_lm_head(int(t), w.ctypes.data, int(w_stride), int(rows), int(cols), x.ctypes.data, n,
                              int(valid_rows), logits.ctypes.data, res.ctypes.data, int(th)), "lm_head")
    return res, logits


def argmax_words(logits) -> np.ndarray:
    """Result words [n_vec, 3] of cpu::argmax per row (poisoned words for a row with a NaN)."""
    lg = _f32(logits)
    lg = lg.reshape(-1, lg.shape[-1]) if lg.ndim > 1 else lg.reshape(1, -1)
    res = np.empty((lg.shape[0], 3), dtype=np.uint32)
    lib().oracle_argmax_words(lg.ctypes.data, lg.shape[1], lg.shape[0], res.ctypes.data)
    return res


def swiglu(g, u) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().oracle_swiglu(g.ctypes.data, u.ctypes.data, out.ctypes.data, g.size)
    return out


def rms_norm(x, w, eps: float = 1e-6) -> np.ndarray:
    """cpu::rms_norm of the rows of x (2-D) with weight w."""
    x = _f32(x)
    x2 = x.reshape(-1, x.shape[-1]) if x.ndim > 1 else x.reshape(1, -1)
    w = _f32(w)
    out = np.empty_like(x2)
    lib().oracle_rms_norm(x2.ctypes.data, x2.shape[1], w.ctypes.data, out.ctypes.data, x2.shape[1], x2.shape[0], x2.shape[1],
                          float(eps))
    return out.reshape(x.shape)


def gate_up_swiglu(t: int, wg, wu, rows: int, cols: int, x, threads: int = 0) -> np.ndarray:
    wg, wu = _u8(wg), _u8(wu)
    x = _f32(x).reshape(-1, cols)
    out = np.empty((x.shape[0], rows), dtype=np.float32)
    th = threads or lib().oracle_default_threads()
    _chk(lib().oracle_gate_up_swiglu(int(t), wg.ctypes.data, wu.ctypes.data, 0, int(rows), int(cols), x.ctypes.data,
                                     x.shape[0], out.ctypes.data, int(th)), "gate_up_swiglu")
    return out


def default_threads() -> int:
    return int(lib().oracle_default_threads())
