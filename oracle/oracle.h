/*
 * CPU oracle for the quantized matrix-multiply path. TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, in plain C, the reference CPU backend's semantics for the path
 * (dequantize_row + cpu::matmul + cpu::swiglu). It is the checker for the HIP kernels: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The product
 * (halo_amd/) never links, loads or calls it, and has no CPU fallback.
 *
 * Every function names the reference file:line it follows. Build flags mirror the reference's
 * CPU backend: -O2 -g -ffp-contract=off, no -march (backends/cpu/CMakeLists.txt:14-16,
 * CMakeLists.txt:24-29).
 *
 * Type ids are ggml's (include/halo/tensor/dtype.h:18-49): F32 = 0, F16 = 1, Q4_0 = 2,
 * Q8_0 = 8, Q3_K = 11, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ4_NL = 20, IQ3_S = 21, IQ4_XS = 23
 * (the weight types of the reference's HIP GEMV test matrix, tests/unit/hip/test_hip_gemv.cpp:
 * 217-218), and the rest of the reference dequantizer's dispatch (quant.cpp:386-407): Q4_1 = 3,
 * Q5_0 = 6, Q5_1 = 7, Q2_K = 10, BF16 = 30. F32 rows are read in place by the matmul.
 *
 * Return codes: 0 = ok, ORACLE_EMODEL (1) = bad element count / byte size (the reference's
 * Error(Model), quant.cpp:411-428), ORACLE_EUNSUPPORTED (2) = type not on this path
 * (Error(Unsupported), quant.cpp:404-407), ORACLE_EKERNEL (3) = shape/alias error
 * (Error(Kernel), matmul.cpp:38-43).
 */
#ifndef HALO_ORACLE_H
#define HALO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORACLE_OK = 0, ORACLE_EMODEL = 1, ORACLE_EUNSUPPORTED = 2, ORACLE_EKERNEL = 3 };

/* include/halo/tensor/fp16.h:19-37: exact fp16 -> fp32 widening (subnormals, inf, NaN). */
float oracle_fp16_to_fp32(uint16_t h);

/* src/tensor/dtype.cpp:19-51: block geometry. Returns 0 for a type not on this path. */
uint32_t oracle_block_elems(uint32_t type);
uint32_t oracle_block_bytes(uint32_t type);

/* src/tensor/quant.cpp:411-418: bytes of one row of n elements; sets *err on failure. */
uint64_t oracle_row_bytes(uint32_t type, int64_t n, int* err);

/* src/tensor/quant.cpp:430-435: dequantize n elements (whole blocks) from src into dst. */
int oracle_dequantize_row(uint32_t type, const uint8_t* src, float* dst, int64_t n);

/*
 * Test helper (no reference counterpart): splits every dequantized weight into the two
 * exactly-representable terms the reference expression subtracts, w = fl(a - b):
 *   Q4_K  a = (d*sc)*q,       b = dmin*m                     (quant.cpp:258-265)
 *   Q5_K  a = (d*sc)*q,       b = dmin*m                     (quant.cpp:289-290)
 *   Q6_K  a = (d*sc)*(q-32),  b = 0                          (quant.cpp:318-321)
 *   Q4_0  a = (q-8)*d,        b = 0                          (quant.cpp:84-87)
 *   Q8_0  a = q*d,            b = 0                          (quant.cpp:147-148)
 *   IQ4_XS a = dl*table[q],   b = 0                          (quant.cpp:340-341)
 *   IQ4_NL a = d*table[q],    b = 0                          (quant.cpp:160-161)
 *   Q3_K  a = (d*(sc-32))*q,  b = 0                          (quant.cpp:220-226)
 *   IQ3_S a = (db*g)*sign,    b = 0                          (quant.cpp:368-369)
 *   Q4_1  a = q*d,            b = -m                         (quant.cpp:101-102)
 *   Q5_1  a = q*d,            b = -m                         (quant.cpp:136-137)
 *   Q2_K  a = dl*q,           b = ml                         (quant.cpp:181, :186)
 *   Q5_0  a = (q-16)*d,       b = 0; BF16 a = w, b = 0       (quant.cpp:118-119, :72-74)
 * and also returns the "factored" magnitude terms the GPU kernels sum: the offset they take
 * out of the quant, in off[] (Q4_0 8*d, Q6_K 32*d*sc, Q8_0 128*d, IQ4_XS 128*dl, IQ4_NL
 * 128*d, Q3_K 4*dl, IQ3_S 16*db), else 0. F32 and F16 have no terms (ORACLE_EUNSUPPORTED).
 * Used to size summation-error bounds.
 */
int oracle_dequant_terms(uint32_t type, const uint8_t* src, float* a, float* b, float* off, int64_t n);

/* backends/cpu/kernel_common.h:16-27: fixed-order 8-lane fp32 dot product. */
float oracle_dot(const float* a, const float* b, size_t n);

/* src/tensor/quant.cpp:447-466: dequantize in 256-element chunks, accumulate in double. */
int oracle_vec_dot_row(uint32_t type, const uint8_t* row, const float* x, int64_t n, float* out);

/*
 * backends/cpu/matmul.cpp:37-59 over src/backend/cpu_backend.cpp:193-211's weight matrix:
 * y[t][n] = dot(x_t, dequantize_row(W row n)) for t < n_vec, n < rows.
 *   w: rows rows, w_stride BYTES apart (0 = row_bytes); x / y: x_stride / y_stride FLOATS
 *   apart (0 = dense). 16-row blocks over a static partition on `threads` threads
 *   (include/halo/backends/cpu/thread_pool.h:58-76, :103-113); results are independent of
 *   `threads`.
 */
int oracle_matmul(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t rows, uint32_t cols,
                  const float* x, uint64_t x_stride, uint32_t n_vec, float* y, uint64_t y_stride,
                  uint32_t threads);

/* backends/cpu/ops_basic.cpp:165-167 + kernel_common.h:32: out = silu(g) * u, elementwise. */
void oracle_swiglu(const float* g, const float* u, float* out, size_t n);

/*
 * cpu::rms_norm (backends/cpu/ops_basic.cpp:18-33): per row, mean = sum_squares(x) / cols with
 * sum_squares = dot(x, x) (kernel_common.h:29), inv = 1 / sqrt(mean + eps), out = (x * inv) * w.
 * Strides in floats (0 = cols); out may be x itself.
 */
void oracle_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride,
                     uint32_t rows, uint32_t cols, float eps);

/*
 * The reference FFN composition (src/models/qwen35.cpp:789-805): gemv(gate), gemv(up),
 * swiglu -> out[t][n] = silu(Wg x_t)[n] * (Wu x_t)[n]. Both weights share type and shape.
 */
int oracle_gate_up_swiglu(uint32_t type, const uint8_t* wg, const uint8_t* wu, uint64_t w_stride,
                          uint32_t rows, uint32_t cols, const float* x, uint32_t n_vec, float* out,
                          uint32_t threads);

/*
 * CpuBackend::lm_head (src/backend/cpu_backend.cpp:669-770): logits by cpu::matmul in slabs of
 * 8192 rows and the fused argmax over exactly those values (ties to the lowest index; a NaN
 * logit poisons its vector; rows >= valid_rows, when valid_rows != 0, are not ranked).
 * result: n_vec triples {index, value bits, poisoned} (kArgmaxResultBytes = 12,
 * include/halo/backend/backend.h:430-431). logits: n_vec x rows floats, or NULL.
 */
int oracle_lm_head(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t rows, uint32_t cols, const float* x,
                   uint32_t n_vec, uint32_t valid_rows, float* logits, uint32_t* result, uint32_t threads);

/*
 * cpu::argmax per row (backends/cpu/matmul.cpp:61-72: the first maximum, a row replacing the best
 * only when strictly greater) as result words {index, value bits, poisoned}; a NaN in the row
 * (the CPU's Error(Kernel)) gives the poisoned words {0xFFFFFFFF, quiet NaN, 1}, as LM_HEAD's
 * (src/backend/cpu_backend.cpp:745-747, :825-833). logits: n_vec rows of n floats, dense.
 */
void oracle_argmax_words(const float* logits, uint32_t n, uint32_t n_vec, uint32_t* result);

/* include/halo/backends/cpu/thread_pool.h:58-64: part i of [0, n) split into `parts`. */
void oracle_partition_range(size_t n, size_t parts, size_t i, size_t* begin, size_t* end);

/* std::thread::hardware_concurrency() equivalent (thread_pool.h:53-54). */
uint32_t oracle_default_threads(void);

#ifdef __cplusplus
}
#endif

#endif
