/*
 * halo_mi355x: MI355X (gfx950) quantized matrix-multiply backend, C ABI.
 *
 * This is the seam between host code and the hand-written HIP kernels. It replaces the HIP
 * backend's launcher seam of the reference (backends/hip/src/launch.h:16-37:
 * `int launch_gemv_*(const kern::GemvParams&, const kern::Launch&, void* stream)`, returning
 * the hipError_t as an int). Every entry point takes plain pointers, sizes and a hipStream_t
 * passed as `void*`, validates its arguments on the host, enqueues work, and returns a status
 * code; no exception crosses the ABI. halo_mi_last_error() gives the message of the last
 * failing call on the calling thread.
 *
 * Device pointers are HIP device memory on the current device. `stream` may be NULL (the
 * null stream). Work is asynchronous: outputs are valid after the stream is synchronized.
 *
 * Status codes follow the reference's error mapping (include/halo/backend/backend.h:24-26):
 * shape / alias / range / alignment -> HALO_MI_E_KERNEL, dtype or limit -> HALO_MI_E_UNSUPPORTED,
 * unknown variant id -> HALO_MI_E_CONFIG, allocation -> HALO_MI_E_MEMORY, a HIP runtime error
 * -> HALO_MI_E_DEVICE.
 */
#ifndef HALO_MI355X_H
#define HALO_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------------------------- */
enum {
    HALO_MI_OK = 0,
    HALO_MI_E_KERNEL = 1,      /* shape, alias, range or alignment problem */
    HALO_MI_E_UNSUPPORTED = 2, /* weight type or limit not supported */
    HALO_MI_E_CONFIG = 3,      /* unknown variant id */
    HALO_MI_E_MEMORY = 4,      /* allocation failure */
    HALO_MI_E_DEVICE = 5       /* HIP runtime / launch failure */
};

/* Message of the last failing call on this thread ("" when none). */
const char* halo_mi_last_error(void);

/* ---- weight types (ggml ids, include/halo/tensor/dtype.h:18-49) ------------------------- */
/*
 * Every type of the reference's CPU dequantizer (src/tensor/quant.cpp:386-407) is decoded on
 * the GGUF layout by halo_mi_dequant_rows, halo_mi_get_rows and the reference-order GEMV
 * (HALO_MI_GEMV_GGUF_REF), bitwise as dequantize_row and cpu::matmul. The SLAB layout, and with
 * it every fast kernel, takes Q4_0, Q8_0, Q4_K, Q5_K, Q6_K and IQ4_XS. The reference's HIP
 * backend has kernels for eleven of them (backends/hip/src/ops.cpp:531-549: not BF16, Q4_1,
 * Q5_0, Q5_1, Q2_K); the C++ backend of this library refuses the same five.
 */
enum {
    HALO_MI_F32 = 0,
    HALO_MI_F16 = 1,
    HALO_MI_Q4_0 = 2,
    HALO_MI_Q4_1 = 3,
    HALO_MI_Q5_0 = 6,
    HALO_MI_Q5_1 = 7,
    HALO_MI_Q8_0 = 8,
    HALO_MI_Q2_K = 10,
    HALO_MI_Q3_K = 11,
    HALO_MI_Q4_K = 12,
    HALO_MI_Q5_K = 13,
    HALO_MI_Q6_K = 14,
    HALO_MI_IQ4_NL = 20,
    HALO_MI_IQ3_S = 21,
    HALO_MI_IQ4_XS = 23,
    HALO_MI_BF16 = 30
};

/* ---- weight layouts ---------------------------------------------------------------------- */
/*
 * HALO_MI_LAYOUT_GGUF: rows of GGUF blocks exactly as in the file (w_stride bytes apart, any
 *   alignment). What the reference imports (src/backend/hip_adapter.cpp:502-515).
 * HALO_MI_LAYOUT_SLAB: the device layout written by halo_mi_repack_slab(). Rows are grouped
 *   in slabs of 64; inside a slab every plane is slot-major and row-minor, so one wave's
 *   load of a slot covers 64 rows contiguously. A slab has exactly 64 * row_bytes bytes; the
 *   last slab of a matrix is zero-padded to 64 rows. The GGUF bytes are recoverable with
 *   halo_mi_unpack_slab().
 */
enum { HALO_MI_LAYOUT_GGUF = 0, HALO_MI_LAYOUT_SLAB = 1 };

/* Rows per slab. */
#define HALO_MI_SLAB_ROWS 64u

/* ---- gemv variants (append-only ids; 0 = default for the layout) ------------------------ */
/*
 * Counterpart of the reference's KernelChoice registry (backend.h:173-176, ids pinned by
 * tests/unit/backend/test_hip_backend.cpp:925-981). These are this library's own ids; the
 * reference registry ids they take behind its HIP backend are listed with the C++ backend
 * (include/halo_mi355x_backend.hpp).
 *   0 HALO_MI_GEMV_DEFAULT   GGUF layout -> gemv_gguf_ref; SLAB layout -> gemv_slab_auto.
 *   1 HALO_MI_GEMV_GGUF_REF  GGUF layout, 8 lanes per output in cpu::detail::dot's order:
 *                            bit-identical to the CPU backend.
 *   2 HALO_MI_GEMV_SLAB      SLAB layout, wave64 row-per-lane weight stream, split-K inside
 *                            the workgroup and across workgroups (fixed-order fix-up); any
 *                            n_vec (4 per pass over the weights). Within the summation bound;
 *                            every row is bitwise independent of n_vec.
 *   3 HALO_MI_GEMM_SLAB_BF16 SLAB layout, bf16 MFMA GEMM (dequantized W and x rounded to
 *                            bf16, fp32 accumulate) on M tiles of 64 / 128 / 256 rows by n_vec;
 *                            any n_vec.
 *   4 HALO_MI_GEMV_SLAB_AUTO SLAB layout: 2 for n_vec <= 2 (Q6_K: <= 4); 8 for the rest up to
 *                            n_vec <= 8 (2 when cols is not a multiple of 256); so up to 8
 *                            vectors the result is within 2's bound.
 *                            Above 8, the small-M bf16 GEMM (same numerics as 3) for n_vec <= 32
 *                            when cols is a multiple of 256; else 5 when n_vec > 256 and its
 *                            tiles fill the GPU, else 3.
 *   5 HALO_MI_GEMM_SLAB_BF16_M512  the bf16 MFMA GEMM on 512-row M tiles (every wave both
 *                            dequantizes and multiplies; same numerics as 3); any n_vec.
 *   6 HALO_MI_GEMV_SLAB_VALU the SLAB GEMV with its multiply-adds on the VALU instead of the
 *                            matrix core (Q4_0, Q8_0, Q4_K, Q6_K; no fused norm); the same
 *                            split and bound as 2.
 *   7 HALO_MI_GEMM_SLAB_BF16_SMALL_M  the bf16 MFMA GEMM's small-M kernel (no LDS stage; waves
 *                            dequantize their own MFMA operands): n_vec <= 32, cols a multiple
 *                            of 256; same numerics as 3.
 *   8 HALO_MI_GEMM_SLAB_EXACT_SMALL_M  the exact-product small-M GEMM: the slab GEMV's
 *                            arithmetic (integer codes times x split exactly into three bf16
 *                            pieces, fp32 sums, scales applied per slot) on 32x32 MFMA tiles;
 *                            n_vec <= 8, cols a multiple of 256; within the bound of 2. Its K
 *                            split is the one planned for 8 vectors whatever n_vec is, so rows do
 *                            not depend on n_vec.
 *   9 HALO_MI_GEMM_SLAB_EXACT_INVARIANT  8's kernel for any n_vec, in passes of 8 vectors:
 *                            every row of y is bitwise the row an n_vec = 1 call
 *                            gives (the batch-invariance contract of GemvArgs::allow_gemm =
 *                            false, backend.h:298-304). Where that split does not fit the shape
 *                            (cols not a multiple of 256, or more partial sums than the stream's
 *                            workspace holds) it runs 2, which is batch-invariant too: the
 *                            choice follows the shape only. Within the bound of 2. Faster than
 *                            2 from 3 vectors (one pass over the weights up to 8), slower at 1.
 */
enum {
    HALO_MI_GEMV_DEFAULT = 0,
    HALO_MI_GEMV_GGUF_REF = 1,
    HALO_MI_GEMV_SLAB = 2,
    HALO_MI_GEMM_SLAB_BF16 = 3,
    HALO_MI_GEMV_SLAB_AUTO = 4,
    HALO_MI_GEMM_SLAB_BF16_M512 = 5,
    HALO_MI_GEMV_SLAB_VALU = 6,
    HALO_MI_GEMM_SLAB_BF16_SMALL_M = 7,
    HALO_MI_GEMM_SLAB_EXACT_SMALL_M = 8,
    HALO_MI_GEMM_SLAB_EXACT_INVARIANT = 9,
    HALO_MI_GEMV_VARIANT_LAST = 9
};

/*
 * y[t][n] = sum_i x[t][i] * W[n][i] for t < n_vec, n < rows, i < cols.
 * Replaces backend::GemvArgs + Backend::gemv (include/halo/backend/backend.h:283-314, :562)
 * at the launcher level, as kern::GemvParams does (backends/hip/kernels/gemv.h:267-281).
 *   w: device weights in `layout`; for GGUF, w_stride = bytes between rows (0 = row_bytes);
 *      for SLAB, w_stride must be 0.
 *   x: n_vec rows of cols fp32, x_stride floats apart (0 = cols).
 *   y: n_vec rows of rows fp32, y_stride floats apart (0 = rows). y must not overlap x or w.
 *   norm_w (optional, cols fp32): the fused input norm of GemvArgs::norm_w / norm_eps
 *      (backend.h:292-299): y = W (rms_norm(x) * norm_w) with eps = norm_eps, x the raw rows;
 *      rms_norm as cpu::rms_norm (backends/cpu/ops_basic.cpp:18-33). Every variant, layout and
 *      n_vec (the reference accepts it on one Vulkan path only):
 *        - GGUF reference variant: x is normalized first exactly as cpu::rms_norm, so y is
 *          bitwise rms_norm then matmul;
 *        - bf16 GEMM variants: the same normalized x, rounded to bf16 while it is staged;
 *        - SLAB GEMV (2 and the GEMV legs of the auto variants), one vector: inside the MFMA
 *          GEMV's launch, one dispatch: every workgroup computes 1 / rms in cpu::rms_norm's
 *          order and normalizes its own x elements as cpu::rms_norm rounds them (cols <= 8192);
 *        - otherwise (more vectors, wider rows, variant 6): x is normalized into the stream's
 *          workspace by the RMS_NORM kernel, then the GEMV runs on it.
 *      So y is bitwise halo_mi_rms_norm then the same variant without the norm, at any n_vec
 *      (the reference's Limits::max_fused_norm_cols contract, backend.h:236-242).
 *      norm_w must not overlap y.
 */
typedef struct halo_mi_gemv_params {
    uint32_t type;
    uint32_t layout;
    const void* w;
    uint64_t w_stride;
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    uint32_t rows;
    uint32_t cols;
    uint32_t n_vec;
    uint32_t variant;
    const float* norm_w;
    float norm_eps;
} halo_mi_gemv_params;

int halo_mi_gemv(const halo_mi_gemv_params* p, void* stream);

/*
 * halo_mi_gemv without any allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same operands, checks and results as halo_mi_gemv (bitwise) for the
 * calls that run the SLAB GEMV: variants 2 and 6 at any n_vec, and 0 and 4 where their auto
 * choice is the SLAB GEMV (up to 2 vectors; up to 4 for Q6_K and for Q4_K, Q5_K and IQ4_XS
 * matrices of at most 128 slabs; up to 8 where the exact small-M GEMM's plan does not fit).
 * Where 0 or 4 would run a GEMM kernel, and for the GEMM variants, it returns
 * HALO_MI_E_UNSUPPORTED. The split-K words, slab counters and status word live in a fixed
 * device array of this library (about 8.3 MiB per GPU, held until the process ends), not in a
 * per-stream workspace: a shape whose split needs more than 65536 slabs of counters or 2^20
 * words (e.g. the 17408 x 5120 headline needs 2^17.7) returns HALO_MI_E_UNSUPPORTED. Every call
 * on one GPU shares that array, so calls that overlap in time on one GPU (other streams, other
 * threads) race and give wrong results: order them. halo_mi_stream_check also reports this
 * array's status word.
 */
int halo_mi_gemv_noalloc(const halo_mi_gemv_params* p, void* stream);

/*
 * Grouped GEMV: several SLAB matrices that share x, in one launch per pair of weight types,
 * e.g. a layer's q, k and v projections (Q4_K q and k, Q6_K v) after the same input norm. The
 * reference issues them one by one on one stream (Qwen35::Impl::gemv,
 * src/models/qwen35.cpp:486-498), and each small projection then pays a whole launch's ramp and
 * drain; row-fusing them into one matrix (halo_mi_upload_tensors) needs equal types.
 *   segs[i]: the segment's weight type, SLAB image (16-byte aligned), rows, and output y_i
 *            (n_vec rows of rows floats, y_stride apart, 0 = rows): y_i = W_i x (with the fused
 *            norm: W_i (rms_norm(x) * norm_w), as halo_mi_gemv).
 *   x, x_stride, cols, n_vec, norm_w, norm_eps: shared, with halo_mi_gemv's meaning.
 * Numerics: halo_mi_gemv's SLAB GEMV bound per output (the K split follows the group's total
 * slabs, so a row may round differently from a call of its own; rows stay independent of n_vec).
 * No output may overlap x, norm_w, any segment's weights or another output.
 * n_segs <= HALO_MI_GEMV_GROUP_MAX; more than two weight types take one launch per pair.
 */
#define HALO_MI_GEMV_GROUP_MAX 4u

typedef struct halo_mi_gemv_segment {
    uint32_t type;
    const void* w;
    uint32_t rows;
    float* y;
    uint64_t y_stride;
} halo_mi_gemv_segment;

typedef struct halo_mi_gemv_group_params {
    const halo_mi_gemv_segment* segs;
    uint32_t n_segs;
    const float* x;
    uint64_t x_stride;
    uint32_t cols;
    uint32_t n_vec;
    const float* norm_w;
    float norm_eps;
} halo_mi_gemv_group_params;

int halo_mi_gemv_group(const halo_mi_gemv_group_params* p, void* stream);

/*
 * Grouped bf16 GEMM: the same segments and operands as halo_mi_gemv_group, computed by the bf16
 * MFMA GEMM (the prefill path, GemvArgs::allow_gemm: halo_mi_gemv's numerics for more than 8
 * vectors), with x staged once for all segments and one launch per pair of weight types (M
 * tiles of 64 / 128 / 256 rows by n_vec; when a launch's tiles fill less than half the GPU,
 * every tile is split over the same K chunks and one reduce adds them in chunk order). The
 * reference issues the projections one by one (Qwen35::Impl::gemv, src/models/qwen35.cpp:
 * 486-498); a layer's q, k and v at M = 512 then pay three x stagings, three under-filled
 * launches and three reduces. Numerics per output: halo_mi_gemv's bf16 GEMM bound; x rows
 * 16-byte aligned (x_stride a multiple of 4 floats), as the single-matrix GEMM.
 */
int halo_mi_gemm_group(const halo_mi_gemv_group_params* p, void* stream);

/*
 * Fused FFN gate/up: out[t][n] = silu((Wg x_t)[n]) * (Wu x_t)[n], silu(v) = v / (1 + exp(-v)).
 * The reference composes it as gemv(gate), gemv(up), swiglu (src/models/qwen35.cpp:789-805;
 * backends/cpu/ops_basic.cpp:165-167); here both matmuls and the epilogue are one launch.
 * Wg and Wu share type, layout and shape (rows x cols). SLAB layout only; variant 0/4 = auto
 * (the gemv pair for n_vec <= 2, the exact small-M GEMM (8) for 3 and 4 when cols is a multiple
 * of 256, else the gemv pair up to 4; above 4 the bf16 GEMM, its M
 * tiles chosen as for halo_mi_gemv), 2 = gemv kernel (any n_vec, 4 vectors per pass over the
 * weights), 3 / 5 / 7 = bf16 MFMA GEMM on 64..256 / 512-row / small-M tiles, 8 = the exact
 * small-M GEMM (n_vec <= 8). The GEMMs' SiLU is the fast form (relative error at most
 * (1.5 |v| + 8) 2^-24), the gemv pair's the IEEE one. out may not overlap x, Wg or Wu.
 * norm_w / norm_eps (optional): the fused input norm as for halo_mi_gemv (the FFN's
 * post-attention norm folded into the pair).
 */
typedef struct halo_mi_gate_up_params {
    uint32_t type;
    uint32_t layout;
    const void* w_gate;
    const void* w_up;
    const float* x;
    uint64_t x_stride;
    float* out;
    uint64_t out_stride;
    uint32_t rows;
    uint32_t cols;
    uint32_t n_vec;
    uint32_t variant;
    const float* norm_w;
    float norm_eps;
} halo_mi_gate_up_params;

int halo_mi_gate_up_swiglu(const halo_mi_gate_up_params* p, void* stream);

/*
 * LM head: the gemv over the vocabulary plus the fused argmax. Replaces Backend::lm_head and
 * LmHeadArgs (include/halo/backend/backend.h:433-460, :572); the semantics are
 * CpuBackend::lm_head's (src/backend/cpu_backend.cpp:669-770):
 *   - the argmax is taken over exactly the values the gemv produces: higher value first, ties
 *     to the lowest index;
 *   - a NaN logit poisons only its own vector: its result is {0xFFFFFFFF, quiet NaN, 1};
 *   - rows at or past valid_rows (when not 0) are not ranked (GGUF LM-head padding), but a NaN
 *     in them still poisons; the logits of every row are still written;
 *   - a vector with no ranked row reports {0xFFFFFFFF, 0.0f, 0}.
 * gemv: the operands and variant as for halo_mi_gemv, except that y may be NULL (the logits are
 *   not kept). With the SLAB layout and variant 0, 2 or 4 the argmax is fused into the slab
 *   GEMV (any n_vec); the GGUF reference kernel and the MFMA GEMM variants (1, 3, 5) rank the
 *   logits afterwards and need y.
 * result: n_vec triples of uint32 {index, value bits, poisoned} (HALO_MI_ARGMAX_RESULT_BYTES
 *   each, 4-byte aligned), as kArgmaxResultBytes (backend.h:430-431).
 * ids (optional): n_vec int32 winning indices, 0 for a poisoned vector or one with no ranked row.
 * ids_slots / ids_scatter (optional, both or neither, only with ids): vector t's id is also
 *   written to ids_scatter[ids_slots[t]]; a slot at or past ids_scatter_len is not written.
 * None of result, ids, ids_scatter may overlap x, w, y or each other.
 */
#define HALO_MI_ARGMAX_RESULT_BYTES 12u

typedef struct halo_mi_lm_head_params {
    halo_mi_gemv_params gemv;
    void* result;
    uint32_t valid_rows;
    int32_t* ids;
    const uint32_t* ids_slots;
    int32_t* ids_scatter;
    uint64_t ids_scatter_len;
} halo_mi_lm_head_params;

int halo_mi_lm_head(const halo_mi_lm_head_params* p, void* stream);

/*
 * ARGMAX (ArgmaxArgs, backend.h:463-468; CpuBackend::argmax, src/backend/cpu_backend.cpp:772-783):
 * for each of n_vec rows of n fp32 logits (logits_stride floats apart, 0 = n) the result words
 * {index, value bits, poisoned} of halo_mi_lm_head: the highest value, ties to the lowest index;
 * a NaN poisons its row's words (the CPU backend's Error(Kernel) for it). n >= 1. result may not
 * overlap logits.
 */
int halo_mi_argmax(const float* logits, uint64_t logits_stride, uint32_t n, uint32_t n_vec, void* result, void* stream);

/*
 * SWIGLU: out[r][c] = silu(gate[r][c]) * up[r][c] for rows x cols fp32 (strides in floats,
 * 0 = cols). The reference's op (backends/cpu/ops_basic.cpp:165-167, EltwiseArgs at
 * include/halo/backend/backend.h:420-427). out may not overlap gate or up.
 */
int halo_mi_swiglu(const float* gate, uint64_t gate_stride, const float* up, uint64_t up_stride, float* out,
                   uint64_t out_stride, uint32_t rows, uint32_t cols, void* stream);

/*
 * Dequantize rows [first_row, first_row + n_rows) of W to fp32 (out rows out_stride floats
 * apart, 0 = cols), bit-identical to tensor::dequantize_row (src/tensor/quant.cpp:430-435).
 * Works on both layouts; it shares its unpacking code with the gemv/gemm kernels.
 * The reference counterpart at the backend level is GET_ROWS (backend.h:254-263).
 */
int halo_mi_dequant_rows(uint32_t type, uint32_t layout, const void* w, uint64_t w_stride,
                         uint32_t rows, uint32_t cols, uint32_t first_row, uint32_t n_rows,
                         float* out, uint64_t out_stride, void* stream);

/*
 * GET_ROWS (GetRowsArgs, include/halo/backend/backend.h:254-263; CPU at
 * src/backend/cpu_backend.cpp:284-303; the HIP status word at backends/hip/src/ops.cpp:982-1012):
 * out[i] = dequant(table row ids[i]) for i < n_ids, bit-identical to tensor::dequantize_row.
 *   table: n_rows rows of cols weights in `layout` (GGUF: table_stride bytes apart, 0 =
 *          row_bytes; SLAB: table_stride 0). ids: n_ids int32 on the device.
 *   out: n_ids rows of cols fp32, out_stride floats apart (0 = cols); must not overlap table,
 *        ids or status.
 *   status (optional, one uint32 on the device): an id outside [0, n_rows) leaves its output
 *        row unwritten and sets HALO_MI_STATUS_BAD_INDEX (the reference's kStatusBadIndex,
 *        backends/hip/kernels/hd.h:156) in it. Ids live on the device, so this is where the CPU
 *        backend's Error(Kernel) shows: read the word after the stream is done.
 *   status_keep: 0 = the call clears the word first (it reports this call only); otherwise the
 *        bits accumulate over calls until the caller clears the word (a stream's report up to
 *        its next wait).
 */
#define HALO_MI_STATUS_BAD_INDEX 8u

typedef struct halo_mi_get_rows_params {
    uint32_t type;
    uint32_t layout;
    const void* table;
    uint64_t table_stride;
    uint32_t n_rows;
    uint32_t cols;
    const int32_t* ids;
    uint32_t n_ids;
    float* out;
    uint64_t out_stride;
    uint32_t* status;
    uint32_t status_keep;
} halo_mi_get_rows_params;

int halo_mi_get_rows(const halo_mi_get_rows_params* p, void* stream);

/*
 * RMS_NORM (RmsNormArgs, backend.h:267-272; cpu::rms_norm, backends/cpu/ops_basic.cpp:18-33):
 * out[r] = (x[r] * inv) * w with inv = 1 / sqrt(dot(x[r], x[r]) / cols + eps), bitwise equal to
 * the CPU (the sum of squares in cpu::detail::dot's order). rows x cols fp32, strides in floats
 * (0 = cols); out may be x itself with the same stride, or must not overlap x or w. This is the
 * normalization halo_mi_gemv's fused norm applies for the reference and GEMM variants.
 */
int halo_mi_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride,
                     uint32_t rows, uint32_t cols, float eps, void* stream);

/* ---- stream state --------------------------------------------------------------------------- */
/*
 * The kernels' own failures cannot be returned by the call that enqueued them. A split-K
 * reduction of the SLAB GEMV waits for the partial sums of the slab's other workgroups for a
 * bounded time; if it gives up, the output holds NaN and the stream's status word gets
 * HALO_MI_STATUS_SPLITK_TIMEOUT. halo_mi_stream_check() synchronizes `stream`, reads and clears
 * the word and returns HALO_MI_E_DEVICE when it was set (the reference's device-loss path,
 * Stream::wait() -> Error(Device), backend.h:495-506); the workspace is then reset.
 */
#define HALO_MI_STATUS_SPLITK_TIMEOUT 0x100u
int halo_mi_stream_check(void* stream);

/*
 * Every (device, stream) pair that runs a gemv-family call gets a workspace of device memory
 * (split-K words, GEMM partials and staging, argmax parts, normalized x: about 136 MiB), allocated on the
 * first call. halo_mi_stream_release() synchronizes `stream` and frees its workspace on the
 * current device; call it before destroying the stream. A later call on the stream allocates
 * a new one.
 */
int halo_mi_stream_release(void* stream);

/*
 * Test hook, no counterpart in the reference: with force != 0 every split-K reduction of the
 * SLAB GEMV waits for a tag no partial carries, for spin_limit rounds (0 = the default bound),
 * then gives up as above; force = 0 restores normal operation. The kernels still exit
 * normally. Process-wide; for the failure-path tests only.
 */
int halo_mi_test_splitk_timeout(uint32_t spin_limit, int force);

/*
 * Measurement helper, no reference counterpart: one launch that only reads `bytes` of device
 * memory at p (16 B per load, `unroll` loads of 2/4/8/16 in flight per thread, `workgroups` of
 * 256 threads, grid-stride) and writes nothing (sink, workgroups * 256 uint32, is written only
 * for an input no benchmark uses). Its duration is the single-launch read floor of that many
 * bytes, the bound a GEMV streaming the same bytes cannot beat.
 */
int halo_mi_stream_read(const void* p, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t* sink, void* stream);

/* ---- geometry ------------------------------------------------------------------------------ */
/* Bytes of one GGUF row of `cols` elements (src/tensor/quant.cpp:411-418); 0 on error. */
uint64_t halo_mi_row_bytes(uint32_t type, uint32_t cols);
/* Bytes of the SLAB image of a rows x cols matrix (rows rounded up to 64); 0 on error. */
uint64_t halo_mi_slab_bytes(uint32_t type, uint32_t rows, uint32_t cols);

/* ---- upload and repack (north-star part (c)) ------------------------------------------------ */
/*
 * Device-side repack: GGUF rows (src_stride bytes apart, any alignment) -> SLAB image.
 * Replaces the reference's load-time repack (src/tensor/repack.cpp:100-124, called from
 * src/models/qwen35.cpp:324-346) with a layout for this backend's kernels.
 */
int halo_mi_repack_slab(uint32_t type, const void* src, uint64_t src_stride, uint32_t rows,
                        uint32_t cols, void* dst, void* stream);
/* Exact inverse on the device: SLAB image -> GGUF rows (dst_stride bytes apart, 0 = dense). */
int halo_mi_unpack_slab(uint32_t type, const void* src, uint32_t rows, uint32_t cols, void* dst,
                        uint64_t dst_stride, void* stream);
/* Host versions of the same two maps (identical bytes). */
int halo_mi_repack_slab_host(uint32_t type, const void* src, uint64_t src_stride, uint32_t rows,
                             uint32_t cols, void* dst);
int halo_mi_unpack_slab_host(uint32_t type, const void* src, uint32_t rows, uint32_t cols,
                             void* dst, uint64_t dst_stride);
/*
 * Model-scale upload: host GGUF rows (e.g. the mmap'd file, GgufFile::tensor_data,
 * src/model/gguf.cpp:540-549) -> SLAB images in device memory, for many tensors in one call.
 * Replaces Backend::import_host_readonly's device copy (src/backend/hip_adapter.cpp:502-515)
 * plus the loader's repack, and builds the row-fused projections of try_make_fused
 * (src/models/qwen35.cpp:253-288; gate|up, q|k|v, beta|alpha) on the way: a tensor's parts are
 * matrices of its type and cols whose rows are concatenated, in order, into one matrix.
 *   parts[i].src: host rows, src_stride bytes apart (0 = row_bytes); any host memory.
 *   dst: device memory of halo_mi_slab_bytes(type, sum of the parts' rows, cols) bytes,
 *        16-byte aligned; destinations must not overlap.
 *   chunk_bytes: rows move in chunks of about this size (0 = 64 MiB), whole slabs of one tensor;
 *   host_threads: threads that gather a chunk into pinned memory (0 = up to 8).
 * A three-stage pipeline over 4 chunk slots: the host gathers chunk i + 2 into pinned memory
 * while the copy engine moves chunk i + 1 (on a stream of its own) and `stream` repacks chunk i.
 * Returns after the last chunk has been repacked. The GGUF bytes remain recoverable
 * (halo_mi_unpack_slab).
 */
typedef struct halo_mi_upload_part {
    const void* src;
    uint64_t src_stride;
    uint32_t rows;
} halo_mi_upload_part;

typedef struct halo_mi_upload_tensor {
    uint32_t type;
    uint32_t cols;
    const halo_mi_upload_part* parts;
    uint32_t n_parts;
    void* dst;
} halo_mi_upload_tensor;

int halo_mi_upload_tensors(const halo_mi_upload_tensor* tensors, uint32_t n, uint64_t chunk_bytes,
                           uint32_t host_threads, void* stream);

/*
 * One tensor, one part: halo_mi_upload_tensors with host_threads = 0.
 */
int halo_mi_upload_slab(uint32_t type, const void* host_src, uint64_t src_stride, uint32_t rows,
                        uint32_t cols, void* dst, uint64_t chunk_bytes, void* stream);

/* ---- synthetic inputs (no reference counterpart: the reference has no quantizer) ----------- */
/* Portable SplitMix64 + Box-Muller normal fill: out[i] = mean + std * N(0, 1), seed-determined. */
void halo_mi_fill_normal(uint64_t seed, float* out, uint64_t n, float mean, float std);
/* fp32 -> GGUF blocks for Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_XS; n must be a multiple of the block size.
 * `threads` = 0 uses all host threads. Deterministic for any thread count. */
int halo_mi_quantize(uint32_t type, const float* src, uint64_t n, void* dst, uint32_t threads);

#ifdef __cplusplus
}
#endif

#endif
