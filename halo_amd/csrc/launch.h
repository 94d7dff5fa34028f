// Internal host-side interface between the C ABI (api.hip) and the kernel files of the
// halo_mi355x library: argument blocks, the per-stream workspace, validation helpers and the
// launchers each kernel file exports.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"
#include "slab_layout.h"

namespace halo_mi {

constexpr uint32_t kMaxGemvVec = 4;  // vectors per slab-gemv launch
// Auto choice for the fused gate/up pair: up to this many vectors an exact-product kernel (the
// GEMV pair, or the exact small-M GEMM from 3 vectors); beyond, the bf16 MFMA GEMM.
constexpr uint32_t kGateUpGemvMax = 4;

// Argmax of one vector over a range of rows: the best (value, index) by the CPU's order (higher
// value first, ties to the lower index; index kNoIndex when no row ranks) and whether any row
// of the range was NaN.
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;
struct ArgPart {
    float value;
    uint32_t index;
    uint32_t nan;
    uint32_t pad;
};

struct GemvSlabArgs {
    const uint8_t* w0;  // slab image (gate, or the only matrix)
    const uint8_t* w1;  // up matrix (PAIR) or null
    const float* x;
    uint64_t x_stride;
    float* y;           // may be null when parts is set (the logits are not kept)
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
    uint32_t ks;          // K chunks per slab
    uint64_t* slots;      // [slabs][chunks][NV][64] partials as (value, ready) words, 0 between launches
    uint32_t* counters;   // [slabs], zero between launches
    // LM head (non-pair only): the argmax of each slab's 64 rows per vector, parts[v][slab]; rows
    // at or past valid_rows (when not 0) are not ranked, but a NaN in them still counts
    ArgPart* parts = nullptr;
    uint32_t valid_rows = 0;
    // Fused input norm: y = W (rms_norm(x) * norm_w) when norm_w is set. One vector: inside the
    // MFMA kernel (every workgroup computes 1 / rms itself); otherwise the launcher normalizes x
    // into the workspace first (the RMS_NORM kernel) and the kernels see only the normalized
    // rows. Both are bitwise cpu::rms_norm then the unfused GEMV.
    const float* norm_w = nullptr;
    float norm_eps = 0.0f;
    // In-kernel norm with split K: the first workgroup alone runs the norm's chains and publishes
    // 1 / rms to every slab's word (fp32 bits and the slab's launch tag, as the split-K words);
    // the other workgroups wait for their slab's word. Null: every workgroup runs the chains.
    uint64_t* norm_words = nullptr;  // [slabs], 0 between launches (the slab's reducer clears it)
    uint32_t norm_slabs = 0;         // slabs the first workgroup publishes for
    // Workspace indexing in a grouped launch (k_gemv_mx_group): this matrix's first slab among
    // the launch's slabs, and the launch's workgroups (0: a launch of its own).
    uint32_t slab0 = 0;
    uint32_t wg_total = 0;
    // Even split (k_gemv_mx_even): the launch's `even` workgroups take equal shares of the
    // (slab, matrix, slot group) units, and a slab's pieces meet in `even_stride` word sets
    // (0: the chunked split, ks K chunks per slab). With the in-kernel norm, norm_words then
    // holds one word per workgroup (the workgroup clears it when it has read it).
    uint32_t even = 0;
    uint32_t even_stride = 0;
    float even_inv_ngrp = 0.0f, even_inv_units = 0.0f;  // 1 / slot groups per row, 1 / the launch's units
    // The stream's status word: a split-K wait that gives up sets kStatusSplitKTimeout.
    uint32_t* status = nullptr;
    // Test hooks, set only by halo_mi_test_splitk_timeout: the reducer's wait bound (0 = the
    // default) and a mask that makes it wait for a tag no chunk writes (a forced timeout).
    uint32_t spin_limit = 0;
    uint64_t tag_flip = 0;
    // The VALU slab kernel (k_gemv_slab) instead of the MFMA one (variant HALO_MI_GEMV_SLAB_VALU).
    bool valu = false;
};

// Sets a's test hooks from halo_mi_test_splitk_timeout's process-wide setting (no-op otherwise).
void apply_test_hooks(GemvSlabArgs& a);

// Split-K tickets and words. A slab's counter holds the arrivals of the running launch in its low
// kTicketBits bits and the slab's launch generation above them; a partial's word carries the
// generation (kTagMask bits of it, plus a bit that makes the tag non-zero) in its high half.
constexpr uint32_t kTicketBits = 12;
constexpr uint32_t kArrivalMask = (1u << kTicketBits) - 1;
constexpr uint32_t kMaxChunks = kArrivalMask;  // K chunks x matrices of one slab
constexpr uint32_t kTagMask = 0x7FFFFu;
// Status word bits (the stream's, read and cleared by halo_mi_stream_check).
constexpr uint32_t kStatusSplitKTimeout = 0x100u;

// M tile family of the bf16 GEMM: chosen by shape, k_gemm_pc (64..256 rows) or k_gemm_lm (512 rows)
constexpr uint32_t kGemmTilesAuto = 0, kGemmTilesPc = 1, kGemmTilesLm = 2, kGemmTilesSm = 3, kGemmTilesSx = 4,
                   kGemmTilesSxFixed = 5;  // k_gemm_sx for any n_vec, in passes of kGemmSxMaxRows
constexpr uint32_t kGemmSxMaxRows = 8;  // x rows of the exact small-M GEMM (k_gemm_sx)

struct GemmArgs {
    const uint8_t* w0;
    const uint8_t* w1;
    const float* x;
    uint64_t x_stride;
    float* y;
    uint64_t y_stride;
    uint32_t rows, cols, n_vec;
    uint32_t tiles = kGemmTilesAuto;  // M tile family: kGemmTiles*
    // Fused input norm: x is normalized exactly as cpu::rms_norm while it is staged as bf16
    const float* norm_w = nullptr;
    float norm_eps = 0.0f;
};

// ---- split-K workspace, one per (device, stream) ------------------------------------------
// Calls on one stream run in order, so they can share it. It is allocated on the first call
// on a stream (hipMalloc; counters cleared by a fill kernel on that stream, never a memset);
// a call on a stream that is being captured into a graph and has no workspace yet runs
// without split-K.
constexpr uint64_t kPartialFloats = 8ull << 20;  // GEMM split-tile partials: 32 MiB
constexpr uint64_t kSlots = 4ull << 20;          // GEMV split-K words: 32 MiB
constexpr uint64_t kCounters = 1ull << 20;        // slabs (64M rows)
constexpr uint64_t kXbElems = 16ull << 20;        // bf16 copy of x for the GEMM: 32 MiB
constexpr uint64_t kArgParts = 1ull << 20;        // LM-head argmax parts (16 B each): 16 MiB
constexpr uint64_t kNormFloats = 4ull << 20;      // normalized x rows (reference-order GEMV): 16 MiB
constexpr uint64_t kInvFloats = 1ull << 20;       // per-row 1 / rms of x (GEMM staging): 4 MiB

struct Workspace {
    uint32_t* status = nullptr;  // one word: kStatus* bits set by the kernels since the last check
    float* partials = nullptr;
    uint64_t* slots = nullptr;
    uint32_t* counters = nullptr;
    __bf16* xb = nullptr;
    ArgPart* parts = nullptr;
    float* xn = nullptr;
    float* inv = nullptr;
};

// The workspace of (current device, st); *out is null when st is being captured and has none yet.
int workspace_for(hipStream_t st, Workspace** out);

// HIP status -> library status (HALO_MI_E_DEVICE with the runtime's message).
int hip_status(hipError_t e, const char* op);
// Whether byte ranges [a, a + na) and [b, b + nb) overlap (empty ranges never do).
bool ranges_overlap(const void* a, uint64_t na, const void* b, uint64_t nb);
// Extent in bytes of `rows` rows of `row_bytes` spaced `stride` bytes apart.
uint64_t extent(uint64_t rows, uint64_t stride, uint64_t row_bytes);
// Common checks for the x / y operands of a gemv-shaped call.
int check_xy(const char* op, const float* x, uint64_t x_stride, const float* y, uint64_t y_stride, uint32_t rows,
             uint32_t cols, uint32_t n_vec);

// The no-alloc scratch's status word on the current device (0 when halo_mi_gemv_noalloc never ran
// here), read on st and cleared with the scratch's words and counters when set.
int noalloc_status_take(hipStream_t st, uint32_t* word);

// The kernel variant the auto ids (0 and 4 on a SLAB call; 0 of the gate/up pair) run for a shape.
uint32_t auto_gemv_variant(uint32_t type, uint32_t rows, uint32_t cols, uint32_t n_vec, bool pair);

// The checks halo_mi_gemv makes on a SLAB-layout call, bar the variant id: shapes, strides,
// alignment, overlap and the fused norm's operand. xs / ys receive the resolved strides (floats).
int check_gemv_slab_call(const halo_mi_gemv_params* p, const char* op, uint64_t* xs, uint64_t* ys);

// ---- launchers (arguments already validated; they return a status) ---------------------------
// k_dequant.hip
int launch_repack_slab(uint32_t type, const uint8_t* src, uint64_t src_stride, uint32_t rows, uint32_t cols,
                       uint8_t* dst, hipStream_t st);
int launch_unpack_slab(uint32_t type, const uint8_t* src, uint32_t rows, uint32_t cols, uint8_t* dst,
                       uint64_t dst_stride, hipStream_t st);
// Rows [first_row, first_row + n_rows) of W, or with ids the rows ids[0 .. n_rows) (GET_ROWS):
// an id outside [0, table_rows) leaves its output row unwritten and sets kStatusBadIndex in
// *status (when given).
int launch_dequant_gguf(uint32_t type, const uint8_t* w, uint64_t w_stride, uint32_t cols, uint32_t first_row,
                        uint32_t n_rows, float* out, uint64_t out_stride, hipStream_t st, const int32_t* ids = nullptr,
                        uint32_t table_rows = 0, uint32_t* status = nullptr);
int launch_dequant_slab(uint32_t type, const uint8_t* w, uint32_t cols, uint32_t first_row, uint32_t n_rows, float* out,
                        uint64_t out_stride, hipStream_t st, const int32_t* ids = nullptr, uint32_t table_rows = 0,
                        uint32_t* status = nullptr);
constexpr uint32_t kStatusBadIndex = 8u;  // the reference's status bit for a GET_ROWS id outside the table
int launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t st);
// The read floor's stream (halo_mi_stream_read): unroll 2, 4, 8 or 16 loads of 16 B per thread.
int launch_stream_read(const void* p, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t* sink, hipStream_t st);
// k_gemv.hip
int launch_gemv_gguf_ref(uint32_t type, const uint8_t* w, uint64_t w_stride, const float* x, uint64_t x_stride, float* y,
                         uint64_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_vec, hipStream_t st);
template <bool PAIR>
int launch_gemv_slab(uint32_t type, GemvSlabArgs a, hipStream_t st);
// k_gemv_group.hip: SLAB matrices sharing x in one launch per pair of weight types
struct GroupSeg {
    uint32_t type;
    const void* w;
    uint32_t rows;
    float* y;
    uint64_t y_stride;  // floats, already resolved (not 0)
};
int launch_gemv_group(const GroupSeg* segs, uint32_t n, const float* x, uint64_t x_stride, uint32_t cols, uint32_t n_vec,
                      const float* norm_w, float eps, hipStream_t st);
// k_gemm.hip: the same segments on the bf16 MFMA GEMM (x staged once, one launch per type pair)
int launch_gemm_group(const GroupSeg* segs, uint32_t n, const float* x, uint64_t x_stride, uint32_t cols, uint32_t n_vec,
                      const float* norm_w, float eps, hipStream_t st);
// k_gemm.hip
template <bool PAIR>
int launch_gemm_pc(uint32_t type, const GemmArgs& a, hipStream_t st);
// k_gemm_sx.hip: the exact-product small-M GEMM (1..kGemmSxMaxRows rows of x, cols a multiple
// of 256). gemm_sx_plan: whether a shape fits, its K chunks (those of kGemmSxMaxRows vectors
// whatever n_vec is, so rows do not depend on n_vec) and LDS bytes.
bool gemm_sx_plan(uint32_t units, uint32_t cols, uint32_t n_vec, uint32_t* kc, size_t* lds);
int launch_gemm_sx(uint32_t type, bool pair, const GemmArgs& g, Workspace* ws, uint32_t units, hipStream_t st);
// k_argmax.hip: stage 1 over a logits buffer (64-row parts, as the fused GEMV epilogue writes
// them), and stage 2: parts -> the result words, ids and scattered ids of each vector
int launch_argmax_parts(const float* logits, uint64_t stride, uint32_t rows, uint32_t n_vec, uint32_t valid_rows,
                        ArgPart* parts, hipStream_t st);
int launch_argmax_finish(const ArgPart* parts, uint32_t n_parts, uint32_t n_vec, uint32_t* result, int32_t* ids,
                         const uint32_t* ids_slots, int32_t* ids_scatter, uint64_t scatter_len, hipStream_t st);
int launch_swiglu(const float* g, uint64_t gs, const float* u, uint64_t us, float* out, uint64_t os, uint32_t rows,
                  uint32_t cols, hipStream_t st);
// k_norm.hip: cpu::rms_norm, bitwise (the sum of squares in cpu::detail::dot's order). out may
// be x itself (same stride). inv_rows: only the per-row 1 / sqrt(mean + eps), for the staging
// of a normalized x.
int launch_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride, uint32_t rows,
                    uint32_t cols, float eps, hipStream_t st);
int launch_rms_inv(const float* x, uint64_t x_stride, uint32_t rows, uint32_t cols, float eps, float* inv,
                   hipStream_t st);

}  // namespace halo_mi
