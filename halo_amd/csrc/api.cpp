// The extern "C" entry points of the halo_mi355x library (include/halo_mi355x.h): argument
// validation with the reference's error mapping (include/halo/backend/backend.h:24-26), the
// per-stream workspace, and the dispatch to the kernel files' launchers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "launch.h"

namespace halo_mi {

int hip_status(hipError_t e, const char* op) {
    if (e == hipSuccess) return HALO_MI_OK;
    return set_error(HALO_MI_E_DEVICE, "%s: %s", op, hipGetErrorString(e));
}

bool ranges_overlap(const void* a, uint64_t na, const void* b, uint64_t nb) {
    if (na == 0 || nb == 0 || a == nullptr || b == nullptr) return false;
    const auto pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + nb && pb < pa + na;
}

uint64_t extent(uint64_t rows, uint64_t stride, uint64_t row_bytes) { return rows ? (rows - 1) * stride + row_bytes : 0; }



namespace {
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, Workspace> g_ws;
// halo_mi_test_splitk_timeout's setting (0 / false: the kernels' own defaults)
std::atomic<uint32_t> g_test_spin_limit{0};
std::atomic<bool> g_test_flip{false};

void free_workspace(Workspace& w) {
    void* bufs[] = {w.status, w.partials, w.slots, w.counters, w.xb, w.parts, w.xn, w.inv};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    w = Workspace{};
}

// Clears the counters, the split-K words and the status word (fill kernels on st, never a memset).
int clear_workspace(const Workspace& w, hipStream_t st) {
    if (launch_fill_u32(w.counters, kCounters, 0u, st) != HALO_MI_OK ||
        launch_fill_u32(reinterpret_cast<uint32_t*>(w.slots), 2 * kSlots, 0u, st) != HALO_MI_OK ||
        launch_fill_u32(w.status, 1, 0u, st) != HALO_MI_OK)
        return set_error(HALO_MI_E_DEVICE, "workspace: clearing failed");
    return HALO_MI_OK;
}
}  // namespace

void apply_test_hooks(GemvSlabArgs& a) {
    a.spin_limit = g_test_spin_limit.load(std::memory_order_relaxed);
    a.tag_flip = g_test_flip.load(std::memory_order_relaxed) ? (1ull << 63) : 0ull;
}

int workspace_for(hipStream_t st, Workspace** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "gemv: hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find({dev, st});
    if (it != g_ws.end()) {
        *out = &it->second;
        return HALO_MI_OK;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (st != nullptr && hipStreamIsCapturing(st, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
        *out = nullptr;  // cannot allocate under capture: caller runs without split-K
        return HALO_MI_OK;
    }
    Workspace w;
    struct Alloc {
        void** p;
        uint64_t bytes;
        const char* what;
    };
    const Alloc allocs[] = {
        {reinterpret_cast<void**>(&w.status), 256, "the status word"},
        {reinterpret_cast<void**>(&w.partials), kPartialFloats * sizeof(float), "the GEMM partials"},
        {reinterpret_cast<void**>(&w.counters), kCounters * sizeof(uint32_t), "the split-K counters"},
        {reinterpret_cast<void**>(&w.xb), kXbElems * sizeof(__bf16), "the bf16 staging buffer for x"},
        {reinterpret_cast<void**>(&w.slots), kSlots * sizeof(uint64_t), "the split-K words"},
        {reinterpret_cast<void**>(&w.parts), kArgParts * sizeof(ArgPart), "the argmax parts"},
        {reinterpret_cast<void**>(&w.xn), kNormFloats * sizeof(float), "the normalized x rows"},
        {reinterpret_cast<void**>(&w.inv), kInvFloats * sizeof(float), "the norm scales"},
    };
    for (const Alloc& al : allocs)
        if (hipMalloc(al.p, al.bytes) != hipSuccess) {
            free_workspace(w);
            return set_error(HALO_MI_E_MEMORY, "workspace: cannot allocate %s", al.what);
        }
    if (clear_workspace(w, st) != HALO_MI_OK) {
        (void)hipStreamSynchronize(st);
        free_workspace(w);
        return set_error(HALO_MI_E_DEVICE, "workspace: init failed");
    }
    *out = &(g_ws[{dev, st}] = w);
    return HALO_MI_OK;
}

int check_xy(const char* op, const float* x, uint64_t x_stride, const float* y, uint64_t y_stride, uint32_t rows,
             uint32_t cols, uint32_t n_vec) {
    if (n_vec == 0 || rows == 0 || cols == 0) return HALO_MI_OK;
    if (!x || !y) return set_error(HALO_MI_E_KERNEL, "%s: operand x or y is empty", op);
    if (n_vec > 1 && x_stride < cols)
        return set_error(HALO_MI_E_KERNEL, "%s: x row stride %llu < %u floats", op, (unsigned long long)x_stride, cols);
    if (n_vec > 1 && y_stride < rows)
        return set_error(HALO_MI_E_KERNEL, "%s: y row stride %llu < %u floats", op, (unsigned long long)y_stride, rows);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: x and y must be 4-byte aligned", op);
    if (ranges_overlap(y, extent(n_vec, y_stride * 4, (uint64_t)rows * 4), x, extent(n_vec, x_stride * 4, (uint64_t)cols * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: y overlaps x", op);
    return HALO_MI_OK;
}


// The fused norm's operand: norm_w (cols floats, 4-byte aligned) must not overlap the output.
int check_norm(const char* op, const float* norm_w, uint32_t cols, const void* out, uint64_t out_bytes) {
    if (!norm_w) return HALO_MI_OK;
    if (reinterpret_cast<uintptr_t>(norm_w) % 4) return set_error(HALO_MI_E_KERNEL, "%s: norm_w must be 4-byte aligned", op);
    if (ranges_overlap(norm_w, (uint64_t)cols * 4, out, out_bytes)) return set_error(HALO_MI_E_KERNEL, "%s: norm_w overlaps the output", op);
    return HALO_MI_OK;
}

int check_gemv_slab_call(const halo_mi_gemv_params* p, const char* op, uint64_t* xs, uint64_t* ys) {
    int code;
    (void)row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    *xs = p->x_stride ? p->x_stride : p->cols;
    *ys = p->y_stride ? p->y_stride : p->rows;
    if ((code = check_xy(op, p->x, *xs, p->y, *ys, p->rows, p->cols, p->n_vec))) return code;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    if (!p->w) return set_error(HALO_MI_E_KERNEL, "%s: operand w is empty", op);
    const uint64_t yext = extent(p->n_vec, *ys * 4, (uint64_t)p->rows * 4);
    if ((code = check_norm(op, p->norm_w, p->cols, p->y, yext))) return code;
    if (p->layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: needs the SLAB layout", op);
    if (!is_quant(p->type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    if (p->w_stride != 0) return set_error(HALO_MI_E_KERNEL, "%s: a SLAB operand has no row stride", op);
    if (reinterpret_cast<uintptr_t>(p->w) % 16) return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
    if (ranges_overlap(p->y, yext, p->w, halo_mi_slab_bytes(p->type, p->rows, p->cols)))
        return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
    return HALO_MI_OK;
}

// The GEMM's M tile family for a requested variant id (the auto ids choose by shape).
// The kernel the auto variant runs for n_vec vectors (measured on MI355X at the BASELINE shapes):
//   - the slab GEMV (exact products) up to 2 vectors (Q6_K, and Q4_K, Q5_K and IQ4_XS matrices
//     of at most 128 slabs: up to 4), where it streams the weights fastest (6144 x 5120 at 4
//     vectors: Q4_K 11.2 against 14.8 us, IQ4_XS 13.3 against 17.9, Q5_K 15.6 against 17.2; at
//     192 slabs the small-M GEMM is ahead again for Q4_K, 19.2 against 19.7 us);
//   - the exact-product small-M GEMM from 3 (gate/up pair: 3 and 4), which streams them once for
//     up to 8 vectors with the same arithmetic (plain matrices at 5..8 vectors: twice as fast as
//     two GEMV passes);
//   - above, the bf16 GEMM families (the pair from 5 vectors).
// The exact GEMM needs cols a multiple of 256 (and its workspace to hold the shape); otherwise
// the GEMV. The choice depends on the shape only, so a call with the fused norm takes the same
// kernel as rms_norm followed by the plain call.
uint32_t auto_gemv_variant(uint32_t type, uint32_t rows, uint32_t cols, uint32_t n_vec, bool pair) {
    const uint32_t slabs = (rows + kSlabRows - 1) / kSlabRows;
    const bool small = slabs <= 128 && (type == kQ4_K || type == kQ5_K || type == kIQ4_XS);
    const uint32_t gemv_max = pair ? 2u : (type == kQ6_K || small ? 4u : 2u);
    const uint32_t exact_max = pair ? kGateUpGemvMax : kGemmSxMaxRows;
    if (n_vec <= gemv_max) return HALO_MI_GEMV_SLAB;
    if (n_vec <= exact_max) {
        uint32_t kc = 0;
        size_t lds = 0;
        if (gemm_sx_plan(pair ? slabs : (slabs + 1) / 2, cols, n_vec, &kc, &lds))
            return HALO_MI_GEMM_SLAB_EXACT_SMALL_M;
        return n_vec <= 8 ? HALO_MI_GEMV_SLAB : HALO_MI_GEMM_SLAB_BF16;
    }
    return HALO_MI_GEMM_SLAB_BF16;
}

// Variant 9 where the exact GEMM's fixed split fits the shape, else the slab GEMV (variant 2):
// a function of the shape only, so rows stay independent of n_vec either way.
uint32_t exact_invariant_or_gemv(uint32_t rows, uint32_t cols, bool pair) {
    const uint32_t slabs = (rows + kSlabRows - 1) / kSlabRows;
    uint32_t kc = 0;
    size_t lds = 0;
    return gemm_sx_plan(pair ? slabs : (slabs + 1) / 2, cols, kGemmSxMaxRows, &kc, &lds)
               ? HALO_MI_GEMM_SLAB_EXACT_INVARIANT
               : HALO_MI_GEMV_SLAB;
}

uint32_t gemm_tiles(uint32_t variant) {
    switch (variant) {
        case HALO_MI_GEMM_SLAB_BF16: return kGemmTilesPc;
        case HALO_MI_GEMM_SLAB_BF16_M512: return kGemmTilesLm;
        case HALO_MI_GEMM_SLAB_BF16_SMALL_M: return kGemmTilesSm;
        case HALO_MI_GEMM_SLAB_EXACT_SMALL_M: return kGemmTilesSx;
        case HALO_MI_GEMM_SLAB_EXACT_INVARIANT: return kGemmTilesSxFixed;
        default: return kGemmTilesAuto;
    }
}

}  // namespace halo_mi

using namespace halo_mi;

extern "C" {

int halo_mi_gemv(const halo_mi_gemv_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "gemv: null params");
    const char* op = "MATMUL";
    int code;
    const uint64_t rb = row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    uint32_t variant = p->variant;
    if (variant > HALO_MI_GEMV_VARIANT_LAST)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, variant);
    if (variant == HALO_MI_GEMV_DEFAULT)
        variant = p->layout == HALO_MI_LAYOUT_SLAB ? HALO_MI_GEMV_SLAB_AUTO : HALO_MI_GEMV_GGUF_REF;
    const uint64_t xs = p->x_stride ? p->x_stride : p->cols;
    const uint64_t ys = p->y_stride ? p->y_stride : p->rows;
    if ((code = check_xy(op, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec))) return code;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    if (!p->w) return set_error(HALO_MI_E_KERNEL, "%s: operand w is empty", op);
    auto st = static_cast<hipStream_t>(stream);
    const uint64_t yext = extent(p->n_vec, ys * 4, (uint64_t)p->rows * 4);
    if ((code = check_norm(op, p->norm_w, p->cols, p->y, yext))) return code;
    if (variant == HALO_MI_GEMV_GGUF_REF) {
        if (p->layout != HALO_MI_LAYOUT_GGUF)
            return set_error(HALO_MI_E_CONFIG, "%s: variant %u needs the GGUF layout", op, variant);
        const uint64_t ws = p->w_stride ? p->w_stride : rb;
        if (p->rows > 1 && ws < rb)
            return set_error(HALO_MI_E_KERNEL, "%s: operand w row stride %llu < row bytes %llu", op, (unsigned long long)ws,
                             (unsigned long long)rb);
        if (p->type == kF32 && ((reinterpret_cast<uintptr_t>(p->w) | ws) % 4))
            return set_error(HALO_MI_E_KERNEL, "%s: operand w is not 4-byte aligned", op);
        if (ranges_overlap(p->y, yext, p->w, extent(p->rows, ws, rb))) return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
        if (!p->norm_w)
            return launch_gemv_gguf_ref(p->type, static_cast<const uint8_t*>(p->w), ws, p->x, xs, p->y, ys, p->rows,
                                        p->cols, p->n_vec, st);
        // rms_norm (bitwise cpu::rms_norm) into the workspace, then the reference-order gemv,
        // as many vectors at a time as the buffer holds
        Workspace* wsp = nullptr;
        if ((code = workspace_for(st, &wsp))) return code;
        if (!wsp) return set_error(HALO_MI_E_MEMORY, "%s: the fused norm needs this stream's workspace (make one call on it before capturing)", op);
        const uint32_t per = (uint32_t)std::min<uint64_t>(kNormFloats / p->cols, p->n_vec);
        if (per == 0) return set_error(HALO_MI_E_UNSUPPORTED, "%s: cols %u too large for the norm buffer", op, p->cols);
        for (uint32_t t0 = 0; t0 < p->n_vec; t0 += per) {
            const uint32_t n = std::min(per, p->n_vec - t0);
            if ((code = launch_rms_norm(p->x + (uint64_t)t0 * xs, xs, p->norm_w, wsp->xn, p->cols, n, p->cols, p->norm_eps, st)))
                return code;
            if ((code = launch_gemv_gguf_ref(p->type, static_cast<const uint8_t*>(p->w), ws, wsp->xn, p->cols,
                                             p->y + (uint64_t)t0 * ys, ys, p->rows, p->cols, n, st)))
                return code;
        }
        return HALO_MI_OK;
    }
    if (p->layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: variant %u needs the SLAB layout", op, variant);
    if (!is_quant(p->type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    if (p->w_stride != 0) return set_error(HALO_MI_E_KERNEL, "%s: a SLAB operand has no row stride", op);
    if (reinterpret_cast<uintptr_t>(p->w) % 16) return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
    if (ranges_overlap(p->y, yext, p->w, halo_mi_slab_bytes(p->type, p->rows, p->cols)))
        return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
    if (variant == HALO_MI_GEMV_SLAB_AUTO) variant = auto_gemv_variant(p->type, p->rows, p->cols, p->n_vec, false);
    if (variant == HALO_MI_GEMM_SLAB_EXACT_INVARIANT) variant = exact_invariant_or_gemv(p->rows, p->cols, false);
    if (variant == HALO_MI_GEMV_SLAB || variant == HALO_MI_GEMV_SLAB_VALU) {
        GemvSlabArgs a{static_cast<const uint8_t*>(p->w), nullptr, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec};
        a.norm_w = p->norm_w;
        a.norm_eps = p->norm_eps;
        a.valu = variant == HALO_MI_GEMV_SLAB_VALU;
        return launch_gemv_slab<false>(p->type, a, st);
    }
    const bool exact = variant == HALO_MI_GEMM_SLAB_EXACT_SMALL_M || variant == HALO_MI_GEMM_SLAB_EXACT_INVARIANT;
    if (!exact && (p->x_stride % 4 || reinterpret_cast<uintptr_t>(p->x) % 16))
        return set_error(HALO_MI_E_KERNEL, "%s: the bf16 MFMA GEMM needs 16-byte aligned x rows", op);
    GemmArgs a{static_cast<const uint8_t*>(p->w), nullptr, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec};
    a.tiles = exact ? gemm_tiles(variant) : gemm_tiles(p->variant);
    a.norm_w = p->norm_w;
    a.norm_eps = p->norm_eps;
    return launch_gemm_pc<false>(p->type, a, st);
}

}  // extern "C"

namespace {

// The checks both grouped entry points make (halo_mi_gemv_group's contract); segs and *xs
// receive the resolved segments and x stride. *empty: nothing to compute.
int check_group(const halo_mi_gemv_group_params* p, const char* op, GroupSeg (&segs)[HALO_MI_GEMV_GROUP_MAX], uint64_t* xs,
                bool* empty) {
    *empty = true;
    if (!p) return set_error(HALO_MI_E_KERNEL, "%s: null params", op);
    if (p->n_segs == 0 || p->n_vec == 0) return HALO_MI_OK;
    if (!p->segs) return set_error(HALO_MI_E_KERNEL, "%s: null segment list", op);
    if (p->n_segs > HALO_MI_GEMV_GROUP_MAX)
        return set_error(HALO_MI_E_UNSUPPORTED, "%s: %u segments (at most %u)", op, p->n_segs, HALO_MI_GEMV_GROUP_MAX);
    if (!p->x) return set_error(HALO_MI_E_KERNEL, "%s: operand x is empty", op);
    *xs = p->x_stride ? p->x_stride : p->cols;
    if (p->n_vec > 1 && *xs < p->cols) return set_error(HALO_MI_E_KERNEL, "%s: x row stride < cols", op);
    if (reinterpret_cast<uintptr_t>(p->x) % 4) return set_error(HALO_MI_E_KERNEL, "%s: x must be 4-byte aligned", op);
    const uint64_t xext = extent(p->n_vec, *xs * 4, (uint64_t)p->cols * 4);
    uint64_t wext[HALO_MI_GEMV_GROUP_MAX], yext[HALO_MI_GEMV_GROUP_MAX];
    for (uint32_t i = 0; i < p->n_segs; ++i) {
        const halo_mi_gemv_segment& g = p->segs[i];
        int code;
        (void)row_bytes_checked(g.type, p->cols, &code, op);
        if (code) return code;
        if (!is_quant(g.type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: segment %u: type %u has no SLAB layout", op, i, g.type);
        const uint64_t ys = g.y_stride ? g.y_stride : g.rows;
        if (g.rows && (!g.w || !g.y)) return set_error(HALO_MI_E_KERNEL, "%s: segment %u: operand w or y is empty", op, i);
        if (p->n_vec > 1 && ys < g.rows) return set_error(HALO_MI_E_KERNEL, "%s: segment %u: y row stride < rows", op, i);
        if ((reinterpret_cast<uintptr_t>(g.w) % 16) || (reinterpret_cast<uintptr_t>(g.y) % 4))
            return set_error(HALO_MI_E_KERNEL, "%s: segment %u: w must be 16-byte and y 4-byte aligned", op, i);
        wext[i] = halo_mi_slab_bytes(g.type, g.rows, p->cols);
        yext[i] = g.rows ? extent(p->n_vec, ys * 4, (uint64_t)g.rows * 4) : 0;
        segs[i] = GroupSeg{g.type, g.w, g.rows, g.y, ys};
    }
    for (uint32_t i = 0; i < p->n_segs; ++i) {
        const void* y = p->segs[i].y;
        if (ranges_overlap(y, yext[i], p->x, xext) ||
            ranges_overlap(y, yext[i], p->norm_w, p->norm_w ? (uint64_t)p->cols * 4 : 0))
            return set_error(HALO_MI_E_KERNEL, "%s: segment %u: y overlaps x or norm_w", op, i);
        for (uint32_t j = 0; j < p->n_segs; ++j) {
            if (ranges_overlap(y, yext[i], p->segs[j].w, wext[j]))
                return set_error(HALO_MI_E_KERNEL, "%s: segment %u: y overlaps the weights of segment %u", op, i, j);
            if (j != i && ranges_overlap(y, yext[i], p->segs[j].y, yext[j]))
                return set_error(HALO_MI_E_KERNEL, "%s: the outputs of segments %u and %u overlap", op, i, j);
        }
    }
    if (p->norm_w && reinterpret_cast<uintptr_t>(p->norm_w) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: norm_w must be 4-byte aligned", op);
    *empty = false;
    return HALO_MI_OK;
}

}  // namespace

extern "C" {

int halo_mi_gemv_group(const halo_mi_gemv_group_params* p, void* stream) {
    clear_error();
    GroupSeg segs[HALO_MI_GEMV_GROUP_MAX];
    uint64_t xs = 0;
    bool empty = true;
    if (int rc = check_group(p, "MATMUL_GROUP", segs, &xs, &empty)) return rc;
    if (empty) return HALO_MI_OK;
    return launch_gemv_group(segs, p->n_segs, p->x, xs, p->cols, p->n_vec, p->norm_w, p->norm_eps,
                             static_cast<hipStream_t>(stream));
}

int halo_mi_gemm_group(const halo_mi_gemv_group_params* p, void* stream) {
    clear_error();
    const char* op = "GEMM_GROUP";
    GroupSeg segs[HALO_MI_GEMV_GROUP_MAX];
    uint64_t xs = 0;
    bool empty = true;
    if (int rc = check_group(p, op, segs, &xs, &empty)) return rc;
    if (empty) return HALO_MI_OK;
    if (xs % 4 || reinterpret_cast<uintptr_t>(p->x) % 16)
        return set_error(HALO_MI_E_KERNEL, "%s: the bf16 MFMA GEMM needs 16-byte aligned x rows", op);
    return launch_gemm_group(segs, p->n_segs, p->x, xs, p->cols, p->n_vec, p->norm_w, p->norm_eps,
                             static_cast<hipStream_t>(stream));
}

int halo_mi_lm_head(const halo_mi_lm_head_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "lm_head: null params");
    const char* op = "LM_HEAD";
    const halo_mi_gemv_params& g = p->gemv;
    int code;
    const uint64_t rb = row_bytes_checked(g.type, g.cols, &code, op);
    if (code) return code;
    uint32_t variant = g.variant;
    if (variant > HALO_MI_GEMV_VARIANT_LAST)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, variant);
    const bool slab = g.layout == HALO_MI_LAYOUT_SLAB;
    const bool fused = slab && (variant == HALO_MI_GEMV_DEFAULT || variant == HALO_MI_GEMV_SLAB ||
                                variant == HALO_MI_GEMV_SLAB_AUTO || variant == HALO_MI_GEMV_SLAB_VALU);
    if (!fused && !g.y) return set_error(HALO_MI_E_KERNEL, "%s: variant %u ranks the logits: gemv.y is needed", op, variant);
    if ((p->ids_slots == nullptr) != (p->ids_scatter == nullptr) || (p->ids_scatter && !p->ids))
        return set_error(HALO_MI_E_KERNEL, "%s: ids_slots and ids_scatter go together, and only with ids", op);
    if (g.n_vec == 0) return HALO_MI_OK;
    if (!p->result) return set_error(HALO_MI_E_KERNEL, "%s: operand result is empty", op);
    if ((reinterpret_cast<uintptr_t>(p->result) | reinterpret_cast<uintptr_t>(p->ids) |
         reinterpret_cast<uintptr_t>(p->ids_slots) | reinterpret_cast<uintptr_t>(p->ids_scatter)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: result and ids must be 4-byte aligned", op);
    const uint64_t xs = g.x_stride ? g.x_stride : g.cols;
    const uint64_t ys = g.y_stride ? g.y_stride : g.rows;
    const uint64_t res_bytes = (uint64_t)g.n_vec * HALO_MI_ARGMAX_RESULT_BYTES, ids_bytes = (uint64_t)g.n_vec * 4;
    const uint64_t xext = extent(g.n_vec, xs * 4, (uint64_t)g.cols * 4), yext = g.y ? extent(g.n_vec, ys * 4, (uint64_t)g.rows * 4) : 0;
    const uint64_t wext = slab ? halo_mi_slab_bytes(g.type, g.rows, g.cols)
                               : extent(g.rows, g.w_stride ? g.w_stride : rb, rb);
    struct Out {
        const void* p;
        uint64_t n;
        const char* name;
    };
    const Out outs[] = {{p->result, res_bytes, "result"},
                        {p->ids, p->ids ? ids_bytes : 0, "ids"},
                        {p->ids_scatter, p->ids_scatter ? p->ids_scatter_len * 4 : 0, "ids_scatter"}};
    for (size_t i = 0; i < 3; ++i) {
        if (ranges_overlap(outs[i].p, outs[i].n, g.x, xext) || ranges_overlap(outs[i].p, outs[i].n, g.w, wext) ||
            ranges_overlap(outs[i].p, outs[i].n, g.y, yext) || ranges_overlap(outs[i].p, outs[i].n, p->ids_slots, p->ids_slots ? ids_bytes : 0) ||
            ranges_overlap(outs[i].p, outs[i].n, g.norm_w, g.norm_w ? (uint64_t)g.cols * 4 : 0))
            return set_error(HALO_MI_E_KERNEL, "%s: %s overlaps an operand", op, outs[i].name);
        for (size_t j = 0; j < i; ++j)
            if (ranges_overlap(outs[i].p, outs[i].n, outs[j].p, outs[j].n))
                return set_error(HALO_MI_E_KERNEL, "%s: %s overlaps %s", op, outs[i].name, outs[j].name);
    }
    if (g.rows == 0) return set_error(HALO_MI_E_KERNEL, "%s: no rows to rank", op);
    auto st = static_cast<hipStream_t>(stream);
    Workspace* ws = nullptr;
    if ((code = workspace_for(st, &ws))) return code;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "%s: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)", op);
    const uint32_t n_parts = (g.rows + kSlabRows - 1) / kSlabRows;
    if ((uint64_t)n_parts * g.n_vec > kArgParts)
        return set_error(HALO_MI_E_UNSUPPORTED, "%s: %u vectors of %u rows exceed the argmax workspace", op, g.n_vec, g.rows);
    if (fused) {
        // halo_mi_gemv's checks, with y optional
        if (!g.x) return set_error(HALO_MI_E_KERNEL, "%s: operand x is empty", op);
        if (g.n_vec > 1 && xs < g.cols) return set_error(HALO_MI_E_KERNEL, "%s: x row stride %llu < %u floats", op,
                                                        (unsigned long long)xs, g.cols);
        if (reinterpret_cast<uintptr_t>(g.x) % 4) return set_error(HALO_MI_E_KERNEL, "%s: x must be 4-byte aligned", op);
        if (g.y && ((code = check_xy(op, g.x, xs, g.y, ys, g.rows, g.cols, g.n_vec)))) return code;
        if (!is_quant(g.type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, g.type);
        if (!g.w) return set_error(HALO_MI_E_KERNEL, "%s: operand w is empty", op);
        if (g.w_stride != 0) return set_error(HALO_MI_E_KERNEL, "%s: a SLAB operand has no row stride", op);
        if (reinterpret_cast<uintptr_t>(g.w) % 16) return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
        if (ranges_overlap(g.y, yext, g.w, wext)) return set_error(HALO_MI_E_KERNEL, "%s: y overlaps w", op);
        if ((code = check_norm(op, g.norm_w, g.cols, g.y, yext))) return code;
        GemvSlabArgs a{static_cast<const uint8_t*>(g.w), nullptr, g.x, xs, g.y, ys, g.rows, g.cols, g.n_vec};
        a.parts = ws->parts;
        a.valid_rows = p->valid_rows;
        a.norm_w = g.norm_w;
        a.norm_eps = g.norm_eps;
        a.valu = variant == HALO_MI_GEMV_SLAB_VALU;
        if ((code = launch_gemv_slab<false>(g.type, a, st))) return code;
    } else {
        if ((code = halo_mi_gemv(&g, stream))) return code;
        if ((code = launch_argmax_parts(g.y, ys, g.rows, g.n_vec, p->valid_rows, ws->parts, st))) return code;
    }
    return launch_argmax_finish(ws->parts, n_parts, g.n_vec, static_cast<uint32_t*>(p->result), p->ids, p->ids_slots,
                                p->ids_scatter, p->ids_scatter_len, st);
}

int halo_mi_gate_up_swiglu(const halo_mi_gate_up_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "gate_up: null params");
    const char* op = "GATE_UP_SWIGLU";
    int code;
    (void)row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    if (p->layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: needs the SLAB layout", op);
    if (!is_quant(p->type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    uint32_t variant = p->variant;
    if (variant == HALO_MI_GEMV_GGUF_REF || variant > HALO_MI_GEMV_VARIANT_LAST)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, variant);
    const uint64_t xs = p->x_stride ? p->x_stride : p->cols;
    const uint64_t os = p->out_stride ? p->out_stride : p->rows;
    if ((code = check_xy(op, p->x, xs, p->out, os, p->rows, p->cols, p->n_vec))) return code;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    if (!p->w_gate || !p->w_up) return set_error(HALO_MI_E_KERNEL, "%s: operand w_gate or w_up is empty", op);
    if ((reinterpret_cast<uintptr_t>(p->w_gate) | reinterpret_cast<uintptr_t>(p->w_up)) % 16)
        return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
    const uint64_t wbytes = halo_mi_slab_bytes(p->type, p->rows, p->cols);
    const uint64_t oext = extent(p->n_vec, os * 4, (uint64_t)p->rows * 4);
    if (ranges_overlap(p->out, oext, p->w_gate, wbytes) || ranges_overlap(p->out, oext, p->w_up, wbytes))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps a weight operand", op);
    if ((code = check_norm(op, p->norm_w, p->cols, p->out, oext))) return code;
    if (variant == HALO_MI_GEMV_DEFAULT || variant == HALO_MI_GEMV_SLAB_AUTO)
        variant = auto_gemv_variant(p->type, p->rows, p->cols, p->n_vec, true);
    if (variant == HALO_MI_GEMM_SLAB_EXACT_INVARIANT) variant = exact_invariant_or_gemv(p->rows, p->cols, true);
    auto st = static_cast<hipStream_t>(stream);
    if (variant == HALO_MI_GEMV_SLAB || variant == HALO_MI_GEMV_SLAB_VALU) {
        GemvSlabArgs a{static_cast<const uint8_t*>(p->w_gate), static_cast<const uint8_t*>(p->w_up), p->x, xs, p->out, os,
                       p->rows, p->cols, p->n_vec};
        a.norm_w = p->norm_w;
        a.norm_eps = p->norm_eps;
        a.valu = variant == HALO_MI_GEMV_SLAB_VALU;
        return launch_gemv_slab<true>(p->type, a, st);
    }
    const bool exact = variant == HALO_MI_GEMM_SLAB_EXACT_SMALL_M || variant == HALO_MI_GEMM_SLAB_EXACT_INVARIANT;
    if (!exact && (xs % 4 || reinterpret_cast<uintptr_t>(p->x) % 16))
        return set_error(HALO_MI_E_KERNEL, "%s: the bf16 MFMA GEMM needs 16-byte aligned x rows", op);
    GemmArgs a{static_cast<const uint8_t*>(p->w_gate), static_cast<const uint8_t*>(p->w_up), p->x, xs, p->out, os,
               p->rows, p->cols, p->n_vec};
    a.tiles = exact ? gemm_tiles(variant) : gemm_tiles(p->variant);
    a.norm_w = p->norm_w;
    a.norm_eps = p->norm_eps;
    return launch_gemm_pc<true>(p->type, a, st);
}

int halo_mi_argmax(const float* logits, uint64_t logits_stride, uint32_t n, uint32_t n_vec, void* result, void* stream) {
    clear_error();
    const char* op = "ARGMAX_FUSED";
    if (n_vec == 0) return HALO_MI_OK;
    if (n == 0) return set_error(HALO_MI_E_KERNEL, "%s: empty row", op);
    if (!logits || !result) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    const uint64_t ls = logits_stride ? logits_stride : n;
    if (n_vec > 1 && ls < n) return set_error(HALO_MI_E_KERNEL, "%s: logits row stride < n", op);
    if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(result)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: operands must be 4-byte aligned", op);
    if (ranges_overlap(result, (uint64_t)n_vec * HALO_MI_ARGMAX_RESULT_BYTES, logits, extent(n_vec, ls * 4, (uint64_t)n * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: result overlaps logits", op);
    auto st = static_cast<hipStream_t>(stream);
    Workspace* ws = nullptr;
    int code;
    if ((code = workspace_for(st, &ws))) return code;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "%s: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)", op);
    const uint32_t n_parts = (n + kSlabRows - 1) / kSlabRows;
    if ((uint64_t)n_parts * n_vec > kArgParts)
        return set_error(HALO_MI_E_UNSUPPORTED, "%s: %u rows of %u exceed the argmax workspace", op, n_vec, n);
    if ((code = launch_argmax_parts(logits, ls, n, n_vec, 0, ws->parts, st))) return code;
    return launch_argmax_finish(ws->parts, n_parts, n_vec, static_cast<uint32_t*>(result), nullptr, nullptr, nullptr, 0, st);
}

int halo_mi_swiglu(const float* gate, uint64_t gate_stride, const float* up, uint64_t up_stride, float* out,
                   uint64_t out_stride, uint32_t rows, uint32_t cols, void* stream) {
    clear_error();
    const char* op = "SWIGLU";
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (!gate || !up || !out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (gate_stride == 0) gate_stride = cols;
    if (up_stride == 0) up_stride = cols;
    if (out_stride == 0) out_stride = cols;
    if (rows > 1 && (gate_stride < cols || up_stride < cols || out_stride < cols))
        return set_error(HALO_MI_E_KERNEL, "%s: row stride < cols", op);
    if ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(out)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: operands must be 4-byte aligned", op);
    const uint64_t oext = extent(rows, out_stride * 4, (uint64_t)cols * 4);
    if (ranges_overlap(out, oext, gate, extent(rows, gate_stride * 4, (uint64_t)cols * 4)) ||
        ranges_overlap(out, oext, up, extent(rows, up_stride * 4, (uint64_t)cols * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps an input", op);
    return launch_swiglu(gate, gate_stride, up, up_stride, out, out_stride, rows, cols, static_cast<hipStream_t>(stream));
}

int halo_mi_dequant_rows(uint32_t type, uint32_t layout, const void* w, uint64_t w_stride, uint32_t rows, uint32_t cols,
                         uint32_t first_row, uint32_t n_rows, float* out, uint64_t out_stride, void* stream) {
    clear_error();
    const char* op = "DEQUANT";
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, op);
    if (code) return code;
    if (first_row > rows || n_rows > rows - first_row)
        return set_error(HALO_MI_E_KERNEL, "%s: rows [%u, %u) out of %u", op, first_row, first_row + n_rows, rows);
    if (n_rows == 0 || cols == 0) return HALO_MI_OK;
    if (!w || !out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (out_stride == 0) out_stride = cols;
    if (n_rows > 1 && out_stride < cols) return set_error(HALO_MI_E_KERNEL, "%s: out stride < cols", op);
    auto st = static_cast<hipStream_t>(stream);
    if (layout == HALO_MI_LAYOUT_GGUF) {
        if (w_stride == 0) w_stride = rb;
        if (rows > 1 && w_stride < rb) return set_error(HALO_MI_E_KERNEL, "%s: w stride < row bytes", op);
        return launch_dequant_gguf(type, static_cast<const uint8_t*>(w), w_stride, cols, first_row, n_rows, out, out_stride,
                                   st);
    }
    if (layout != HALO_MI_LAYOUT_SLAB) return set_error(HALO_MI_E_CONFIG, "%s: unknown layout %u", op, layout);
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, type);
    return launch_dequant_slab(type, static_cast<const uint8_t*>(w), cols, first_row, n_rows, out, out_stride, st);
}

int halo_mi_get_rows(const halo_mi_get_rows_params* p, void* stream) {
    clear_error();
    if (!p) return set_error(HALO_MI_E_KERNEL, "get_rows: null params");
    const char* op = "GET_ROWS";
    int code;
    const uint64_t rb = row_bytes_checked(p->type, p->cols, &code, op);
    if (code) return code;
    if (p->n_rows > 0x7FFFFFFFu) return set_error(HALO_MI_E_KERNEL, "%s: n_rows %u exceeds int32 ids", op, p->n_rows);
    if (p->layout != HALO_MI_LAYOUT_GGUF && p->layout != HALO_MI_LAYOUT_SLAB)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown layout %u", op, p->layout);
    if (p->layout == HALO_MI_LAYOUT_SLAB && !is_quant(p->type))
        return set_error(HALO_MI_E_UNSUPPORTED, "%s: type %u has no SLAB layout", op, p->type);
    auto st = static_cast<hipStream_t>(stream);
    if (p->status) {
        if (reinterpret_cast<uintptr_t>(p->status) % 4) return set_error(HALO_MI_E_KERNEL, "%s: status must be 4-byte aligned", op);
        if (!p->status_keep && (code = launch_fill_u32(p->status, 1, 0u, st))) return code;
    }
    if (p->n_ids == 0 || p->cols == 0) return HALO_MI_OK;
    if (!p->table || !p->ids || !p->out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (p->n_rows == 0) return set_error(HALO_MI_E_KERNEL, "%s: the table has no rows", op);
    const uint64_t os = p->out_stride ? p->out_stride : p->cols;
    if (p->n_ids > 1 && os < p->cols) return set_error(HALO_MI_E_KERNEL, "%s: out stride < cols", op);
    if ((reinterpret_cast<uintptr_t>(p->out) | reinterpret_cast<uintptr_t>(p->ids)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: out and ids must be 4-byte aligned", op);
    uint64_t ts = p->table_stride, tbytes;
    if (p->layout == HALO_MI_LAYOUT_GGUF) {
        if (ts == 0) ts = rb;
        if (p->n_rows > 1 && ts < rb) return set_error(HALO_MI_E_KERNEL, "%s: table stride < row bytes", op);
        if (p->type == kF32 && ((reinterpret_cast<uintptr_t>(p->table) | ts) % 4))
            return set_error(HALO_MI_E_KERNEL, "%s: an F32 table must be 4-byte aligned", op);
        tbytes = extent(p->n_rows, ts, rb);
    } else {
        if (ts != 0) return set_error(HALO_MI_E_KERNEL, "%s: a SLAB operand has no row stride", op);
        if (reinterpret_cast<uintptr_t>(p->table) % 16) return set_error(HALO_MI_E_KERNEL, "%s: SLAB weights must be 16-byte aligned", op);
        tbytes = halo_mi_slab_bytes(p->type, p->n_rows, p->cols);
    }
    const uint64_t oext = extent(p->n_ids, os * 4, (uint64_t)p->cols * 4);
    if (ranges_overlap(p->out, oext, p->table, tbytes) || ranges_overlap(p->out, oext, p->ids, (uint64_t)p->n_ids * 4) ||
        ranges_overlap(p->out, oext, p->status, p->status ? 4 : 0))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps an operand", op);
    if (ranges_overlap(p->status, p->status ? 4 : 0, p->table, tbytes) ||
        ranges_overlap(p->status, p->status ? 4 : 0, p->ids, (uint64_t)p->n_ids * 4))
        return set_error(HALO_MI_E_KERNEL, "%s: status overlaps an operand", op);
    if (p->layout == HALO_MI_LAYOUT_GGUF)
        return launch_dequant_gguf(p->type, static_cast<const uint8_t*>(p->table), ts, p->cols, 0, p->n_ids, p->out, os, st,
                                   p->ids, p->n_rows, p->status);
    return launch_dequant_slab(p->type, static_cast<const uint8_t*>(p->table), p->cols, 0, p->n_ids, p->out, os, st, p->ids,
                               p->n_rows, p->status);
}

int halo_mi_rms_norm(const float* x, uint64_t x_stride, const float* w, float* out, uint64_t out_stride, uint32_t rows,
                     uint32_t cols, float eps, void* stream) {
    clear_error();
    const char* op = "RMS_NORM";
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (!x || !w || !out) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (x_stride == 0) x_stride = cols;
    if (out_stride == 0) out_stride = cols;
    if (rows > 1 && (x_stride < cols || out_stride < cols)) return set_error(HALO_MI_E_KERNEL, "%s: row stride < cols", op);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: operands must be 4-byte aligned", op);
    const uint64_t oext = extent(rows, out_stride * 4, (uint64_t)cols * 4);
    const bool same = out == x && out_stride == x_stride;  // in place, as cpu::rms_norm allows
    if (!same && ranges_overlap(out, oext, x, extent(rows, x_stride * 4, (uint64_t)cols * 4)))
        return set_error(HALO_MI_E_KERNEL, "%s: out overlaps x", op);
    if (ranges_overlap(out, oext, w, (uint64_t)cols * 4)) return set_error(HALO_MI_E_KERNEL, "%s: out overlaps w", op);
    return launch_rms_norm(x, x_stride, w, out, out_stride, rows, cols, eps, static_cast<hipStream_t>(stream));
}

int halo_mi_repack_slab(uint32_t type, const void* src, uint64_t src_stride, uint32_t rows, uint32_t cols, void* dst,
                        void* stream) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "repack_slab");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "repack_slab: type %u has no SLAB layout", type);
    if (src_stride == 0) src_stride = rb;
    if (rows > 1 && src_stride < rb) return set_error(HALO_MI_E_KERNEL, "repack_slab: row stride < row bytes");
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    if (ranges_overlap(dst, halo_mi_slab_bytes(type, rows, cols), src, extent(rows, src_stride, rb)))
        return set_error(HALO_MI_E_KERNEL, "repack_slab: dst overlaps src");
    return launch_repack_slab(type, static_cast<const uint8_t*>(src), src_stride, rows, cols, static_cast<uint8_t*>(dst),
                              static_cast<hipStream_t>(stream));
}

int halo_mi_unpack_slab(uint32_t type, const void* src, uint32_t rows, uint32_t cols, void* dst, uint64_t dst_stride,
                        void* stream) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "unpack_slab");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "unpack_slab: type %u has no SLAB layout", type);
    if (dst_stride == 0) dst_stride = rb;
    if (rows > 1 && dst_stride < rb) return set_error(HALO_MI_E_KERNEL, "unpack_slab: row stride < row bytes");
    if (rows == 0 || cols == 0) return HALO_MI_OK;
    return launch_unpack_slab(type, static_cast<const uint8_t*>(src), rows, cols, static_cast<uint8_t*>(dst), dst_stride,
                              static_cast<hipStream_t>(stream));
}

int halo_mi_stream_read(const void* p, uint64_t bytes, uint32_t workgroups, uint32_t unroll, uint32_t* sink, void* stream) {
    clear_error();
    const char* op = "stream_read";
    if (bytes == 0) return HALO_MI_OK;
    if (!p || !sink) return set_error(HALO_MI_E_KERNEL, "%s: empty operand", op);
    if (bytes % 16 || reinterpret_cast<uintptr_t>(p) % 16 || reinterpret_cast<uintptr_t>(sink) % 4)
        return set_error(HALO_MI_E_KERNEL, "%s: p and bytes must be 16-byte aligned, sink 4-byte aligned", op);
    if (workgroups == 0 || workgroups > (1u << 20)) return set_error(HALO_MI_E_KERNEL, "%s: workgroups out of range", op);
    if (unroll != 2 && unroll != 4 && unroll != 8 && unroll != 16)
        return set_error(HALO_MI_E_KERNEL, "%s: unroll must be 2, 4, 8 or 16", op);
    return launch_stream_read(p, bytes, workgroups, unroll, sink, static_cast<hipStream_t>(stream));
}

int halo_mi_stream_check(void* stream) {
    clear_error();
    auto st = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "stream_check: hipGetDevice failed");
    // both status words are read and cleared before anything is reported: the no-alloc scratch's
    // (shared by the device) and this stream's workspace's
    uint32_t na_word = 0;
    if (int rc = noalloc_status_take(st, &na_word)) return rc;
    uint32_t word = 0;
    Workspace w;
    bool have_ws = false;
    {
        std::lock_guard<std::mutex> lock(g_ws_mu);
        auto it = g_ws.find({dev, st});
        if (it != g_ws.end()) {
            w = it->second;
            have_ws = true;
        }
    }
    if (have_ws) {
        if (int rc = hip_status(hipMemcpyAsync(&word, w.status, sizeof(word), hipMemcpyDeviceToHost, st), "stream_check"))
            return rc;
        if (int rc = hip_status(hipStreamSynchronize(st), "stream_check")) return rc;
        if (word != 0) {
            // the words and counters of a wait that gave up are in an unknown state: start again clean
            if (int rc = clear_workspace(w, st)) return rc;
        }
    }
    if (int rc = hip_status(hipStreamSynchronize(st), "stream_check")) return rc;
    if (word == 0 && na_word == 0) return HALO_MI_OK;
    return set_error(HALO_MI_E_DEVICE, "stream_check: a split-K reduction gave up waiting for partial sums (stream "
                                       "workspace status 0x%x, halo_mi_gemv_noalloc scratch status 0x%x); outputs written "
                                       "since the last check hold NaN", word, na_word);
}

int halo_mi_stream_release(void* stream) {
    clear_error();
    auto st = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "stream_release: hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mu);
    auto it = g_ws.find({dev, st});
    if (it == g_ws.end()) return HALO_MI_OK;
    const int rc = hip_status(hipStreamSynchronize(st), "stream_release");
    free_workspace(it->second);
    g_ws.erase(it);
    return rc;
}

int halo_mi_test_splitk_timeout(uint32_t spin_limit, int force) {
    clear_error();
    g_test_spin_limit.store(spin_limit, std::memory_order_relaxed);
    g_test_flip.store(force != 0, std::memory_order_relaxed);
    return HALO_MI_OK;
}

}  // extern "C"
