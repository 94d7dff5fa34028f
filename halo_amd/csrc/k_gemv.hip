// gfx950 GEMV kernels of the halo_mi355x library (M = 1..8):
//   k_gemv_gguf_ref  GGUF layout, 8 lanes per output in cpu::detail::dot's order
//                    (backends/cpu/kernel_common.h:16-27 of the reference): bit-identical to the
//                    CPU backend.
//   k_gemv_slab      SLAB layout, VALU: one row per lane, a wave streams 64 rows slot by slot.
//   k_gemv_mx        SLAB layout, the same stream with the multiply-adds on
//                    v_mfma_f32_4x4x4_16b_bf16 (the default).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "gemv_device.h"

namespace halo_mi {
namespace {

using namespace dev;

// Work split of a slab-GEMV launch: ks K chunks per slab (more than one only when the slabs
// alone cannot fill the chip; the chunks then meet in the workspace), nw waves per workgroup
// (about two slot groups per wave, so each wave streams with one group in flight).
struct GemvSplit {
    uint32_t ks, nw;
};

// words: workspace words per (slab, chunk) and vector (64 partials, plus one with the norm).
GemvSplit pick_split(uint32_t slabs, uint32_t S, uint32_t nv, uint32_t mats, bool have_ws, uint32_t words) {
    // One slot group per wave for mid-size matrices, two for large ones (measured on MI355X,
    // 17408 x 5120 and 151936 x 5120 Q4_K).
    static const uint32_t target_env = [] {
        const char* e = std::getenv("HALO_MI_GEMV_WGS");  // tuning knob: min workgroups per launch
        return e ? (uint32_t)std::max(1, std::atoi(e)) : 0u;
    }();
    static const int gpw_env = [] {
        const char* e = std::getenv("HALO_MI_GEMV_GPW");  // tuning knob: slot groups per wave
        return e ? std::max(1, std::atoi(e)) : 0;
    }();
    const uint32_t groups_per_wave = gpw_env ? (uint32_t)gpw_env : (slabs >= 1024 ? 2u : 1u);
    const uint32_t ngrp = (S + 7) / 8;
    uint32_t ks = 1;
    const uint32_t units = std::max(slabs, 1u) * mats;
    // Measured on MI355X: about 4 workgroups per slab up to 1088 per launch; small matrices
    // gain more from a short split-K fix-up than from more workgroups (floor of 128).
    const uint32_t target_wg = target_env ? target_env : std::clamp(4 * units, 128u, 1088u);
    if (have_ws && units < target_wg) ks = std::min((target_wg + units - 1) / units, ngrp);
    while (ks > 1 && (uint64_t)slabs * ks * mats * nv * words > kSlots) --ks;
    const uint32_t gwg = (ngrp + ks - 1) / ks;
    uint32_t nw = std::clamp((gwg + groups_per_wave - 1) / groups_per_wave, 1u, 16u);
    // a wave holds the x sums of at most 4 groups (one per lane)
    while (ks < ngrp && (gwg + nw - 1) / nw > 4) {
        if (nw < 16) ++nw;
        else ++ks;
        const uint32_t g2 = (ngrp + ks - 1) / ks;
        if ((g2 + nw - 1) / nw <= 4) break;
    }
    return {ks, nw};
}

template <uint32_t T, int NV, bool PAIR>
int launch_gemv_slab_t(GemvSlabArgs a, uint32_t slabs, Workspace* ws, hipStream_t st) {
    const uint32_t S = a.cols / kSlot;
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    const uint32_t words = a.norm_w ? 65u : 64u;
    const GemvSplit sp = pick_split(slabs, S, NV, MATS, ws != nullptr && slabs <= kCounters, words);
    a.ks = sp.ks;
    a.slots = ws ? ws->slots : nullptr;
    a.counters = ws ? ws->counters : nullptr;
    static const bool valu = [] {
        const char* e = std::getenv("HALO_MI_GEMV_VALU");
        return e && *e == '1';
    }();
    if constexpr (T != kQ5_K && T != kIQ4_XS) {  // the VALU kernel covers the first four formats
        if (valu && !a.norm_w) {
            if (a.ks * MATS > 1 && (uint64_t)slabs * a.ks * MATS * NV * 64 > kSlots)
                return set_error(HALO_MI_E_UNSUPPORTED, "gemv: %u rows exceed the split-K workspace", a.rows);
            const size_t lds = (size_t)sp.nw * NV * 64 * sizeof(float);
            hipLaunchKernelGGL((k_gemv_slab<T, NV, PAIR>), dim3(slabs * a.ks * MATS), dim3(64 * sp.nw), lds, st, a);
            return hip_status(hipGetLastError(), "gemv_slab launch");
        }
    }
    // MFMA kernel. Below 1024 slabs it runs one slot group per wave: enough K chunks that a
    // chunk's groups fit one workgroup (at most 16 waves, 64 KB of LDS with the waves' A tables).
    const size_t per_wave = NV * 64 * sizeof(float) + mx_table_bytes<NV>();
    const uint32_t ngrp = (S + 7) / 8;
    uint32_t nw1 = mx_max_threads<T, NV, true>() / 64;
    while (nw1 > 1 && nw1 * per_wave > 65536) --nw1;
    // The fused norm runs on the one-group kernel only (its registers stay out of the streaming
    // loop), whatever the number of slabs.
    if (ws && (slabs < 1024 || a.norm_w) && slabs <= kCounters) {
        uint32_t ks = std::max(a.ks, (ngrp + nw1 - 1) / nw1);
        ks = std::min(ks, ngrp);
        if ((uint64_t)slabs * ks * MATS * NV * words <= kSlots) a.ks = ks;
    }
    const uint32_t gwg = (ngrp + a.ks - 1) / a.ks;  // groups of the largest chunk
    // the chunks of a slab (or the pair's two matrices) meet in the workspace words
    if (a.ks * MATS > 1 && (uint64_t)slabs * a.ks * MATS * NV * words > kSlots)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv: %u rows exceed the split-K workspace", a.rows);
    if (gwg <= nw1 && (a.ks == 1 || ws)) {
        if (a.norm_w)
            hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, true, true>), dim3(slabs * a.ks * MATS), dim3(64 * gwg), gwg * per_wave,
                               st, a);
        else
            hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, true>), dim3(slabs * a.ks * MATS), dim3(64 * gwg), gwg * per_wave, st, a);
        return hip_status(hipGetLastError(), "gemv_slab launch");
    }
    if (a.norm_w)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv: the fused norm over %u rows x %u cols needs more split-K "
                                                "workspace than this stream has (or a workspace at all)", a.rows, a.cols);
    uint32_t nw = std::min(sp.nw, mx_max_threads<T, NV, false>() / 64);
    while (nw > 1 && nw * per_wave > 65536) --nw;
    hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, false>), dim3(slabs * a.ks * MATS), dim3(64 * nw), nw * per_wave, st, a);
    return hip_status(hipGetLastError(), "gemv_slab launch");
}

template <uint32_t T, bool PAIR>
int launch_gemv_slab_nv(const GemvSlabArgs& a, uint32_t slabs, Workspace* ws, hipStream_t st) {
    switch (a.n_vec) {
        case 1: return launch_gemv_slab_t<T, 1, PAIR>(a, slabs, ws, st);
        case 2: return launch_gemv_slab_t<T, 2, PAIR>(a, slabs, ws, st);
        case 3: return launch_gemv_slab_t<T, 3, PAIR>(a, slabs, ws, st);
        default: return launch_gemv_slab_t<T, 4, PAIR>(a, slabs, ws, st);
    }
}


}  // namespace

template <bool PAIR>
int launch_gemv_slab(uint32_t type, GemvSlabArgs a, hipStream_t st) {
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    // the pair's gate and up sums always meet in the workspace
    if (PAIR && !ws)
        return set_error(HALO_MI_E_MEMORY, "gate_up: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    if (PAIR && slabs > kCounters) return set_error(HALO_MI_E_UNSUPPORTED, "gate_up: %u rows exceed the workspace", a.rows);
    const uint32_t total = a.n_vec;
    for (uint32_t t0 = 0; t0 < total; t0 += kMaxGemvVec) {
        GemvSlabArgs c = a;
        c.n_vec = std::min(kMaxGemvVec, total - t0);
        c.x = a.x + (uint64_t)t0 * a.x_stride;
        c.y = a.y ? a.y + (uint64_t)t0 * a.y_stride : nullptr;
        if (a.parts) c.parts = a.parts + (uint64_t)t0 * slabs;
        int rc;
        switch (type) {
            case kQ4_0: rc = launch_gemv_slab_nv<kQ4_0, PAIR>(c, slabs, ws, st); break;
            case kQ8_0: rc = launch_gemv_slab_nv<kQ8_0, PAIR>(c, slabs, ws, st); break;
            case kQ4_K: rc = launch_gemv_slab_nv<kQ4_K, PAIR>(c, slabs, ws, st); break;
            case kQ5_K: rc = launch_gemv_slab_nv<kQ5_K, PAIR>(c, slabs, ws, st); break;
            case kIQ4_XS: rc = launch_gemv_slab_nv<kIQ4_XS, PAIR>(c, slabs, ws, st); break;
            default: rc = launch_gemv_slab_nv<kQ6_K, PAIR>(c, slabs, ws, st); break;
        }
        if (rc) return rc;
    }
    return HALO_MI_OK;
}

template int launch_gemv_slab<false>(uint32_t, GemvSlabArgs, hipStream_t);
template int launch_gemv_slab<true>(uint32_t, GemvSlabArgs, hipStream_t);

int launch_gemv_gguf_ref(uint32_t type, const uint8_t* w, uint64_t w_stride, const float* x, uint64_t x_stride, float* y,
                         uint64_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_vec, hipStream_t st) {
    hipLaunchKernelGGL(k_gemv_gguf_ref, dim3((rows + 31) / 32), dim3(256), 0, st, type, w, w_stride, x, x_stride, y,
                       y_stride, rows, cols, n_vec);
    return hip_status(hipGetLastError(), "gemv_gguf_ref launch");
}

}  // namespace halo_mi
