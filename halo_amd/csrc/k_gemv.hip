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
#include <mutex>

#include "gemv_device.h"

namespace halo_mi {
namespace {

using namespace dev;

// Work split of a slab-GEMV launch: ks K chunks per slab (more than one only when the slabs
// alone cannot fill the chip; the chunks then meet in the workspace), nw waves per workgroup.
//
// Every quantity here is chosen as for the widest launch (kMaxGemvVec vectors), never from the
// launch's own vector count: the K chunks and the waves of a chunk fix the order in which a
// row's sum is added up, so a row of an n_vec > 1 call is bitwise the row of its n_vec == 1
// call (GemvArgs::allow_gemm off, include/halo/backend/backend.h:298-302 of the reference).
struct GemvSplit {
    uint32_t ks, nw;
    bool one;  // one slot group per wave (k_gemv_mx's ONE form)
};

template <uint32_t T>
GemvSplit pick_split(uint32_t slabs, uint32_t S, uint32_t mats, bool have_ws) {
    constexpr uint32_t NVW = kMaxGemvVec;
    // One slot group per wave for mid-size matrices, two for large ones (measured on MI355X,
    // 17408 x 5120 and 151936 x 5120 Q4_K).
    const uint32_t groups_per_wave = slabs >= 1024 ? 2u : 1u;
    const uint32_t ngrp = (S + 7) / 8;
    const uint32_t units = std::max(slabs, 1u) * mats;
    auto fits = [&](uint32_t k) {
        return k * mats <= kMaxChunks && (uint64_t)slabs * k * mats * NVW * 64 <= kSlots;
    };
    uint32_t ks = 1;
    // Measured on MI355X: about 4 workgroups per slab up to 1088 per launch; small matrices
    // gain more from a short split-K fix-up than from more workgroups: 2 per slab up to 128
    // slabs (5120 x 5120 Q4_K: 7.56 -> 6.74 us; 12288 x 5120 keeps 4: 9.67 against 10.17 us),
    // and a floor of 128.
    const uint32_t target_wg = std::clamp((units <= 128 ? 2 : 4) * units, 128u, 1088u);
    if (have_ws && units < target_wg) ks = std::min((target_wg + units - 1) / units, ngrp);
    while (ks > 1 && !fits(ks)) --ks;
    // The one-group form (below 1024 slabs): enough K chunks that a chunk's groups fit one
    // workgroup (LDS: the waves' partials and A tables).
    // Up to 16 waves per workgroup (160 KB of LDS per workgroup) when the matrix has at most 128
    // units: fewer, larger workgroups (measured on MI355X: 6144 x 5120 Q4_K 7.81 -> 6.91 us at
    // M = 1, 14.1 -> 11.3 us at M = 4). Larger matrices keep 8: with 10 waves the 17408 x 5120
    // gate/up pair gained at M = 1 (22.9 -> 21.4 us) but lost at M = 2 (28.7 -> 33.7 us), and the
    // split may not depend on the number of vectors.
    const size_t per_wave = NVW * 64 * sizeof(float) + mx_table_bytes<NVW>();
    uint32_t nw1 = std::min(mx_max_threads<T, NVW, true>() / 64, units <= 128 ? 16u : 8u);
    while (nw1 > 1 && nw1 * per_wave > 163840) --nw1;
    if (have_ws && slabs < 1024) {
        const uint32_t k1 = std::min(std::max(ks, (ngrp + nw1 - 1) / nw1), ngrp);
        if (fits(k1)) ks = k1;
    }
    const uint32_t gwg = (ngrp + ks - 1) / ks;  // groups of the largest chunk
    if (gwg <= nw1 && (ks == 1 || have_ws)) return {ks, gwg, true};
    uint32_t nw = std::clamp((gwg + groups_per_wave - 1) / groups_per_wave, 1u, 16u);
    // a wave holds the x sums of at most 4 groups (one per lane)
    while (ks < ngrp && (gwg + nw - 1) / nw > 4) {
        if (nw < 16) ++nw;
        else ++ks;
        const uint32_t g2 = (ngrp + ks - 1) / ks;
        if ((g2 + nw - 1) / nw <= 4) break;
    }
    nw = std::min(nw, mx_max_threads<T, NVW, false>() / 64);
    while (nw > 1 && nw * per_wave > 65536) --nw;
    return {ks, nw, false};
}

// Even split (k_gemv_mx_even), for launches of at least kEvenMinGroups slot groups in the one-group
// form: W = 2 workgroups per CU of an MI355X, each with an equal share of the groups, so every CU
// streams the same bytes. Shape-only like the chunked split (rows are bitwise independent of
// n_vec), and fixed for the full chip (the sums do not depend on how many CUs the device has).
// Measured on MI355X at 17408 x 5120 (1088 chunked workgroups), M = 1 / 2 / 4: Q4_K 12.86 / 15.2 /
// 23.4 -> 12.1 / 14.4 / 22.2 us (18.0 -> 17.3 with the fused norm), Q5_K 15.6 / - / 26.4 -> 14.8 /
// - / 20.3, Q8_0 25.5 / 31.8 / 37.1 -> 19.4 / 21.1 / 24.1. 3 and 4 workgroups per CU were slower at
// 2 to 4 vectors; the gate/up pair's shares (22 units) do not fit one workgroup at 2 per CU, and
// with 3 or 4 per CU it measured no better than chunked.
constexpr uint32_t kEvenMinGroups = 4096;
struct EvenSplit {
    uint32_t W = 0, nu = 0, stride = 0;  // workgroups, units of the largest share, pieces per slab
};

template <uint32_t T>
EvenSplit pick_even(uint32_t slabs, uint32_t S, uint32_t mats, bool have_ws) {
    const uint32_t ngrp = (S + 7) / 8, G = slabs * mats * ngrp;
    // Q6_K keeps the chunked split: its 2-vector kernel holds 170 VGPRs (2 waves per SIMD), and
    // with two units per wave the even split measured slower at every vector count (5120 x 17408:
    // 19.2 -> 20.3 us at M = 1, 24.9 / 25.8 / 28.4 -> 27.8 / 29.2 / 31.1 at M = 2 / 3 / 4)
    if (T == kQ6_K || !have_ws || slabs >= 1024 || G < kEvenMinGroups) return {};
    // a share's units must fit one workgroup at every vector count
    uint32_t max_nu = std::min(16u, even_units_per_wave<T, 1>() * mx_max_threads<T, 1, true>() / 64);
    max_nu = std::min(max_nu, even_units_per_wave<T, 2>() * mx_max_threads<T, 2, true>() / 64);
    max_nu = std::min(max_nu, even_units_per_wave<T, 3>() * mx_max_threads<T, 3, true>() / 64);
    max_nu = std::min(max_nu, even_units_per_wave<T, 4>() * mx_max_threads<T, 4, true>() / 64);
    const uint32_t W = kEvenW, nu = (G + W - 1) / W;
    if (nu > max_nu || even_lds_bytes<kMaxGemvVec>(nu, 1) > 65536) return {};
    const uint32_t per = G / W;  // the fewest units of a share
    const uint32_t stride = mats * ((ngrp + per - 1) / per + 1);
    if (stride > kMaxChunks || (uint64_t)slabs * stride * kMaxGemvVec * 64 > kSlots) return {};
    return {W, nu, stride};
}

// Waves per SIMD that a kernel's registers allow (512 VGPRs per lane on a CDNA SIMD, 8 waves at most).
uint32_t kernel_waves_per_simd(const void* fn) {
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, fn) != hipSuccess || at.numRegs <= 0) return 1;
    return (uint32_t)std::clamp(512 / ((at.numRegs + 7) / 8 * 8), 1, 8);
}

// Waves per workgroup of an even launch with NV vectors: one unit per wave when the CUs hold the
// launch's workgroups that way (always at one vector), else as many as hold them in one round, at
// most even_units_per_wave units per wave. The sums do not depend on it.
template <uint32_t T, int NV, bool PAIR, bool NORM>
uint32_t even_waves(const EvenSplit& ev) {
    static const uint32_t wps = kernel_waves_per_simd(reinterpret_cast<const void*>(&k_gemv_mx_even<T, NV, PAIR, NORM>));
    const uint32_t max_nw = mx_max_threads<T, NV, true>() / 64;
    const uint32_t fit = 4 * wps / (ev.W / 256);  // waves per workgroup with all of them resident on 256 CUs
    const uint32_t nw = std::max(std::min(ev.nu, fit), (ev.nu + even_units_per_wave<T, NV>() - 1) / even_units_per_wave<T, NV>());
    return std::min(nw, max_nw);  // pick_even keeps every share within max_nw waves
}

// slots_cap / counters_cap: the split-K words and slab counters the workspace holds. The split is
// always chosen for the allocated workspace's capacity (kSlots, kCounters), so a smaller workspace
// (halo_mi_gemv_noalloc's scratch) gives the same bits or refuses the shape.
template <uint32_t T, int NV, bool PAIR>
int launch_gemv_slab_t(GemvSlabArgs a, uint32_t slabs, Workspace* ws, uint64_t slots_cap, uint64_t counters_cap,
                       hipStream_t st) {
    const uint32_t S = a.cols / kSlot;
    constexpr uint32_t MATS = PAIR ? 2 : 1;
    const bool have_ws = ws != nullptr && slabs <= kCounters;
    const GemvSplit sp = pick_split<T>(slabs, S, MATS, have_ws);
    a.ks = sp.ks;
    a.slots = ws ? ws->slots : nullptr;
    a.counters = ws ? ws->counters : nullptr;
    a.status = ws ? ws->status : nullptr;
    apply_test_hooks(a);
    const EvenSplit ev = a.valu ? EvenSplit{} : pick_even<T>(slabs, S, MATS, have_ws);
    if (ev.W) {
        a.ks = 0;
        a.even = ev.W;
        a.even_stride = ev.stride;
        a.even_inv_ngrp = 1.0f / (float)((S + 7) / 8);
        a.even_inv_units = 1.0f / (float)(slabs * MATS * ((S + 7) / 8));
        const uint64_t words = (uint64_t)slabs * ev.stride * kMaxGemvVec * 64;
        if (words > slots_cap || slabs > counters_cap)
            return set_error(HALO_MI_E_UNSUPPORTED, "gemv: %u rows x %u cols exceed the split-K workspace (%llu words, %llu slabs)",
                             a.rows, a.cols, (unsigned long long)slots_cap, (unsigned long long)counters_cap);
        if (a.norm_w) {  // the in-kernel norm (one vector; norm_in_kernel chose it)
            if constexpr (NV == 1) {
                // the first workgroup runs the norm's chains and publishes 1 / rms in one word per
                // workgroup, kept at the end of the split-K words (0 between launches); one unit
                // per wave
                const uint32_t nw = ev.nu;
                a.norm_words = nullptr;
                if (words + ev.W <= slots_cap)
                    a.norm_words = ws->slots + (slots_cap - ev.W);
                hipLaunchKernelGGL((k_gemv_mx_even<T, 1, PAIR, true>), dim3(ev.W), dim3(64 * nw),
                                   even_lds_bytes<1>(ev.nu, nw) + norm_lds_bytes(a.cols), st, a);
                return hip_status(hipGetLastError(), "gemv_slab launch");
            } else {
                return set_error(HALO_MI_E_CONFIG, "gemv: the in-kernel norm takes one vector");
            }
        }
        const uint32_t nw = even_waves<T, NV, PAIR, false>(ev);
        if (nw * even_units_per_wave<T, NV>() < ev.nu)
            return set_error(HALO_MI_E_UNSUPPORTED, "gemv: even split of %u units over %u waves", ev.nu, nw);
        hipLaunchKernelGGL((k_gemv_mx_even<T, NV, PAIR>), dim3(ev.W), dim3(64 * nw), even_lds_bytes<NV>(ev.nu, nw), st, a);
        return hip_status(hipGetLastError(), "gemv_slab launch");
    }
    // the chunks of a slab (or the pair's two matrices) meet in the workspace words
    if (a.ks * MATS > 1 &&
        (!have_ws || (uint64_t)slabs * a.ks * MATS * kMaxGemvVec * 64 > slots_cap || slabs > counters_cap))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv: %u rows x %u cols exceed the split-K workspace (%llu words, %llu slabs)",
                         a.rows, a.cols, (unsigned long long)slots_cap, (unsigned long long)counters_cap);
    const size_t lds = mx_lds_bytes<NV>(sp.nw);
    if (a.valu) {  // the VALU kernel (variant HALO_MI_GEMV_SLAB_VALU): the first four formats
        if constexpr (T != kQ5_K && T != kIQ4_XS) {
            hipLaunchKernelGGL((k_gemv_slab<T, NV, PAIR>), dim3(slabs * a.ks * MATS), dim3(64 * sp.nw),
                               (size_t)sp.nw * NV * 64 * sizeof(float), st, a);
            return hip_status(hipGetLastError(), "gemv_slab launch");
        } else {
            return set_error(HALO_MI_E_UNSUPPORTED, "gemv: the VALU slab kernel covers Q4_0, Q8_0, Q4_K and Q6_K only");
        }
    }
    const dim3 grid(slabs * a.ks * MATS), block(64 * sp.nw);
    if (a.norm_w) {  // the in-kernel norm (one vector; norm_in_kernel chose it)
        if constexpr (NV == 1) {
            // with split K, the first workgroup alone runs the norm's chains and publishes 1 / rms
            // in one word per slab, kept at the end of the split-K words (0 between launches)
            const uint64_t words = (uint64_t)slabs * a.ks * MATS * kMaxGemvVec * 64;
            a.norm_words = nullptr;
            if (a.ks * MATS > 1 && slabs <= 64 * kNormPublishPerLane && words + slabs <= slots_cap) {
                a.norm_words = ws->slots + (slots_cap - slabs);
                a.norm_slabs = slabs;
            }
            const size_t ln = lds + norm_lds_bytes(a.cols);
            if (sp.one) hipLaunchKernelGGL((k_gemv_mx<T, 1, PAIR, true, true>), grid, block, ln, st, a);
            else hipLaunchKernelGGL((k_gemv_mx<T, 1, PAIR, false, true>), grid, block, ln, st, a);
            return hip_status(hipGetLastError(), "gemv_slab launch");
        } else {
            return set_error(HALO_MI_E_CONFIG, "gemv: the in-kernel norm takes one vector");
        }
    }
    if (sp.one) hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, true>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((k_gemv_mx<T, NV, PAIR, false>), grid, block, lds, st, a);
    return hip_status(hipGetLastError(), "gemv_slab launch");
}

// Whether a one-vector call with the fused norm runs it inside the GEMV: the MFMA kernel, a row
// of at most kNormMaxCols floats that the workgroup loads in one round (kNormPerThread per
// thread), and LDS for the chain rows beside the kernel's own.
template <uint32_t T>
bool norm_in_kernel_t(uint32_t slabs, uint32_t cols, uint32_t mats, bool have_ws) {
    const EvenSplit ev = pick_even<T>(slabs, cols / kSlot, mats, have_ws);
    const uint32_t nw = ev.W ? ev.nu : pick_split<T>(slabs, cols / kSlot, mats, have_ws).nw;
    const size_t lds = ev.W ? even_lds_bytes<1>(ev.nu, nw) : mx_lds_bytes<1>(nw);
    const uint32_t full = cols - cols % 8u;
    return full > 0 && cols <= kNormMaxCols && cols % 32 == 0 && full <= kNormPerThread * 64 * nw &&
           lds + norm_lds_bytes(cols) <= 163840;
}

bool norm_in_kernel(uint32_t type, uint32_t slabs, uint32_t cols, uint32_t mats, bool have_ws) {
    switch (type) {
        case kQ4_0: return norm_in_kernel_t<kQ4_0>(slabs, cols, mats, have_ws);
        case kQ8_0: return norm_in_kernel_t<kQ8_0>(slabs, cols, mats, have_ws);
        case kQ4_K: return norm_in_kernel_t<kQ4_K>(slabs, cols, mats, have_ws);
        case kQ5_K: return norm_in_kernel_t<kQ5_K>(slabs, cols, mats, have_ws);
        case kIQ4_XS: return norm_in_kernel_t<kIQ4_XS>(slabs, cols, mats, have_ws);
        case kQ6_K: return norm_in_kernel_t<kQ6_K>(slabs, cols, mats, have_ws);
        default: return false;
    }
}

template <uint32_t T, bool PAIR>
int launch_gemv_slab_nv(const GemvSlabArgs& a, uint32_t slabs, Workspace* ws, uint64_t slots_cap, uint64_t counters_cap,
                        hipStream_t st) {
    switch (a.n_vec) {
        case 1: return launch_gemv_slab_t<T, 1, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
        case 2: return launch_gemv_slab_t<T, 2, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
        case 3: return launch_gemv_slab_t<T, 3, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
        default: return launch_gemv_slab_t<T, 4, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
    }
}

// The slab GEMV over a given workspace (vectors in launches of at most kMaxGemvVec). With the
// fused norm, as many rows of x as ws->xn holds (xn_cap floats) are normalized into it first by
// the RMS_NORM kernel (bitwise cpu::rms_norm), and the GEMV reads them: the result is bitwise
// RMS_NORM then the same GEMV.
template <bool PAIR>
int launch_gemv_slab_in(uint32_t type, GemvSlabArgs a, Workspace* ws, uint64_t slots_cap, uint64_t counters_cap,
                        uint64_t xn_cap, hipStream_t st) {
    const uint32_t slabs = (a.rows + kSlabRows - 1) / kSlabRows;
    // the pair's gate and up sums always meet in the workspace
    if (PAIR && !ws)
        return set_error(HALO_MI_E_MEMORY, "gate_up: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    if (PAIR && slabs > counters_cap) return set_error(HALO_MI_E_UNSUPPORTED, "gate_up: %u rows exceed the workspace", a.rows);
    // One vector: the norm inside the GEMV, one dispatch (bitwise the RMS_NORM kernel's rows)
    if (a.norm_w && a.n_vec == 1 && !a.valu &&
        norm_in_kernel(type, slabs, a.cols, PAIR ? 2u : 1u, ws != nullptr && slabs <= kCounters)) {
        switch (type) {
            case kQ4_0: return launch_gemv_slab_nv<kQ4_0, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
            case kQ8_0: return launch_gemv_slab_nv<kQ8_0, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
            case kQ4_K: return launch_gemv_slab_nv<kQ4_K, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
            case kQ5_K: return launch_gemv_slab_nv<kQ5_K, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
            case kIQ4_XS: return launch_gemv_slab_nv<kIQ4_XS, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
            default: return launch_gemv_slab_nv<kQ6_K, PAIR>(a, slabs, ws, slots_cap, counters_cap, st);
        }
    }
    uint32_t per_norm = 0;  // vectors normalized at a time (a multiple of kMaxGemvVec)
    if (a.norm_w) {
        if (!ws || !ws->xn)
            return set_error(HALO_MI_E_MEMORY, "gemv: the fused norm needs this stream's workspace (make one call on it "
                                               "before capturing)");
        per_norm = (uint32_t)std::min<uint64_t>(xn_cap / a.cols / kMaxGemvVec * kMaxGemvVec, 1u << 30);
        if (per_norm == 0)
            return set_error(HALO_MI_E_UNSUPPORTED, "gemv: cols %u too large for the fused norm's buffer (%llu floats)", a.cols,
                             (unsigned long long)xn_cap);
    }
    const uint32_t total = a.n_vec;
    for (uint32_t t0 = 0; t0 < total; t0 += kMaxGemvVec) {
        GemvSlabArgs c = a;
        c.n_vec = std::min(kMaxGemvVec, total - t0);
        c.x = a.x + (uint64_t)t0 * a.x_stride;
        if (a.norm_w) {
            const uint32_t k = t0 % per_norm;  // this chunk's row in the normalized block
            if (k == 0) {
                const uint32_t nb = std::min(per_norm, total - t0);
                if (int rc = launch_rms_norm(c.x, a.x_stride, a.norm_w, ws->xn, a.cols, nb, a.cols, a.norm_eps, st))
                    return rc;
            }
            c.x = ws->xn + (uint64_t)k * a.cols;
            c.x_stride = a.cols;
            c.norm_w = nullptr;
        }
        c.y = a.y ? a.y + (uint64_t)t0 * a.y_stride : nullptr;
        if (a.parts) c.parts = a.parts + (uint64_t)t0 * slabs;
        int rc;
        switch (type) {
            case kQ4_0: rc = launch_gemv_slab_nv<kQ4_0, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
            case kQ8_0: rc = launch_gemv_slab_nv<kQ8_0, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
            case kQ4_K: rc = launch_gemv_slab_nv<kQ4_K, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
            case kQ5_K: rc = launch_gemv_slab_nv<kQ5_K, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
            case kIQ4_XS: rc = launch_gemv_slab_nv<kIQ4_XS, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
            default: rc = launch_gemv_slab_nv<kQ6_K, PAIR>(c, slabs, ws, slots_cap, counters_cap, st); break;
        }
        if (rc) return rc;
    }
    return HALO_MI_OK;
}

}  // namespace

template <bool PAIR>
int launch_gemv_slab(uint32_t type, GemvSlabArgs a, hipStream_t st) {
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    return launch_gemv_slab_in<PAIR>(type, a, ws, kSlots, kCounters, kNormFloats, st);
}

template int launch_gemv_slab<false>(uint32_t, GemvSlabArgs, hipStream_t);
template int launch_gemv_slab<true>(uint32_t, GemvSlabArgs, hipStream_t);

// ---- halo_mi_gemv_noalloc: the slab GEMV over a device-resident scratch array ---------------
// Layout of `scratch`: the status word (256 B), the slab counters, the split-K words. Its size is
// fixed at build time; every GPU the library runs on holds its own copy until the process ends.
constexpr uint64_t kNaStatusBytes = 256;
constexpr uint64_t kNaCounters = 1ull << 16;   // slabs: 4 Mi rows
constexpr uint64_t kNaSlots = 1ull << 20;      // split-K words: 8 MiB
constexpr uint64_t kNaNormFloats = 1ull << 18;  // normalized x rows of the fused norm: 1 MiB
constexpr uint64_t kNaSlotsOff = kNaStatusBytes + kNaCounters * sizeof(uint32_t);
constexpr uint64_t kNaNormOff = kNaSlotsOff + kNaSlots * sizeof(uint64_t);
constexpr uint64_t kNaBytes = kNaNormOff + kNaNormFloats * sizeof(float);
static_assert(kNaSlotsOff % 256 == 0 && kNaNormOff % 256 == 0, "scratch regions 256-byte aligned");

}  // namespace halo_mi

static __device__ __align__(256) unsigned char scratch[halo_mi::kNaBytes];

namespace halo_mi {
namespace {

constexpr int kNaMaxDevices = 64;
std::mutex g_na_mu;
unsigned char* g_na_ptr[kNaMaxDevices];  // the device address of `scratch` on each device, once set up

// The device's scratch address: hipGetSymbolAddress once per device (with that device current);
// the array's host-side name is never used as a device address.
int noalloc_scratch(int dev, unsigned char** out) {
    std::lock_guard<std::mutex> lock(g_na_mu);
    if (dev < 0 || dev >= kNaMaxDevices) return set_error(HALO_MI_E_DEVICE, "gemv_noalloc: device %d out of range", dev);
    if (!g_na_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(HALO_MI_E_DEVICE, "gemv_noalloc: hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        g_na_ptr[dev] = static_cast<unsigned char*>(p);
    }
    *out = g_na_ptr[dev];
    return HALO_MI_OK;
}

}  // namespace

int noalloc_status_take(hipStream_t st, uint32_t* word) {
    *word = 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNaMaxDevices) return HALO_MI_OK;
    unsigned char* base;
    {
        std::lock_guard<std::mutex> lock(g_na_mu);
        base = g_na_ptr[dev];
    }
    if (!base) return HALO_MI_OK;  // never used on this device
    uint32_t* status = reinterpret_cast<uint32_t*>(base);
    if (int rc = hip_status(hipMemcpyAsync(word, status, sizeof(uint32_t), hipMemcpyDeviceToHost, st), "stream_check"))
        return rc;
    if (int rc = hip_status(hipStreamSynchronize(st), "stream_check")) return rc;
    if (*word == 0) return HALO_MI_OK;
    // start again clean: the words and counters of a reduction that gave up are in an unknown state
    if (launch_fill_u32(status, 1, 0u, st) || launch_fill_u32(reinterpret_cast<uint32_t*>(base + kNaStatusBytes), kNaCounters, 0u, st) ||
        launch_fill_u32(reinterpret_cast<uint32_t*>(base + kNaSlotsOff), 2 * kNaSlots, 0u, st))
        return set_error(HALO_MI_E_DEVICE, "stream_check: clearing the no-alloc scratch failed");
    return hip_status(hipStreamSynchronize(st), "stream_check");
}

}  // namespace halo_mi

extern "C" int halo_mi_gemv_noalloc(const halo_mi_gemv_params* p, void* stream) {
    using namespace halo_mi;
    clear_error();
    const char* op = "MATMUL";
    if (!p) return set_error(HALO_MI_E_KERNEL, "gemv_noalloc: null params");
    if (p->variant > HALO_MI_GEMV_VARIANT_LAST)
        return set_error(HALO_MI_E_CONFIG, "%s: unknown kernel variant id %u", op, p->variant);
    uint64_t xs = 0, ys = 0;
    if (int rc = check_gemv_slab_call(p, op, &xs, &ys)) return rc;
    if (p->n_vec == 0 || p->rows == 0) return HALO_MI_OK;
    // Variants 0 and 4 resolve exactly as in halo_mi_gemv (auto_gemv_variant), so that whatever
    // this entry point runs is bitwise what halo_mi_gemv runs for the same call; a shape whose
    // auto choice is a GEMM is refused (its staging and partials do not fit the scratch).
    const uint32_t v = p->variant == HALO_MI_GEMV_DEFAULT || p->variant == HALO_MI_GEMV_SLAB_AUTO
                           ? auto_gemv_variant(p->type, p->rows, p->cols, p->n_vec, false)
                           : p->variant;
    if (v != HALO_MI_GEMV_SLAB && v != HALO_MI_GEMV_SLAB_VALU)
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv_noalloc: variant %u at %u x %u, n_vec %u runs GEMM kernel %u, whose "
                                                "staging does not fit the scratch (only calls that run the slab GEMV)",
                         p->variant, p->rows, p->cols, p->n_vec, v);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "gemv_noalloc: hipGetDevice failed");
    unsigned char* base = nullptr;
    if (int rc = noalloc_scratch(dev, &base)) return rc;
    Workspace ws;
    ws.status = reinterpret_cast<uint32_t*>(base);
    ws.counters = reinterpret_cast<uint32_t*>(base + kNaStatusBytes);
    ws.slots = reinterpret_cast<uint64_t*>(base + kNaSlotsOff);
    ws.xn = reinterpret_cast<float*>(base + kNaNormOff);
    GemvSlabArgs a{static_cast<const uint8_t*>(p->w), nullptr, p->x, xs, p->y, ys, p->rows, p->cols, p->n_vec};
    a.norm_w = p->norm_w;
    a.norm_eps = p->norm_eps;
    a.valu = v == HALO_MI_GEMV_SLAB_VALU;
    return launch_gemv_slab_in<false>(p->type, a, &ws, kNaSlots, kNaCounters, kNaNormFloats, static_cast<hipStream_t>(stream));
}

namespace halo_mi {

int launch_gemv_gguf_ref(uint32_t type, const uint8_t* w, uint64_t w_stride, const float* x, uint64_t x_stride, float* y,
                         uint64_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_vec, hipStream_t st) {
    hipLaunchKernelGGL(k_gemv_gguf_ref, dim3((rows + 31) / 32), dim3(256), 0, st, type, w, w_stride, x, x_stride, y,
                       y_stride, rows, cols, n_vec);
    return hip_status(hipGetLastError(), "gemv_gguf_ref launch");
}

}  // namespace halo_mi
