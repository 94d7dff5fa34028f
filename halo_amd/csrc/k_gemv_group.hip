// Grouped slab GEMV (halo_mi_gemv_group): several SLAB matrices that share x, e.g. a layer's
// q, k and v projections (Q4_K, Q4_K and Q6_K in the reference's hybrid layer), in ONE launch.
// The reference issues them one by one (Qwen35::Impl::gemv, src/models/qwen35.cpp:486-498), so
// each small projection pays a whole launch's ramp and drain.
//
// k_gemv_mx_group<TA, TB, NV>: the workgroups of segment s are the range [wg_end[s - 1],
// wg_end[s]) of the grid; each runs the one-group kernel body of its segment's weight type (TA or
// TB). All segments share the K split (so the workgroup size), x and n_vec; their slabs take
// consecutive places in the workspace's counters and words.
#include "gemv_device.h"

namespace halo_mi {
namespace {

using namespace dev;

struct GemvGroupArgs {
    GemvSlabArgs seg[HALO_MI_GEMV_GROUP_MAX];
    uint32_t type[HALO_MI_GEMV_GROUP_MAX];
    uint32_t wg_end[HALO_MI_GEMV_GROUP_MAX];
    uint32_t n;
};

template <uint32_t TA, uint32_t TB, int NV>
constexpr uint32_t group_max_threads() {
    return std::min(mx_max_threads<TA, NV, true>(), mx_max_threads<TB, NV, true>());
}

// NORM (one vector): the fused norm inside every workgroup (gemv_mx_body's prologue).
template <uint32_t TA, uint32_t TB, int NV, bool NORM>
__global__ __launch_bounds__((group_max_threads<TA, TB, NV>())) void k_gemv_mx_group(GemvGroupArgs g) {
    uint32_t s = 0;
    while (s + 1 < g.n && blockIdx.x >= g.wg_end[s]) ++s;
    const uint32_t bid = blockIdx.x - (s ? g.wg_end[s - 1] : 0u);
    if (g.type[s] == TA) {
        gemv_mx_body<TA, NV, false, true, NORM>(g.seg[s], bid);
    } else {
        if constexpr (TB != TA) gemv_mx_body<TB, NV, false, true, NORM>(g.seg[s], bid);
    }
}

constexpr uint32_t kTypes[6] = {kQ4_0, kQ8_0, kQ4_K, kQ5_K, kQ6_K, kIQ4_XS};

template <int NV, int IA, int IB>
bool launch_pair(uint32_t ta, uint32_t tb, const GemvGroupArgs& g, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
    constexpr uint32_t TA = kTypes[IA], TB = kTypes[IB];
    if (ta != TA || tb != TB) return false;
    if constexpr (NV == 1) {
        if (g.seg[0].norm_w) {
            hipLaunchKernelGGL((k_gemv_mx_group<TA, TB, 1, true>), grid, block, lds, st, g);
            return true;
        }
    }
    hipLaunchKernelGGL((k_gemv_mx_group<TA, TB, NV, false>), grid, block, lds, st, g);
    return true;
}

// (ta, tb) with ta's index <= tb's in kTypes
template <int NV>
bool launch_types(uint32_t ta, uint32_t tb, const GemvGroupArgs& g, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
#define HALO_MI_PAIR(A, B) launch_pair<NV, A, B>(ta, tb, g, grid, block, lds, st)
    return HALO_MI_PAIR(0, 0) || HALO_MI_PAIR(0, 1) || HALO_MI_PAIR(0, 2) || HALO_MI_PAIR(0, 3) || HALO_MI_PAIR(0, 4) ||
           HALO_MI_PAIR(0, 5) || HALO_MI_PAIR(1, 1) || HALO_MI_PAIR(1, 2) || HALO_MI_PAIR(1, 3) || HALO_MI_PAIR(1, 4) ||
           HALO_MI_PAIR(1, 5) || HALO_MI_PAIR(2, 2) || HALO_MI_PAIR(2, 3) || HALO_MI_PAIR(2, 4) || HALO_MI_PAIR(2, 5) ||
           HALO_MI_PAIR(3, 3) || HALO_MI_PAIR(3, 4) || HALO_MI_PAIR(3, 5) || HALO_MI_PAIR(4, 4) || HALO_MI_PAIR(4, 5) ||
           HALO_MI_PAIR(5, 5);
#undef HALO_MI_PAIR
}

int type_index(uint32_t t) {
    for (int i = 0; i < 6; ++i)
        if (kTypes[i] == t) return i;
    return -1;
}

// The one-group waves a workgroup of the pair's kernel may hold (at most 16 waves and 64 KB of
// LDS, as for a single matrix). Taken for the widest launch (kMaxGemvVec vectors) whatever the
// launch's own: the waves of a chunk fix the order of a row's sum, so rows stay bitwise
// independent of n_vec.
template <int NV>
uint32_t group_waves(uint32_t ta, uint32_t tb) {
    auto max_threads = [](uint32_t t) -> uint32_t {
        switch (t) {
            case kQ8_0: return mx_max_threads<kQ8_0, NV, true>();
            case kQ6_K: return mx_max_threads<kQ6_K, NV, true>();
            case kQ5_K: return mx_max_threads<kQ5_K, NV, true>();
            default: return mx_max_threads<kQ4_K, NV, true>();
        }
    };
    const size_t per_wave = NV * 64 * sizeof(float) + mx_table_bytes<NV>();
    uint32_t nw = std::min(max_threads(ta), max_threads(tb)) / 64;
    while (nw > 1 && nw * per_wave > 65536) --nw;
    return nw;
}

// The group's K split and workgroup size (for the widest launch, so rows stay bitwise independent
// of n_vec): ks K chunks, gwg one-group waves per workgroup; false when a chunk does not fit.
bool group_split(uint64_t slabs, uint32_t ta, uint32_t tb, uint32_t cols, uint32_t* ks_out, uint32_t* gwg_out) {
    const uint32_t S = cols / kSlot, ngrp = (S + 7) / 8;
    const uint32_t nw1 = group_waves<kMaxGemvVec>(ta, tb);
    const uint32_t target = std::clamp<uint32_t>((slabs <= 128 ? 2 : 4) * (uint32_t)slabs, 128u, 1088u);
    uint32_t ks = std::min<uint32_t>((target + (uint32_t)slabs - 1) / (uint32_t)slabs, ngrp);
    ks = std::min(std::max(ks, (ngrp + nw1 - 1) / nw1), ngrp);
    *ks_out = ks;
    *gwg_out = (ngrp + ks - 1) / ks;
    return *gwg_out <= nw1;
}

// Whether a one-vector group with the fused norm runs it inside the kernel (as the single-matrix
// GEMV's norm_in_kernel: one load round per workgroup, LDS for the chain rows).
bool group_norm_in_kernel(const GroupSeg* segs, uint32_t n, uint32_t ta, uint32_t tb, uint32_t cols) {
    uint64_t slabs = 0;
    for (uint32_t i = 0; i < n; ++i) slabs += (segs[i].rows + kSlabRows - 1) / kSlabRows;
    uint32_t ks = 0, gwg = 0;
    if (slabs == 0 || !group_split(slabs, ta, tb, cols, &ks, &gwg)) return false;
    const uint32_t full = cols - cols % 8u;
    return full > 0 && cols <= kNormMaxCols && cols % 32 == 0 && full <= kNormPerThread * 64 * gwg &&
           mx_lds_bytes<1>(gwg) + norm_lds_bytes(cols) <= 163840;
}

template <int NV>
int launch_group_nv(const GroupSeg* segs, uint32_t n, uint32_t ta, uint32_t tb, const float* x, uint64_t x_stride,
                    uint32_t cols, Workspace* ws, hipStream_t st, const float* norm_w = nullptr, float eps = 0.0f) {
    const uint32_t S = cols / kSlot, ngrp = (S + 7) / 8;
    uint64_t slabs = 0;
    for (uint32_t i = 0; i < n; ++i) slabs += (segs[i].rows + kSlabRows - 1) / kSlabRows;
    if (slabs == 0) return HALO_MI_OK;
    if (slabs > kCounters) return set_error(HALO_MI_E_UNSUPPORTED, "gemv_group: %llu slabs exceed the workspace", (unsigned long long)slabs);
    // K split: a chip's worth of workgroups (as a single matrix of all the slabs would take), and
    // at least enough chunks that a chunk's slot groups fit one workgroup of one-group waves
    uint32_t ks = 0, gwg = 0;
    const bool fits = group_split(slabs, ta, tb, cols, &ks, &gwg);
    if (ks > 1 && (ks > kMaxChunks || slabs * ks * kMaxGemvVec * 64 > kSlots))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv_group: %llu slabs exceed the split-K workspace", (unsigned long long)slabs);
    if (!fits) return set_error(HALO_MI_E_UNSUPPORTED, "gemv_group: cols %u too large for one workgroup per chunk", cols);
    (void)ngrp;
    GemvGroupArgs g{};
    g.n = n;
    uint32_t slab0 = 0, wg = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t sl = (segs[i].rows + kSlabRows - 1) / kSlabRows;
        GemvSlabArgs a{static_cast<const uint8_t*>(segs[i].w), nullptr, x, x_stride, segs[i].y, segs[i].y_stride,
                       segs[i].rows, cols, (uint32_t)NV};
        a.ks = ks;
        a.norm_w = norm_w;
        a.norm_eps = eps;
        a.slots = ws->slots;
        a.counters = ws->counters;
        a.slab0 = slab0;
        a.status = ws->status;
        apply_test_hooks(a);
        g.seg[i] = a;
        g.type[i] = segs[i].type;
        slab0 += sl;
        wg += sl * ks;
        g.wg_end[i] = wg;
    }
    for (uint32_t i = 0; i < n; ++i) g.seg[i].wg_total = wg;
    const size_t lds = mx_lds_bytes<NV>(gwg) + (norm_w ? norm_lds_bytes(cols) : 0);
    if (!launch_types<NV>(ta, tb, g, dim3(wg), dim3(64 * gwg), lds, st))
        return set_error(HALO_MI_E_UNSUPPORTED, "gemv_group: no kernel for types %u and %u", ta, tb);
    return hip_status(hipGetLastError(), "gemv_group launch");
}

}  // namespace

// With the fused norm, blocks of x rows are normalized into the workspace first by the RMS_NORM
// kernel (bitwise cpu::rms_norm) and the group reads them: the result is bitwise RMS_NORM then
// the same group.
int launch_gemv_group(const GroupSeg* segs, uint32_t n, const float* x, uint64_t x_stride, uint32_t cols, uint32_t n_vec,
                      const float* norm_w, float eps, hipStream_t st) {
    Workspace* ws = nullptr;
    if (int rc = workspace_for(st, &ws)) return rc;
    if (!ws)
        return set_error(HALO_MI_E_MEMORY, "gemv_group: this stream is being captured and has no workspace yet "
                                           "(make one call on it before capturing)");
    // launches of at most two weight types each, in the order the types first appear
    uint32_t types[HALO_MI_GEMV_GROUP_MAX], nt = 0;
    for (uint32_t i = 0; i < n; ++i) {
        bool seen = false;
        for (uint32_t k = 0; k < nt; ++k) seen |= types[k] == segs[i].type;
        if (!seen) types[nt++] = segs[i].type;
    }
    // one vector with the fused norm: inside the kernels when every launch's split allows it
    if (norm_w && n_vec == 1) {
        bool inside = true;
        for (uint32_t k0 = 0; k0 < nt && inside; k0 += 2) {
            uint32_t ta = types[k0], tb = k0 + 1 < nt ? types[k0 + 1] : types[k0];
            if (type_index(ta) > type_index(tb)) std::swap(ta, tb);
            GroupSeg part[HALO_MI_GEMV_GROUP_MAX];
            uint32_t np = 0;
            for (uint32_t i = 0; i < n; ++i)
                if (segs[i].type == ta || segs[i].type == tb) part[np++] = segs[i];
            inside = group_norm_in_kernel(part, np, ta, tb, cols);
        }
        if (inside) {
            for (uint32_t k0 = 0; k0 < nt; k0 += 2) {
                uint32_t ta = types[k0], tb = k0 + 1 < nt ? types[k0 + 1] : types[k0];
                if (type_index(ta) > type_index(tb)) std::swap(ta, tb);
                GroupSeg part[HALO_MI_GEMV_GROUP_MAX];
                uint32_t np = 0;
                for (uint32_t i = 0; i < n; ++i)
                    if (segs[i].type == ta || segs[i].type == tb) part[np++] = segs[i];
                if (int rc = launch_group_nv<1>(part, np, ta, tb, x, x_stride, cols, ws, st, norm_w, eps)) return rc;
            }
            return HALO_MI_OK;
        }
    }
    uint32_t per = n_vec;  // vectors per normalized block
    if (norm_w) {
        per = (uint32_t)std::min<uint64_t>(kNormFloats / cols / kMaxGemvVec * kMaxGemvVec, n_vec);
        if (per == 0) return set_error(HALO_MI_E_UNSUPPORTED, "gemv_group: cols %u too large for the fused norm's buffer", cols);
    }
    for (uint32_t b0 = 0; b0 < n_vec; b0 += per) {
        const uint32_t nb = std::min(per, n_vec - b0);
        const float* xb = x + (uint64_t)b0 * x_stride;
        uint64_t xbs = x_stride;
        if (norm_w) {
            if (int rc = launch_rms_norm(xb, x_stride, norm_w, ws->xn, cols, nb, cols, eps, st)) return rc;
            xb = ws->xn;
            xbs = cols;
        }
        for (uint32_t k0 = 0; k0 < nt; k0 += 2) {
            uint32_t ta = types[k0], tb = k0 + 1 < nt ? types[k0 + 1] : types[k0];
            if (type_index(ta) > type_index(tb)) std::swap(ta, tb);
            GroupSeg part[HALO_MI_GEMV_GROUP_MAX];
            uint32_t np = 0;
            for (uint32_t i = 0; i < n; ++i)
                if (segs[i].type == ta || segs[i].type == tb) part[np++] = segs[i];
            for (uint32_t t0 = 0; t0 < nb; t0 += kMaxGemvVec) {
                const uint32_t nv = std::min(kMaxGemvVec, nb - t0);
                GroupSeg chunk[HALO_MI_GEMV_GROUP_MAX];
                for (uint32_t i = 0; i < np; ++i) {
                    chunk[i] = part[i];
                    chunk[i].y = part[i].y + (uint64_t)(b0 + t0) * part[i].y_stride;
                }
                const float* xc = xb + (uint64_t)t0 * xbs;
                int rc;
                switch (nv) {
                    case 1: rc = launch_group_nv<1>(chunk, np, ta, tb, xc, xbs, cols, ws, st); break;
                    case 2: rc = launch_group_nv<2>(chunk, np, ta, tb, xc, xbs, cols, ws, st); break;
                    case 3: rc = launch_group_nv<3>(chunk, np, ta, tb, xc, xbs, cols, ws, st); break;
                    default: rc = launch_group_nv<4>(chunk, np, ta, tb, xc, xbs, cols, ws, st); break;
                }
                if (rc) return rc;
            }
        }
    }
    return HALO_MI_OK;
}

}  // namespace halo_mi
