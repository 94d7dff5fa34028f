// Test of the C++ Backend adapter (include/halo_mi355x_backend.hpp) against the CPU oracle,
// in the manner of the reference's Pair fixture (tests/unit/backend/test_hip_backend.cpp:146-202):
// the same seeded weights and activations through the backend and through the oracle's
// cpu::matmul restatement, compared bitwise (GGUF reference variant) or within the derived
// summation bound (SLAB variants), plus the reference's error mapping (backend.h:24-26).
//
// Test infrastructure: links oracle/liboracle.so. Built by __graft_entry__.build(); run by
// tests/test_backend_cpp.py (GPU) with no arguments, or with --list (no GPU needed).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <span>
#include <string>
#include <vector>

#include "../../include/halo_mi355x.h"
#include "../../include/halo_mi355x_backend.hpp"
#include "../../oracle/oracle.h"

namespace hb = halo_mi::backend;

namespace {

int g_failures = 0;
int g_checks = 0;

void check(bool ok, const std::string& what) {
    ++g_checks;
    if (!ok) {
        ++g_failures;
        std::printf("FAIL %s\n", what.c_str());
    }
}

int code_of(const std::function<void()>& f) {
    try {
        f();
    } catch (const hb::Error& e) {
        return static_cast<int>(e.code());
    }
    return -1;
}

const char* type_name(uint32_t t) {
    switch (t) {
        case HALO_MI_Q4_0: return "Q4_0";
        case HALO_MI_Q8_0: return "Q8_0";
        case HALO_MI_Q4_K: return "Q4_K";
        case HALO_MI_Q5_K: return "Q5_K";
        case HALO_MI_IQ4_XS: return "IQ4_XS";
        default: return "Q6_K";
    }
}

std::vector<uint8_t> make_weights(uint32_t type, uint32_t rows, uint32_t cols, uint64_t seed) {
    std::vector<float> w((size_t)rows * cols);
    halo_mi_fill_normal(seed, w.data(), w.size(), 0.0f, 0.02f);
    std::vector<uint8_t> q(halo_mi_row_bytes(type, cols) * rows);
    if (halo_mi_quantize(type, w.data(), w.size(), q.data(), 0) != HALO_MI_OK) std::printf("quantize failed\n");
    return q;
}

template <typename T>
std::span<const std::byte> bytes_of(const std::vector<T>& v) {
    return std::as_bytes(std::span<const T>(v));
}

// (d_cpu + d_slab + 4) u sum_i |x_i| (|a_i| + |b_i| + 2 |off_i|): the SLAB GEMV bound.
std::vector<double> slab_bound(uint32_t type, const std::vector<uint8_t>& w, uint32_t rows, uint32_t cols,
                               const std::vector<float>& x, uint32_t n_vec) {
    const uint64_t rb = halo_mi_row_bytes(type, cols);
    std::vector<float> a(cols), b(cols), off(cols);
    std::vector<double> out((size_t)n_vec * rows);
    const double u = std::ldexp(1.0, -24);
    const double depth = (cols / 8 + 4) + (cols / 32 + 64) + 4;
    for (uint32_t n = 0; n < rows; ++n) {
        oracle_dequant_terms(type, w.data() + n * rb, a.data(), b.data(), off.data(), cols);
        for (uint32_t t = 0; t < n_vec; ++t) {
            double m = 0;
            for (uint32_t i = 0; i < cols; ++i)
                m += std::fabs((double)x[(size_t)t * cols + i]) *
                     (std::fabs((double)a[i]) + std::fabs((double)b[i]) + 2 * std::fabs((double)off[i]));
            out[(size_t)t * rows + n] = depth * u * m * (1 + 1e-3) + 1e-30;
        }
    }
    return out;
}

// (2^-8 + 2^-18 + (d_cpu + d_gemm + 2) u) sum_i |x_i| |w_i|: the bf16 GEMM bound (x and w each
// rounded to bf16, products exact in fp32, plus both summation errors).
std::vector<double> gemm_bound(uint32_t type, const std::vector<uint8_t>& w, uint32_t rows, uint32_t cols,
                               const std::vector<float>& x, uint32_t n_vec) {
    const uint64_t rb = halo_mi_row_bytes(type, cols);
    std::vector<float> wf(cols);
    std::vector<double> out((size_t)n_vec * rows);
    const double u = std::ldexp(1.0, -24);
    const double rel = std::ldexp(1.0, -8) + std::ldexp(1.0, -18) + ((cols / 8 + 4) + (cols / 32 + 40) + 2) * u;
    for (uint32_t n = 0; n < rows; ++n) {
        oracle_dequantize_row(type, w.data() + n * rb, wf.data(), cols);
        for (uint32_t t = 0; t < n_vec; ++t) {
            double m = 0;
            for (uint32_t i = 0; i < cols; ++i) m += std::fabs((double)x[(size_t)t * cols + i]) * std::fabs((double)wf[i]);
            out[(size_t)t * rows + n] = rel * m * (1 + 1e-3) + 1e-30;
        }
    }
    return out;
}

double silu(double v) { return v / (1.0 + std::exp(-v)); }

void run_type(hb::Backend& be, hb::Stream& st, uint32_t type) {
    const std::string tn = type_name(type);
    const uint32_t rows = 130, cols = 1024, n_vec = 3;  // two full slabs and a ragged one
    const std::vector<uint8_t> wg = make_weights(type, rows, cols, 11 + type);
    const std::vector<uint8_t> wu = make_weights(type, rows, cols, 41 + type);
    std::vector<float> x((size_t)n_vec * cols);
    halo_mi_fill_normal(1011 + type, x.data(), x.size(), 0.0f, 1.0f);

    auto w_gguf = be.import_host_readonly(bytes_of(wg));
    auto w_slab = be.import_weights(bytes_of(wg), static_cast<hb::DType>(type), rows, cols);
    auto u_slab = be.import_weights(bytes_of(wu), static_cast<hb::DType>(type), rows, cols);
    check(w_gguf->layout() == hb::WeightLayout::Gguf && w_slab->layout() == hb::WeightLayout::Slab,
          tn + ": buffer layouts");
    auto xb = be.allocate(x.size() * 4, hb::Tier::Vram);
    auto yb = be.allocate((size_t)n_vec * rows * 4, hb::Tier::Vram);
    be.upload(st, hb::TensorRef::of(*xb), bytes_of(x));

    std::vector<float> ref((size_t)n_vec * rows), uref((size_t)n_vec * rows);
    oracle_matmul(type, wg.data(), 0, rows, cols, x.data(), 0, n_vec, ref.data(), 0, 1);
    oracle_matmul(type, wu.data(), 0, rows, cols, x.data(), 0, n_vec, uref.data(), 0, 1);
    std::vector<float> y((size_t)n_vec * rows);
    auto download_y = [&](const hb::Buffer& b, std::vector<float>& dst) {
        be.download(st, hb::TensorRef::of(b), std::as_writable_bytes(std::span<float>(dst)));
        st.submit();
        st.wait();
    };

    // default variant on a GGUF buffer: the reference-order kernel, bitwise cpu::matmul
    hb::GemvArgs a;
    a.wtype = static_cast<hb::DType>(type);
    a.w = hb::TensorRef::of(*w_gguf);
    a.x = hb::TensorRef::of(*xb);
    a.y = hb::TensorRef::of(*yb);
    a.rows = rows;
    a.cols = cols;
    a.n_vec = n_vec;
    be.gemv(st, a);
    download_y(*yb, y);
    check(std::memcmp(y.data(), ref.data(), y.size() * 4) == 0, tn + ": GGUF gemv is bitwise cpu::matmul");

    // default variant on a SLAB buffer: within the summation bound
    a.w = hb::TensorRef::of(*w_slab);
    be.gemv(st, a);
    download_y(*yb, y);
    const std::vector<double> tol = slab_bound(type, wg, rows, cols, x, n_vec);
    bool ok = true;
    for (size_t i = 0; i < y.size(); ++i) ok &= std::fabs((double)y[i] - ref[i]) <= tol[i];
    check(ok, tn + ": SLAB gemv within the bound");

    // without allow_gemm a row does not depend on the batch: n_vec = 1 gives row 0 bitwise
    std::vector<float> y1(rows);
    auto y1b = be.allocate((size_t)rows * 4, hb::Tier::Vram);
    hb::GemvArgs a1 = a;
    a1.n_vec = 1;
    a1.y = hb::TensorRef::of(*y1b);
    be.gemv(st, a1);
    download_y(*y1b, y1);
    check(std::memcmp(y1.data(), y.data(), rows * 4) == 0, tn + ": row 0 of n_vec = 3 equals n_vec = 1");

    // LM head: on the GGUF buffer (reference-order gemv, logits kept) the result words equal the
    // oracle's CpuBackend::lm_head bitwise; on the SLAB buffer (argmax fused into the slab gemv,
    // no logits) the result is the first maximum of that gemv's own rows (y from above), and
    // the dense ids follow the index
    {
        std::vector<uint32_t> cpu_res((size_t)n_vec * 3), res((size_t)n_vec * 3);
        oracle_lm_head(type, wg.data(), 0, rows, cols, x.data(), n_vec, 0, nullptr, cpu_res.data(), 1);
        auto rb = be.allocate((size_t)n_vec * hb::kArgmaxResultBytes, hb::Tier::Vram);
        auto ib = be.allocate((size_t)n_vec * 4, hb::Tier::Vram);
        hb::LmHeadArgs h;
        h.gemv = a;
        h.gemv.w = hb::TensorRef::of(*w_gguf);
        h.result = hb::TensorRef::of(*rb);
        h.ids = hb::TensorRef::of(*ib);
        be.lm_head(st, h);
        be.download(st, hb::TensorRef::of(*rb), std::as_writable_bytes(std::span<uint32_t>(res)));
        st.submit();
        st.wait();
        check(res == cpu_res, tn + ": lm_head on GGUF weights equals the CPU's result words");
        h.gemv.w = hb::TensorRef::of(*w_slab);
        h.gemv.y = {};
        be.lm_head(st, h);
        std::vector<int32_t> ids(n_vec);
        be.download(st, hb::TensorRef::of(*rb), std::as_writable_bytes(std::span<uint32_t>(res)));
        be.download(st, hb::TensorRef::of(*ib), std::as_writable_bytes(std::span<int32_t>(ids)));
        st.submit();
        st.wait();
        bool okh = true;
        for (uint32_t t = 0; t < n_vec; ++t) {
            const float* row = y.data() + (size_t)t * rows;
            uint32_t best = 0;
            for (uint32_t n = 1; n < rows; ++n)
                if (row[n] > row[best]) best = n;
            uint32_t vb;
            std::memcpy(&vb, &row[best], 4);
            okh &= res[3 * t] == best && res[3 * t + 1] == vb && res[3 * t + 2] == 0 && ids[t] == (int32_t)best;
        }
        check(okh, tn + ": fused lm_head on SLAB weights is the first maximum of the slab gemv");
        hb::LmHeadArgs bad = h;
        bad.ids = {};
        bad.ids_slots = hb::TensorRef::of(*ib);
        bad.ids_scatter = hb::TensorRef::of(*ib);
        check(code_of([&] { be.lm_head(st, bad); }) == (int)hb::ErrorCode::Api, tn + ": lm_head ids_slots without ids -> Api");
        bad = h;
        bad.gemv.w = hb::TensorRef::of(*w_gguf);
        check(code_of([&] { be.lm_head(st, bad); }) == (int)hb::ErrorCode::Kernel,
              tn + ": lm_head ranking GGUF logits without gemv.y -> Kernel");
    }

    // fused gate/up (GEMV pair and bf16 GEMM variants) against the oracle's composition
    const std::vector<double> tu = slab_bound(type, wu, rows, cols, x, n_vec);
    const std::vector<double> gg = gemm_bound(type, wg, rows, cols, x, n_vec), gu = gemm_bound(type, wu, rows, cols, x, n_vec);
    for (uint32_t variant : {hb::kGateUpGemv, hb::kGateUpGemm, hb::kGateUpGemmM512}) {
        hb::GateUpArgs g;
        g.wtype = static_cast<hb::DType>(type);
        g.w_gate = hb::TensorRef::of(*w_slab);
        g.w_up = hb::TensorRef::of(*u_slab);
        g.x = hb::TensorRef::of(*xb);
        g.out = hb::TensorRef::of(*yb);
        g.rows = rows;
        g.cols = cols;
        g.n_vec = n_vec;
        g.kernel.variant_id = variant;
        be.gate_up_swiglu(st, g);
        download_y(*yb, y);
        bool ok2 = true;
        for (size_t i = 0; i < y.size(); ++i) {
            const bool gemm = variant != hb::kGateUpGemv;
            const double dg = gemm ? gg[i] : tol[i], du = gemm ? gu[i] : tu[i];
            const double o = silu((double)ref[i]) * uref[i];
            const double u24 = std::ldexp(1.0, -24);
            double bound = 1.1 * dg * (std::fabs((double)uref[i]) + du) + (std::fabs(silu(ref[i])) + 1.1 * dg) * du +
                           16 * u24 * std::fabs(o) + 1e-30;
            // the GEMM epilogue's SiLU (v_exp_f32 / v_rcp_f32): relative error <= (1.5 |g| + 8) 2^-24
            if (gemm)
                bound += (1.5 * (std::fabs((double)ref[i]) + dg) + 8) * u24 * (std::fabs(silu(ref[i])) + 1.1 * dg) *
                         (std::fabs((double)uref[i]) + du);
            ok2 &= std::fabs((double)y[i] - o) <= bound;
        }
        check(ok2, tn + ": gate_up_swiglu variant " + std::to_string(variant) + " within the bound");
    }

    // RMS_NORM and the fused norm: rms_norm bitwise; the reference-order gemv with norm_w is
    // bitwise rms_norm then cpu::matmul; the SLAB default within the GEMV bound on the CPU's
    // normalized x plus the norm's own rounding (half the two sums-of-squares orders' error)
    {
        std::vector<float> nw(cols), xn(x.size());
        for (uint32_t i = 0; i < cols; ++i) nw[i] = 0.5f + (float)(i % 7) * 0.125f;
        oracle_rms_norm(x.data(), 0, nw.data(), xn.data(), 0, n_vec, cols, 1e-6f);
        auto nwb = be.allocate((size_t)cols * 4, hb::Tier::Vram);
        auto xnb = be.allocate(x.size() * 4, hb::Tier::Vram);
        be.upload(st, hb::TensorRef::of(*nwb), bytes_of(nw));
        hb::RmsNormArgs rn;
        rn.x = hb::TensorRef::of(*xb);
        rn.w = hb::TensorRef::of(*nwb);
        rn.out = hb::TensorRef::of(*xnb);
        rn.rows = n_vec;
        rn.cols = cols;
        be.rms_norm(st, rn);
        std::vector<float> got(x.size());
        download_y(*xnb, got);
        check(std::memcmp(got.data(), xn.data(), got.size() * 4) == 0, tn + ": rms_norm is bitwise cpu::rms_norm");
        std::vector<float> nref((size_t)n_vec * rows);
        oracle_matmul(type, wg.data(), 0, rows, cols, xn.data(), 0, n_vec, nref.data(), 0, 1);
        hb::GemvArgs an = a;
        an.w = hb::TensorRef::of(*w_gguf);
        an.norm_w = hb::TensorRef::of(*nwb);
        be.gemv(st, an);
        download_y(*yb, y);
        check(std::memcmp(y.data(), nref.data(), y.size() * 4) == 0, tn + ": GGUF gemv with norm_w is bitwise rms_norm + matmul");
        an.w = hb::TensorRef::of(*w_slab);
        be.gemv(st, an);
        download_y(*yb, y);
        std::vector<double> ntol = slab_bound(type, wg, rows, cols, xn, n_vec);
        const double extra = (0.5 * (cols / 8.0 + cols / 256.0 + 30) + 11) / ((cols / 8 + 4) + (cols / 32 + 64) + 4);
        bool okn = true;
        for (size_t i = 0; i < y.size(); ++i) okn &= std::fabs((double)y[i] - nref[i]) <= ntol[i] * (1.0 + extra) * 1.01;
        check(okn, tn + ": SLAB gemv with norm_w within the bound");
        an.norm_w = hb::TensorRef::of(*yb);  // norm_w overlapping y
        check(code_of([&] { be.gemv(st, an); }) == (int)hb::ErrorCode::Kernel, tn + ": norm_w overlapping y -> Kernel");
    }

    // GET_ROWS with device ids and the status word
    {
        const std::vector<int32_t> idv = {7, 0, 129, -3, 7};
        auto idb = be.allocate(idv.size() * 4, hb::Tier::Vram);
        auto sb = be.allocate(4, hb::Tier::Vram);
        auto ob = be.allocate(idv.size() * cols * 4, hb::Tier::Vram);
        be.upload(st, hb::TensorRef::of(*idb), bytes_of(idv));
        std::vector<float> sentinel(idv.size() * cols, 999.0f), got(idv.size() * cols);
        be.upload(st, hb::TensorRef::of(*ob), bytes_of(sentinel));
        hb::GetRowsArgs gr;
        gr.type = static_cast<hb::DType>(type);
        gr.table = hb::TensorRef::of(*w_slab);
        gr.ids = hb::TensorRef::of(*idb);
        gr.out = hb::TensorRef::of(*ob);
        gr.n_rows = rows;
        gr.cols = cols;
        gr.n_ids = (uint32_t)idv.size();
        gr.status = hb::TensorRef::of(*sb);
        be.get_rows(st, gr);
        uint32_t word = 0;
        be.download(st, hb::TensorRef::of(*sb), std::as_writable_bytes(std::span<uint32_t>(&word, 1)));
        download_y(*ob, got);
        std::vector<float> want(cols);
        bool okg = word == hb::kStatusBadIndex;
        for (size_t i = 0; i < idv.size(); ++i) {
            if (idv[i] < 0 || idv[i] >= (int32_t)rows) {
                for (uint32_t c = 0; c < cols; ++c) okg &= got[i * cols + c] == 999.0f;
                continue;
            }
            oracle_dequantize_row(type, wg.data() + (size_t)idv[i] * halo_mi_row_bytes(type, cols), want.data(), cols);
            okg &= std::memcmp(got.data() + i * cols, want.data(), cols * 4) == 0;
        }
        check(okg, tn + ": get_rows bitwise, a bad id unwritten and reported in the status word");
    }

    // error mapping (backend.h:24-26)
    hb::GemvArgs bad = a;
    bad.kernel.variant_id = 99;
    check(code_of([&] { be.gemv(st, bad); }) == (int)hb::ErrorCode::Config, tn + ": unknown variant -> Config");
    bad = a;
    bad.gates.n_v = 1;
    check(code_of([&] { be.gemv(st, bad); }) == (int)hb::ErrorCode::Unsupported, tn + ": GDN gates epilogue -> Unsupported");
    bad = a;
    bad.y = hb::TensorRef::of(*xb);  // y overlaps x
    check(code_of([&] { be.gemv(st, bad); }) == (int)hb::ErrorCode::Kernel, tn + ": y overlapping x -> Kernel");
    bad = a;
    bad.kernel.variant_id = hb::kGemvGgufRef;  // a GGUF-only kernel on a SLAB buffer
    check(code_of([&] { be.gemv(st, bad); }) == (int)hb::ErrorCode::Config, tn + ": layout/variant mismatch -> Config");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
        std::printf("backend_pair: gemv (GGUF ref bitwise, SLAB bound, batch invariance, fused norm), rms_norm, "
                    "get_rows, lm_head, gate_up_swiglu, errors; "
                    "types Q4_0 Q8_0 Q4_K Q6_K Q5_K IQ4_XS\n");
        return 0;
    }
    try {
        auto be = hb::make_mi355x_backend(0);
        check(be->kind() == hb::Kind::Hip, "kind() is Hip");
        check(!be->describe().empty(), "describe()");
        check(!be->lost(), "not lost");
        // the registry's id -> name map is pinned: ids are append-only and never reused
        // (as the reference pins its own, tests/unit/backend/test_hip_backend.cpp:925-981)
        const std::pair<hb::OpId, std::vector<std::pair<uint32_t, std::string>>> pinned[] = {
            {hb::OpId::GetRows, {{hb::kDequantRows, "dequant_rows_exact"}}},
            {hb::OpId::RmsNorm, {{hb::kRmsNorm, "rms_norm_cpu_order"}}},
            {hb::OpId::Gemv,
             {{hb::kGemvGgufRef, "gemv_gguf_ref_b256"}, {hb::kGemvSlab, "gemv_slab_w64"},
              {hb::kGemmSlabBf16, "gemm_slab_bf16_mfma"}, {hb::kGemvSlabAuto, "gemv_slab_auto"},
              {hb::kGemmSlabBf16M512, "gemm_slab_bf16_mfma_m512"}}},
            {hb::OpId::Swiglu, {{hb::kSwiglu, "swiglu_b256"}}},
            {hb::OpId::GateUpSwiglu,
             {{hb::kGateUpGemv, "gate_up_gemv_w64"}, {hb::kGateUpGemm, "gate_up_gemm_bf16_mfma"},
              {hb::kGateUpGemmM512, "gate_up_gemm_bf16_mfma_m512"}}},
            {hb::OpId::LmHead, {{hb::kLmHeadFused, "lm_head_slab_argmax"}}},
        };
        for (const auto& [op, want] : pinned) {
            const auto got = be->variants(op);
            bool same = got.size() == want.size();
            for (size_t i = 0; same && i < want.size(); ++i)
                same = got[i].id == want[i].first && std::string(got[i].name) == want[i].second && got[i].op == op;
            check(same, "variant registry of op " + std::to_string((int)op) + " is the pinned id -> name map");
        }
        auto st = be->create_stream();
        std::vector<std::byte> host(64);
        check(code_of([&] { (void)be->import_host(std::span<std::byte>(host)); }) == (int)hb::ErrorCode::Unsupported,
              "import_host on a device -> Unsupported");
        for (uint32_t t : {HALO_MI_Q4_0, HALO_MI_Q8_0, HALO_MI_Q4_K, HALO_MI_Q6_K, HALO_MI_Q5_K, HALO_MI_IQ4_XS}) {
            std::printf("[case] backend_pair %s\n", type_name(t));
            std::fflush(stdout);
            run_type(*be, *st, t);
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("backend_pair: %d checks, %d failures\n", g_checks, g_failures);
    return g_failures ? 1 : 0;
}
