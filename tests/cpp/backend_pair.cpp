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

void run_type(hb::MiBackend& be, hb::Stream& st, uint32_t type) {
    const std::string tn = type_name(type);
    const uint32_t rows = 130, cols = 1024, n_vec = 3;  // two full slabs and a ragged one
    const std::vector<uint8_t> wg = make_weights(type, rows, cols, 11 + type);
    const std::vector<uint8_t> wu = make_weights(type, rows, cols, 41 + type);
    std::vector<float> x((size_t)n_vec * cols);
    halo_mi_fill_normal(1011 + type, x.data(), x.size(), 0.0f, 1.0f);

    auto w_gguf = be.import_host_readonly(bytes_of(wg));
    auto w_slab = be.import_weights(bytes_of(wg), static_cast<hb::DType>(type), rows, cols);
    auto u_slab = be.import_weights(bytes_of(wu), static_cast<hb::DType>(type), rows, cols);
    check(dynamic_cast<const hb::MiBuffer&>(*w_gguf).layout() == hb::WeightLayout::Gguf &&
              dynamic_cast<const hb::MiBuffer&>(*w_slab).layout() == hb::WeightLayout::Slab,
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
    for (uint32_t variant : {hb::kGateUpGemv, hb::kGateUpGemm, hb::kGateUpGemmM512, hb::kGateUpGemmSmallM,
                             hb::kGateUpExactSmallM, hb::kGateUpExactInvariant}) {
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

    // RMS_NORM and the fused norm: rms_norm bitwise; every gemv with norm_w is bitwise rms_norm
    // then the same gemv (Limits::max_fused_norm_cols), so the reference-order one is bitwise
    // rms_norm then cpu::matmul
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
        check(be.limits().max_fused_norm_cols >= cols, tn + ": max_fused_norm_cols covers the test's cols");
        hb::GemvArgs plain = a;  // the SLAB default on the normalized x
        plain.w = hb::TensorRef::of(*w_slab);
        plain.x = hb::TensorRef::of(*xnb);
        auto y2b = be.allocate((size_t)n_vec * rows * 4, hb::Tier::Vram);
        plain.y = hb::TensorRef::of(*y2b);
        be.gemv(st, plain);
        std::vector<float> y2(y.size());
        download_y(*y2b, y2);
        an.w = hb::TensorRef::of(*w_slab);
        for (uint32_t nv : {n_vec, 1u}) {  // R > 1 verify rows and the R == 1 decode row
            an.n_vec = nv;
            be.gemv(st, an);
            download_y(*yb, y);
            check(std::memcmp(y.data(), y2.data(), (size_t)nv * rows * 4) == 0,
                  tn + ": SLAB gemv with norm_w (n_vec " + std::to_string(nv) + ") is bitwise rms_norm then the SLAB gemv");
        }
        an.n_vec = n_vec;
        an.norm_w = hb::TensorRef::of(*yb);  // norm_w overlapping y
        check(code_of([&] { be.gemv(st, an); }) == (int)hb::ErrorCode::Kernel, tn + ": norm_w overlapping y -> Kernel");
    }

    // GET_ROWS with device ids: an id outside the table fails the stream's next wait() with
    // Error(Kernel), leaves its row unwritten, and the rows of the good ids are bitwise
    {
        const std::vector<int32_t> idv = {7, 0, 129, -3, 7};
        auto idb = be.allocate(idv.size() * 4, hb::Tier::Vram);
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
        be.get_rows(st, gr);
        be.download(st, hb::TensorRef::of(*ob), std::as_writable_bytes(std::span<float>(got)));
        check(code_of([&] { st.wait(); }) == (int)hb::ErrorCode::Kernel, tn + ": get_rows with a bad id -> Kernel at wait()");
        check(code_of([&] { st.wait(); }) == -1, tn + ": the next wait() is clean");
        std::vector<float> want(cols);
        bool okg = true;
        for (size_t i = 0; i < idv.size(); ++i) {
            if (idv[i] < 0 || idv[i] >= (int32_t)rows) {
                for (uint32_t c = 0; c < cols; ++c) okg &= got[i * cols + c] == 999.0f;
                continue;
            }
            oracle_dequantize_row(type, wg.data() + (size_t)idv[i] * halo_mi_row_bytes(type, cols), want.data(), cols);
            okg &= std::memcmp(got.data() + i * cols, want.data(), cols * 4) == 0;
        }
        check(okg, tn + ": get_rows bitwise, a bad id's row unwritten");
        gr.status.word = 0;
        check(code_of([&] { be.get_rows(st, gr); }) == (int)hb::ErrorCode::Unsupported, tn + ": a StatusRef -> Unsupported");
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
    // the reference HIP backend's type set (test_hip_gemv.cpp:307-308): Q4_1 and the other
    // GGUF-layout-only types are refused with its message
    for (hb::DType wt : {hb::DType::Q4_1, hb::DType::Q5_0, hb::DType::Q5_1, hb::DType::Q2_K, hb::DType::BF16}) {
        bad = a;
        bad.wtype = wt;
        std::string msg;
        int code = -1;
        try {
            be.gemv(st, bad);
        } catch (const hb::Error& e) {
            code = static_cast<int>(e.code());
            msg = e.what();
        }
        check(code == (int)hb::ErrorCode::Unsupported && msg.find("no HIP GEMV kernel") != std::string::npos,
              tn + ": type " + std::to_string(static_cast<unsigned>(wt)) + " -> Unsupported, no HIP GEMV kernel");
    }
}

// MiOptions{BatchInvariantKernel::Exact}: allow_gemm == false runs the exact GEMM with its K split
// fixed by the shape. Every row of n_vec = 3 and 9 is the n_vec = 1 row bitwise, rows are within the
// slab bound, and the bits are those of the explicit registry id; the gate/up pair alike.
void run_invariant(hb::MiBackend& be, hb::Stream& st, uint32_t type) {
    const std::string tn = type_name(type) + std::string(" (Exact)");
    const uint32_t rows = 130, cols = 1024, nv = 9;
    const std::vector<uint8_t> wg = make_weights(type, rows, cols, 17 + type);
    const std::vector<uint8_t> wu = make_weights(type, rows, cols, 47 + type);
    std::vector<float> x((size_t)nv * cols);
    halo_mi_fill_normal(1017 + type, x.data(), x.size(), 0.0f, 1.0f);
    auto w_slab = be.import_weights(bytes_of(wg), static_cast<hb::DType>(type), rows, cols);
    auto u_slab = be.import_weights(bytes_of(wu), static_cast<hb::DType>(type), rows, cols);
    auto xb = be.allocate(x.size() * 4, hb::Tier::Vram);
    auto yb = be.allocate((size_t)nv * rows * 4, hb::Tier::Vram);
    be.upload(st, hb::TensorRef::of(*xb), bytes_of(x));
    std::vector<float> ref((size_t)nv * rows);
    oracle_matmul(type, wg.data(), 0, rows, cols, x.data(), 0, nv, ref.data(), 0, 1);
    const std::vector<double> tol = slab_bound(type, wg, rows, cols, x, nv);
    auto run = [&](auto&& call, uint32_t n) {
        std::vector<float> y((size_t)n * rows);
        call(n);
        be.download(st, hb::TensorRef::of(*yb), std::as_writable_bytes(std::span<float>(y)));
        st.submit();
        st.wait();
        return y;
    };
    auto gemv = [&](uint32_t variant) {
        return [&, variant](uint32_t n) {
            hb::GemvArgs a;
            a.wtype = static_cast<hb::DType>(type);
            a.w = hb::TensorRef::of(*w_slab);
            a.x = hb::TensorRef::of(*xb);
            a.y = hb::TensorRef::of(*yb);
            a.rows = rows;
            a.cols = cols;
            a.n_vec = n;
            a.kernel.variant_id = variant;
            be.gemv(st, a);
        };
    };
    auto gate_up = [&](uint32_t variant) {
        return [&, variant](uint32_t n) {
            hb::GateUpArgs g;
            g.wtype = static_cast<hb::DType>(type);
            g.w_gate = hb::TensorRef::of(*w_slab);
            g.w_up = hb::TensorRef::of(*u_slab);
            g.x = hb::TensorRef::of(*xb);
            g.out = hb::TensorRef::of(*yb);
            g.rows = rows;
            g.cols = cols;
            g.n_vec = n;
            g.kernel.variant_id = variant;
            be.gate_up_swiglu(st, g);
        };
    };
    const std::vector<float> y9 = run(gemv(0), nv);
    bool ok = true;
    for (size_t i = 0; i < y9.size(); ++i) ok &= std::fabs((double)y9[i] - ref[i]) <= tol[i];
    check(ok, tn + ": allow_gemm = false gemv within the slab bound");
    for (uint32_t n : {1u, 3u}) {
        const std::vector<float> yn = run(gemv(0), n);
        check(std::memcmp(yn.data(), y9.data(), (size_t)n * rows * 4) == 0,
              tn + ": n_vec = " + std::to_string(n) + " rows equal the n_vec = 9 rows");
    }
    check(run(gemv(hb::kGemmSlabExactInvariant), nv) == y9, tn + ": the default equals registry id 49");
    const std::vector<float> g9 = run(gate_up(0), nv);
    const std::vector<float> g1 = run(gate_up(0), 1);
    check(std::memcmp(g1.data(), g9.data(), rows * 4) == 0, tn + ": gate_up n_vec = 1 row equals row 0 of n_vec = 9");
    check(run(gate_up(hb::kGateUpExactInvariant), nv) == g9, tn + ": gate_up default equals registry id 50");
}

// The reference interface outside the path: every op virtual exists, the ones this backend does
// not run throw Error(Unsupported); run_op dispatches by OpId and rejects mismatched args with
// Error(Api); ARGMAX and COPY run; decode_argmax reads poisoned vectors as {-1, NaN}.
void run_interface(hb::MiBackend& be, hb::Stream& st) {
    hb::Backend& b = be;
    const int U = (int)hb::ErrorCode::Unsupported;
    check(code_of([&] { b.add_rms_norm(st, hb::AddRmsNormArgs{}); }) == U, "add_rms_norm -> Unsupported");
    check(code_of([&] { b.gdn_gates(st, hb::GdnGateArgs{}); }) == U, "gdn_gates -> Unsupported");
    check(code_of([&] { b.conv1d_silu(st, hb::Conv1dArgs{}); }) == U, "conv1d_silu -> Unsupported");
    check(code_of([&] { b.gated_delta_rule(st, hb::GdnArgs{}); }) == U, "gated_delta_rule -> Unsupported");
    check(code_of([&] { b.gated_rms_norm(st, hb::GatedNormArgs{}); }) == U, "gated_rms_norm -> Unsupported");
    check(code_of([&] { b.partial_rope(st, hb::RopeArgs{}); }) == U, "partial_rope -> Unsupported");
    check(code_of([&] { b.kv_write(st, hb::KvWriteArgs{}); }) == U, "kv_write -> Unsupported");
    check(code_of([&] { b.attention(st, hb::AttentionArgs{}); }) == U, "attention -> Unsupported");
    check(code_of([&] { b.mul_sigmoid(st, hb::EltwiseArgs{}); }) == U, "mul_sigmoid -> Unsupported");
    check(code_of([&] { b.add(st, hb::EltwiseArgs{}); }) == U, "add -> Unsupported");
    check(code_of([&] { b.top_k(st, hb::TopKArgs{}); }) == U, "top_k -> Unsupported");
    hb::OpInvocation inv;
    inv.op = hb::OpId::TopK;
    inv.args = hb::TopKArgs{};
    check(code_of([&] { b.run_op(st, inv); }) == U, "run_op(TOP_K) reaches top_k");
    inv.op = hb::OpId::Gemv;  // the args of another op
    check(code_of([&] { b.run_op(st, inv); }) == (int)hb::ErrorCode::Api, "run_op with mismatched args -> Api");
    check(b.limits().max_fused_norm_cols > 0 && b.limits().lm_head_ids, "limits");
    check(b.variants(hb::OpId::Attention).empty(), "no variants for an op this backend does not run");

    // ARGMAX and COPY through run_op
    const uint32_t n = 300, nv = 3;
    std::vector<float> logits((size_t)n * nv);
    halo_mi_fill_normal(77, logits.data(), logits.size(), 0.0f, 1.0f);
    logits[5] = logits[250] = 9.0f;                 // vector 0: a tie, the lower index wins
    logits[n + 17] = std::nanf("");                // vector 1: poisoned
    auto lb = be.allocate(logits.size() * 4, hb::Tier::Vram), lc = be.allocate(logits.size() * 4, hb::Tier::Vram);
    auto rb = be.allocate(nv * hb::kArgmaxResultBytes, hb::Tier::Vram);
    be.upload(st, hb::TensorRef::of(*lb), bytes_of(logits));
    hb::CopyArgs c;
    c.src = hb::TensorRef::of(*lb);
    c.dst = hb::TensorRef::of(*lc);
    c.bytes = logits.size() * 4;
    inv.op = hb::OpId::Copy;
    inv.args = c;
    b.run_op(st, inv);
    hb::ArgmaxArgs am;
    am.logits = hb::TensorRef::of(*lc);
    am.result = hb::TensorRef::of(*rb);
    am.n = n;
    am.n_vec = nv;
    inv.op = hb::OpId::Argmax;
    inv.args = am;
    b.run_op(st, inv);
    std::vector<std::byte> words(nv * hb::kArgmaxResultBytes);
    b.download(st, hb::TensorRef::of(*rb), words);
    st.submit();
    st.wait();
    std::vector<uint32_t> cpu((size_t)nv * 3);
    oracle_argmax_words(logits.data(), n, nv, cpu.data());
    check(std::memcmp(cpu.data(), words.data(), words.size()) == 0, "argmax words equal the oracle's");
    const std::vector<hb::ArgmaxResult> dec = hb::decode_argmax(words);
    check(dec.size() == nv && dec[0].index == 5 && dec[1].index == -1 && std::isnan(dec[1].value), "decode_argmax");
    c.dst = hb::TensorRef::of(*lb);  // overlapping ranges
    c.src = hb::TensorRef{lb.get(), 4, 0, 0};
    c.bytes = 64;
    check(code_of([&] { b.copy(st, c); }) == (int)hb::ErrorCode::Kernel, "copy with overlapping ranges -> Kernel");
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
            {hb::OpId::GetRows, {{37, "dequant_rows_exact"}}},
            {hb::OpId::RmsNorm, {{38, "rms_norm_cpu_order"}}},
            {hb::OpId::Gemv,
             {{30, "gemv_gguf_ref_b256"}, {31, "gemv_slab_w64"}, {32, "gemm_slab_bf16_mfma"}, {33, "gemv_slab_auto"},
              {34, "gemm_slab_bf16_mfma_m512"}, {35, "gemv_slab_valu_w64"}, {36, "gemm_slab_bf16_mfma_small_m"},
              {47, "gemm_slab_exact_small_m"}, {49, "gemm_slab_exact_invariant"}}},
            {hb::OpId::Swiglu, {{39, "swiglu_b256"}}},
            {hb::OpId::LmHead, {{40, "lm_head_argmax_parts"}}},
            {hb::OpId::Argmax, {{41, "argmax_parts_b256"}}},
            {hb::OpId::Copy, {{42, "copy_async"}}},
            {hb::OpId::GateUpSwiglu,
             {{43, "gate_up_gemv_w64"}, {44, "gate_up_gemm_bf16_mfma"}, {45, "gate_up_gemm_bf16_mfma_m512"},
              {46, "gate_up_gemm_bf16_mfma_small_m"}, {48, "gate_up_gemm_exact_small_m"},
              {50, "gate_up_gemm_exact_invariant"}}},
        };
        for (const auto& [op, want] : pinned) {
            const auto got = be->variants(op);
            bool same = got.size() == want.size();
            for (size_t i = 0; same && i < want.size(); ++i)
                same = got[i].id == want[i].first && std::string(got[i].name) == want[i].second && got[i].op == op;
            check(same, "variant registry of op " + std::to_string((int)op) + " is the pinned id -> name map");
        }
        auto st = be->create_stream();
        run_interface(*be, *st);
        std::vector<std::byte> host(64);
        check(code_of([&] { (void)be->import_host(std::span<std::byte>(host)); }) == (int)hb::ErrorCode::Unsupported,
              "import_host on a device -> Unsupported");
        for (uint32_t t : {HALO_MI_Q4_0, HALO_MI_Q8_0, HALO_MI_Q4_K, HALO_MI_Q6_K, HALO_MI_Q5_K, HALO_MI_IQ4_XS}) {
            std::printf("[case] backend_pair %s\n", type_name(t));
            std::fflush(stdout);
            run_type(*be, *st, t);
        }
        auto be_exact = hb::make_mi355x_backend(0, hb::MiOptions{hb::BatchInvariantKernel::Exact});
        auto st_exact = be_exact->create_stream();
        for (uint32_t t : {HALO_MI_Q4_0, HALO_MI_Q8_0, HALO_MI_Q4_K, HALO_MI_Q6_K, HALO_MI_Q5_K, HALO_MI_IQ4_XS}) {
            std::printf("[case] backend_pair Exact %s\n", type_name(t));
            std::fflush(stdout);
            run_invariant(*be_exact, *st_exact, t);
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("backend_pair: %d checks, %d failures\n", g_checks, g_failures);
    return g_failures ? 1 : 0;
}
