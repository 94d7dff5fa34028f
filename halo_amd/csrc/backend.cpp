// The MI355X backend: halo_mi355x_backend.hpp over the halo_mi355x C ABI.
//
// Host validation follows the reference CPU/HIP adapters (src/backend/cpu_backend.cpp:98-162
// Resolver; src/backend/hip_adapter.cpp:612-632 gemv) on device addresses: ownership, range,
// alignment, stride and aliasing are checked before anything is enqueued.
#include "../../include/halo_mi355x_backend.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <bit>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>

#include "../../include/halo_mi355x.h"

namespace halo_mi::backend {

namespace {

[[noreturn]] void fail(ErrorCode code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

void fail(ErrorCode code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw Error(code, buf);
}

#define CHECK(cond, code, ...)              \
    do {                                    \
        if (!(cond)) fail((code), __VA_ARGS__); \
    } while (0)

// C-ABI status -> ErrorCode, with the library's message.
void check_abi(int rc) {
    if (rc == HALO_MI_OK) return;
    const ErrorCode code = rc == HALO_MI_E_KERNEL        ? ErrorCode::Kernel
                           : rc == HALO_MI_E_UNSUPPORTED ? ErrorCode::Unsupported
                           : rc == HALO_MI_E_CONFIG      ? ErrorCode::Config
                           : rc == HALO_MI_E_MEMORY      ? ErrorCode::Memory
                                                         : ErrorCode::Device;
    throw Error(code, halo_mi_last_error());
}

constexpr std::uint64_t kF32 = 4;

std::uint64_t mul_u64(std::uint64_t a, std::uint64_t b, const char* op, const char* what) {
    CHECK(a == 0 || b <= std::numeric_limits<std::uint64_t>::max() / a, ErrorCode::Kernel, "%s: %s size overflows", op, what);
    return a * b;
}

const char* type_name(DType t) {
    switch (t) {
        case DType::F32: return "F32";
        case DType::F16: return "F16";
        case DType::BF16: return "BF16";
        case DType::Q4_0: return "Q4_0";
        case DType::Q4_1: return "Q4_1";
        case DType::Q5_0: return "Q5_0";
        case DType::Q5_1: return "Q5_1";
        case DType::Q2_K: return "Q2_K";
        case DType::Q8_0: return "Q8_0";
        case DType::Q3_K: return "Q3_K";
        case DType::Q4_K: return "Q4_K";
        case DType::Q5_K: return "Q5_K";
        case DType::Q6_K: return "Q6_K";
        case DType::IQ4_NL: return "IQ4_NL";
        case DType::IQ3_S: return "IQ3_S";
        case DType::IQ4_XS: return "IQ4_XS";
        default: return "?";
    }
}

// ---- buffers --------------------------------------------------------------------------------

struct SlabMeta {
    DType type = DType::F32;
    std::uint32_t rows = 0, cols = 0;
};

class DeviceBuffer final : public MiBuffer {
public:
    DeviceBuffer(const Backend* owner, void* mem, std::uint64_t bytes, Tier tier, bool writable, bool host, WeightLayout layout,
                 SlabMeta meta)
        : owner_(owner), mem_(mem), bytes_(bytes), tier_(tier), writable_(writable), host_(host), layout_(layout), meta_(meta) {}
    ~DeviceBuffer() override {
        if (host_) (void)hipHostFree(mem_);
        else (void)hipFree(mem_);
    }
    std::uint64_t bytes() const noexcept override { return bytes_; }
    Tier tier() const noexcept override { return tier_; }
    const Backend* backend() const noexcept override { return owner_; }
    bool writable() const noexcept override { return writable_; }
    const std::byte* host_data() const noexcept override { return host_ ? static_cast<const std::byte*>(mem_) : nullptr; }
    std::byte* host_ptr() const noexcept override { return host_ && writable_ ? static_cast<std::byte*>(mem_) : nullptr; }
    void* device_ptr() const noexcept override { return mem_; }
    WeightLayout layout() const noexcept override { return layout_; }
    const SlabMeta& meta() const noexcept { return meta_; }

private:
    const Backend* owner_;
    void* mem_;
    std::uint64_t bytes_;
    Tier tier_;
    bool writable_, host_;
    WeightLayout layout_;
    SlabMeta meta_;
};

// ---- streams --------------------------------------------------------------------------------

class Mi355xBackend;

// A stream owns its hipStream_t and one device word for the GET_ROWS status bits of the ops
// enqueued since the last wait(); the library's per-stream workspace is released with it.
class HipStream final : public MiStream {
public:
    HipStream(Mi355xBackend* owner, hipStream_t s, std::uint32_t* status) : owner_(owner), s_(s), status_(status) {}
    ~HipStream() override {
        (void)hipStreamSynchronize(s_);
        (void)halo_mi_stream_release(s_);
        (void)hipFree(status_);
        (void)hipStreamDestroy(s_);
    }
    void submit() override {}
    void wait() override;
    void abort() noexcept override { (void)hipStreamSynchronize(s_); }
    void* native() const noexcept override { return s_; }
    const Mi355xBackend* owner() const noexcept { return owner_; }
    // the GET_ROWS status word, marked as used until the next wait()
    std::uint32_t* get_rows_status() noexcept {
        status_used_ = true;
        return status_;
    }

private:
    Mi355xBackend* owner_;
    hipStream_t s_;
    std::uint32_t* status_;
    bool status_used_ = false;
};

// ---- operand resolution ---------------------------------------------------------------------

enum class Access : std::uint8_t { Read, Write };

struct Operand {
    const char* name = "";
    std::uint8_t* base = nullptr;  // device address of row 0
    std::uint64_t stride = 0;      // bytes between rows
    std::uint64_t extent = 0;      // bytes touched
    const DeviceBuffer* buf = nullptr;
};

class Resolver {
public:
    Resolver(const Backend* self, const char* op) : self_(self), op_(op) {}

    // rows x row_bytes at ref; `align` = required alignment of address and stride.
    Operand get(const TensorRef& ref, std::uint64_t rows, std::uint64_t row_bytes, std::uint64_t align, Access access,
                const char* name) const {
        Operand o;
        o.name = name;
        o.stride = ref.row_stride != 0 ? ref.row_stride : row_bytes;
        if ((rows == 0 || row_bytes == 0) && ref.empty()) return o;
        CHECK(!ref.empty(), ErrorCode::Kernel, "%s: operand %s is empty", op_, name);
        const auto* b = dynamic_cast<const DeviceBuffer*>(ref.buffer);
        CHECK(b != nullptr && b->backend() == self_, ErrorCode::Kernel, "%s: operand %s belongs to another backend", op_, name);
        CHECK(access == Access::Read || b->writable(), ErrorCode::Kernel, "%s: output %s is read-only", op_, name);
        CHECK(rows <= 1 || o.stride >= row_bytes, ErrorCode::Kernel, "%s: operand %s row stride %llu < row bytes %llu", op_,
              name, (unsigned long long)o.stride, (unsigned long long)row_bytes);
        o.extent = rows == 0 ? 0 : mul_u64(rows - 1, o.stride, op_, name) + row_bytes;
        CHECK(ref.offset <= b->bytes(), ErrorCode::Kernel, "%s: operand %s offset %llu past buffer end %llu", op_, name,
              (unsigned long long)ref.offset, (unsigned long long)b->bytes());
        const std::uint64_t avail = b->bytes() - ref.offset;
        const std::uint64_t limit = ref.bytes != 0 ? ref.bytes : avail;
        CHECK(limit <= avail, ErrorCode::Kernel, "%s: operand %s range exceeds buffer of %llu bytes", op_, name,
              (unsigned long long)b->bytes());
        CHECK(o.extent <= limit, ErrorCode::Kernel, "%s: operand %s needs %llu bytes, view has %llu", op_, name,
              (unsigned long long)o.extent, (unsigned long long)limit);
        o.base = static_cast<std::uint8_t*>(b->device_ptr()) + ref.offset;
        o.buf = b;
        CHECK(reinterpret_cast<std::uintptr_t>(o.base) % align == 0 && o.stride % align == 0, ErrorCode::Kernel,
              "%s: operand %s is not %llu-byte aligned", op_, name, (unsigned long long)align);
        return o;
    }

    Operand f32(const TensorRef& ref, std::uint64_t rows, std::uint64_t cols, Access access, const char* name) const {
        return get(ref, rows, mul_u64(cols, kF32, op_, name), kF32, access, name);
    }

    // A SLAB weight operand: whole slabs of a buffer imported with import_weights.
    Operand slab(const TensorRef& ref, DType type, std::uint32_t rows, std::uint32_t cols, const char* name) const {
        Operand o;
        o.name = name;
        CHECK(!ref.empty(), ErrorCode::Kernel, "%s: operand %s is empty", op_, name);
        const auto* b = dynamic_cast<const DeviceBuffer*>(ref.buffer);
        CHECK(b != nullptr && b->backend() == self_, ErrorCode::Kernel, "%s: operand %s belongs to another backend", op_, name);
        CHECK(b->layout() == WeightLayout::Slab, ErrorCode::Config, "%s: operand %s is not in the SLAB layout", op_, name);
        const SlabMeta& m = b->meta();
        CHECK(m.type == type && m.cols == cols, ErrorCode::Kernel, "%s: operand %s holds %s x %u, op asks %s x %u", op_, name,
              type_name(m.type), m.cols, type_name(type), cols);
        CHECK(ref.row_stride == 0, ErrorCode::Kernel, "%s: a SLAB operand has no row stride", op_);
        const std::uint64_t sb = halo_mi_slab_bytes(static_cast<std::uint32_t>(type), HALO_MI_SLAB_ROWS, cols);
        CHECK(sb != 0 && ref.offset % sb == 0, ErrorCode::Kernel, "%s: operand %s offset %llu is not a whole slab (%llu B)", op_,
              name, (unsigned long long)ref.offset, (unsigned long long)sb);
        const std::uint64_t first = ref.offset / sb * HALO_MI_SLAB_ROWS;
        CHECK(first <= m.rows && rows <= m.rows - first, ErrorCode::Kernel, "%s: operand %s rows [%llu, %llu) out of %u", op_,
              name, (unsigned long long)first, (unsigned long long)(first + rows), m.rows);
        o.extent = halo_mi_slab_bytes(static_cast<std::uint32_t>(type), rows, cols);
        CHECK(ref.bytes == 0 || ref.bytes >= o.extent, ErrorCode::Kernel, "%s: operand %s needs %llu bytes", op_, name,
              (unsigned long long)o.extent);
        o.base = static_cast<std::uint8_t*>(b->device_ptr()) + ref.offset;
        o.buf = b;
        return o;
    }

    void no_overlap(const Operand& out, const Operand& other) const {
        if (out.extent == 0 || other.extent == 0) return;
        const auto lo1 = reinterpret_cast<std::uintptr_t>(out.base), lo2 = reinterpret_cast<std::uintptr_t>(other.base);
        CHECK(!(lo1 < lo2 + other.extent && lo2 < lo1 + out.extent), ErrorCode::Kernel, "%s: output %s overlaps operand %s",
              op_, out.name, other.name);
    }

    const char* op() const noexcept { return op_; }

private:
    const Backend* self_;
    const char* op_;
};

// ---- variant registry (explicit, append-only ids; grouped by op) ----------------------------

constexpr std::array<VariantInfo, 21> kVariants{{
    {kDequantRows, "dequant_rows_exact", OpId::GetRows, {}},
    {kRmsNorm, "rms_norm_cpu_order", OpId::RmsNorm, {}},
    {kGemvGgufRef, "gemv_gguf_ref_b256", OpId::Gemv, {}},
    {kGemvSlab, "gemv_slab_w64", OpId::Gemv, {}},
    {kGemmSlabBf16, "gemm_slab_bf16_mfma", OpId::Gemv, {}},
    {kGemvSlabAuto, "gemv_slab_auto", OpId::Gemv, {}},
    {kGemmSlabBf16M512, "gemm_slab_bf16_mfma_m512", OpId::Gemv, {}},
    {kGemvSlabValu, "gemv_slab_valu_w64", OpId::Gemv, {}},
    {kGemmSlabBf16SmallM, "gemm_slab_bf16_mfma_small_m", OpId::Gemv, {}},
    {kGemmSlabExactSmallM, "gemm_slab_exact_small_m", OpId::Gemv, {}},
    {kGemmSlabExactInvariant, "gemm_slab_exact_invariant", OpId::Gemv, {}},
    {kSwiglu, "swiglu_b256", OpId::Swiglu, {}},
    {kLmHeadFused, "lm_head_argmax_parts", OpId::LmHead, {}},
    {kArgmax, "argmax_parts_b256", OpId::Argmax, {}},
    {kCopy, "copy_async", OpId::Copy, {}},
    {kGateUpGemv, "gate_up_gemv_w64", OpId::GateUpSwiglu, {}},
    {kGateUpGemm, "gate_up_gemm_bf16_mfma", OpId::GateUpSwiglu, {}},
    {kGateUpGemmM512, "gate_up_gemm_bf16_mfma_m512", OpId::GateUpSwiglu, {}},
    {kGateUpGemmSmallM, "gate_up_gemm_bf16_mfma_small_m", OpId::GateUpSwiglu, {}},
    {kGateUpExactSmallM, "gate_up_gemm_exact_small_m", OpId::GateUpSwiglu, {}},
    {kGateUpExactInvariant, "gate_up_gemm_exact_invariant", OpId::GateUpSwiglu, {}},
}};

bool has_variant(OpId op, std::uint32_t id) {
    if (id == 0) return true;
    return std::any_of(kVariants.begin(), kVariants.end(), [&](const VariantInfo& v) { return v.op == op && v.id == id; });
}

// MATMUL registry id -> the C ABI's variant id (ids 30..36 are in the C ABI's order)
std::uint32_t abi_gemv_variant(std::uint32_t id) {
    return id == 0                         ? HALO_MI_GEMV_DEFAULT
           : id == kGemmSlabExactSmallM    ? HALO_MI_GEMM_SLAB_EXACT_SMALL_M
           : id == kGemmSlabExactInvariant ? HALO_MI_GEMM_SLAB_EXACT_INVARIANT
                                           : id - kGemvGgufRef + 1;
}

void check_no_status(const StatusRef& st, const char* op) {
    CHECK(st.empty(), ErrorCode::Unsupported, "%s: per-sequence status words are not implemented (WS-BI-1)", op);
}

// ---- the backend ----------------------------------------------------------------------------

class Mi355xBackend final : public MiBackend {
public:
    Mi355xBackend(int device, MiOptions options)
        : device_(device),
          invariant_gemv_(options.batch_invariant == BatchInvariantKernel::Exact ? kGemmSlabExactInvariant : kGemvSlab) {
        int n = 0;
        CHECK(hipGetDeviceCount(&n) == hipSuccess && device >= 0 && device < n, ErrorCode::Device,
              "mi355x backend: no HIP device %d (%d visible)", device, n);
        CHECK(hipSetDevice(device) == hipSuccess, ErrorCode::Device, "mi355x backend: hipSetDevice(%d) failed", device);
        hipDeviceProp_t prop{};
        if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
            name_ = prop.gcnArchName;
            cus_ = prop.multiProcessorCount;
        }
    }

    Kind kind() const noexcept override { return Kind::Hip; }
    std::string describe() const override {
        char buf[256];
        std::snprintf(buf, sizeof buf, "mi355x (%s, %d CUs, device %d): SLAB wave64 gemv + bf16 MFMA gemm", name_.c_str(), cus_,
                      device_);
        return buf;
    }
    Limits limits() const noexcept override {
        Limits l;
        l.lm_head_ids = true;
        // Every variant's fused norm is bitwise rms_norm then the same variant unfused; the
        // reference-order variant normalizes a vector at a time into a 4 Mi-float buffer.
        l.max_fused_norm_cols = 4u << 20;
        return l;
    }
    bool lost() const noexcept override { return lost_; }

    void poison(bool kernel_fault) {
        if (kernel_fault) poisoned_ = true;
        else lost_ = true;
    }

    std::unique_ptr<Buffer> allocate(std::uint64_t bytes, Tier tier) override {
        check_alive("allocate");
        void* mem = nullptr;
        const std::uint64_t n = std::max<std::uint64_t>(bytes, 1);
        if (tier == Tier::Vram) {
            CHECK(hipMalloc(&mem, n) == hipSuccess, ErrorCode::Memory, "mi355x backend: cannot allocate %llu bytes",
                  (unsigned long long)bytes);
            // Zero-filled like the CPU backend's allocate, and complete before this returns: the
            // fill runs on the null stream, which the backend's non-blocking streams do not wait
            // for, so an unsynchronized fill could land after the buffer's first upload or kernel
            // write on another stream and zero it.
            const hipError_t fe = hipMemsetAsync(mem, 0, n, nullptr);
            const hipError_t se = fe == hipSuccess ? hipStreamSynchronize(nullptr) : fe;
            if (se != hipSuccess) {
                (void)hipFree(mem);
                fail(ErrorCode::Device, "mi355x backend: zero-filling %llu bytes failed: %s", (unsigned long long)bytes,
                     hipGetErrorString(se));
            }
            return std::make_unique<DeviceBuffer>(this, mem, bytes, tier, true, false, WeightLayout::Gguf, SlabMeta{});
        }
        CHECK(hipHostMalloc(&mem, n, hipHostMallocDefault) == hipSuccess, ErrorCode::Memory,
              "mi355x backend: cannot allocate %llu pinned bytes", (unsigned long long)bytes);
        std::memset(mem, 0, n);
        return std::make_unique<DeviceBuffer>(this, mem, bytes, tier, true, true, WeightLayout::Gguf, SlabMeta{});
    }

    std::unique_ptr<Buffer> import_host(std::span<std::byte>) override {
        // As the reference's HIP backend on a device (hip_adapter.cpp:495-500).
        fail(ErrorCode::Unsupported, "mi355x backend: import_host is not supported on a device (copy into a backend buffer)");
    }

    std::unique_ptr<Buffer> import_host_readonly(std::span<const std::byte> bytes) override {
        check_alive("import_host_readonly");
        void* mem = nullptr;
        const std::uint64_t n = std::max<std::uint64_t>(bytes.size(), 1);
        CHECK(hipMalloc(&mem, n) == hipSuccess, ErrorCode::Memory, "mi355x backend: cannot allocate %llu bytes",
              (unsigned long long)bytes.size());
        if (!bytes.empty() && hipMemcpy(mem, bytes.data(), bytes.size(), hipMemcpyHostToDevice) != hipSuccess) {
            (void)hipFree(mem);
            fail(ErrorCode::Device, "mi355x backend: weight upload failed");
        }
        return std::make_unique<DeviceBuffer>(this, mem, bytes.size(), Tier::Vram, false, false, WeightLayout::Gguf, SlabMeta{});
    }

    std::unique_ptr<Buffer> import_weights(std::span<const std::byte> gguf, DType type, std::uint32_t rows, std::uint32_t cols,
                                           std::uint64_t row_stride) override {
        check_alive("import_weights");
        const auto t = static_cast<std::uint32_t>(type);
        const std::uint64_t rb = halo_mi_row_bytes(t, cols);
        CHECK(type != DType::F32 && rb != 0 && halo_mi_slab_bytes(t, 1, cols) != 0, ErrorCode::Unsupported,
              "import_weights: %s x %u has no SLAB layout", type_name(type), cols);
        const std::uint64_t stride = row_stride ? row_stride : rb;
        CHECK(rows == 0 || gguf.size() >= (rows - 1) * stride + rb, ErrorCode::Kernel,
              "import_weights: %zu bytes hold fewer than %u rows", gguf.size(), rows);
        const std::uint64_t bytes = halo_mi_slab_bytes(t, rows, cols);
        void* mem = nullptr;
        CHECK(hipMalloc(&mem, std::max<std::uint64_t>(bytes, 1)) == hipSuccess, ErrorCode::Memory,
              "import_weights: cannot allocate %llu bytes", (unsigned long long)bytes);
        auto buf = std::make_unique<DeviceBuffer>(this, mem, bytes, Tier::Vram, false, false, WeightLayout::Slab,
                                                  SlabMeta{type, rows, cols});
        check_abi(halo_mi_upload_slab(t, gguf.data(), stride, rows, cols, mem, 0, nullptr));
        return buf;
    }

    std::unique_ptr<Stream> create_stream() override {
        check_alive("create_stream");
        hipStream_t s = nullptr;
        CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess, ErrorCode::Device,
              "mi355x backend: cannot create a stream");
        void* status = nullptr;
        if (hipMalloc(&status, 256) != hipSuccess) {
            (void)hipStreamDestroy(s);
            fail(ErrorCode::Memory, "mi355x backend: cannot allocate a stream's status word");
        }
        if (hipMemsetAsync(status, 0, 4, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
            (void)hipFree(status);
            (void)hipStreamDestroy(s);
            fail(ErrorCode::Device, "mi355x backend: cannot clear a stream's status word");
        }
        return std::make_unique<HipStream>(this, s, static_cast<std::uint32_t*>(status));
    }

    void upload(Stream& s, TensorRef dst, std::span<const std::byte> src) override {
        HipStream& st = stream(s, "upload");
        const Resolver r(this, "upload");
        const Operand d = r.get(dst, 1, src.size(), 1, Access::Write, "dst");
        if (src.empty()) return;
        CHECK(hipMemcpyAsync(d.base, src.data(), src.size(), hipMemcpyHostToDevice, (hipStream_t)st.native()) == hipSuccess,
              ErrorCode::Device, "upload: hipMemcpyAsync failed");
    }

    void download(Stream& s, TensorRef src, std::span<std::byte> dst) override {
        HipStream& st = stream(s, "download");
        const Resolver r(this, "download");
        const Operand o = r.get(src, 1, dst.size(), 1, Access::Read, "src");
        if (dst.empty()) return;
        CHECK(hipMemcpyAsync(dst.data(), o.base, dst.size(), hipMemcpyDeviceToHost, (hipStream_t)st.native()) == hipSuccess,
              ErrorCode::Device, "download: hipMemcpyAsync failed");
    }

    std::span<const VariantInfo> variants(OpId op, std::string_view) const override {
        auto first = std::find_if(kVariants.begin(), kVariants.end(), [&](const VariantInfo& v) { return v.op == op; });
        auto last = std::find_if(first, kVariants.end(), [&](const VariantInfo& v) { return v.op != op; });
        return {first, last};
    }

    void dequant_rows(Stream& s, const DequantRowsArgs& a) override {
        HipStream& st = stream(s, "GET_ROWS");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kDequantRows, ErrorCode::Config,
              "GET_ROWS: unknown kernel variant id %u", a.kernel.variant_id);
        const Resolver r(this, "GET_ROWS");
        const auto t = static_cast<std::uint32_t>(a.type);
        const std::uint64_t rb = row_bytes(a.type, a.cols, r.op());
        CHECK(a.first_row <= a.n_rows_table && a.n_rows <= a.n_rows_table - a.first_row, ErrorCode::Kernel,
              "GET_ROWS: rows [%u, %u) out of %u", a.first_row, a.first_row + a.n_rows, a.n_rows_table);
        const bool slab = is_slab(a.table);
        const Operand table = slab ? r.slab(a.table, a.type, a.n_rows_table, a.cols, "table")
                                   : r.get(a.table, a.n_rows_table, rb, a.type == DType::F32 ? kF32 : 1, Access::Read, "table");
        const Operand out = r.f32(a.out, a.n_rows, a.cols, Access::Write, "out");
        r.no_overlap(out, table);
        if (a.n_rows == 0 || a.cols == 0) return;
        check_abi(halo_mi_dequant_rows(t, slab ? HALO_MI_LAYOUT_SLAB : HALO_MI_LAYOUT_GGUF, table.base, slab ? 0 : table.stride,
                                       a.n_rows_table, a.cols, a.first_row, a.n_rows, reinterpret_cast<float*>(out.base),
                                       out.stride / kF32, st.native()));
    }

    // GET_ROWS with device ids (GetRowsArgs, backend.h:254-263): the id range is checked by the
    // kernel, which sets the stream's status word as the reference's HIP backend does
    // (backends/hip/src/ops.cpp:982-1012); the stream's wait() reports it as Error(Kernel).
    void get_rows(Stream& s, const GetRowsArgs& a) override {
        HipStream& st = stream(s, "GET_ROWS");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kDequantRows, ErrorCode::Config,
              "GET_ROWS: unknown kernel variant id %u", a.kernel.variant_id);
        check_no_status(a.status, "GET_ROWS");
        const Resolver r(this, "GET_ROWS");
        const auto t = static_cast<std::uint32_t>(a.type);
        const std::uint64_t rb = row_bytes(a.type, a.cols, r.op());
        const bool slab = is_slab(a.table);
        const Operand table = slab ? r.slab(a.table, a.type, a.n_rows, a.cols, "table")
                                   : r.get(a.table, a.n_rows, rb, a.type == DType::F32 ? kF32 : 1, Access::Read, "table");
        const Operand ids = r.get(a.ids, 1, mul_u64(a.n_ids, 4, r.op(), "ids"), 4, Access::Read, "ids");
        const Operand out = r.f32(a.out, a.n_ids, a.cols, Access::Write, "out");
        r.no_overlap(out, table);
        r.no_overlap(out, ids);
        if (a.n_ids == 0 || a.cols == 0) return;
        halo_mi_get_rows_params p{t, slab ? (std::uint32_t)HALO_MI_LAYOUT_SLAB : (std::uint32_t)HALO_MI_LAYOUT_GGUF,
                                  table.base, slab ? 0 : table.stride, a.n_rows, a.cols,
                                  reinterpret_cast<const std::int32_t*>(ids.base), a.n_ids,
                                  reinterpret_cast<float*>(out.base), out.stride / kF32, st.get_rows_status(), 1u};
        check_abi(halo_mi_get_rows(&p, st.native()));
    }

    // RMS_NORM (RmsNormArgs, backend.h:267-272): exact aliasing of out and x is allowed, as
    // cpu::rms_norm's check_alias_exact_or_disjoint (backends/cpu/ops_basic.cpp:22) allows it.
    void rms_norm(Stream& s, const RmsNormArgs& a) override {
        HipStream& st = stream(s, "RMS_NORM");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kRmsNorm, ErrorCode::Config,
              "RMS_NORM: unknown kernel variant id %u", a.kernel.variant_id);
        const Resolver r(this, "RMS_NORM");
        const Operand x = r.f32(a.x, a.rows, a.cols, Access::Read, "x");
        const Operand w = r.f32(a.w, 1, a.cols, Access::Read, "w");
        const Operand out = r.f32(a.out, a.rows, a.cols, Access::Write, "out");
        if (!(out.base == x.base && out.stride == x.stride)) r.no_overlap(out, x);
        r.no_overlap(out, w);
        if (a.rows == 0 || a.cols == 0) return;
        check_abi(halo_mi_rms_norm(reinterpret_cast<const float*>(x.base), x.stride / kF32,
                                   reinterpret_cast<const float*>(w.base), reinterpret_cast<float*>(out.base),
                                   out.stride / kF32, a.rows, a.cols, a.eps, st.native()));
    }

    void gemv(Stream& s, const GemvArgs& a) override {
        HipStream& st = stream(s, "MATMUL");
        CHECK(has_variant(OpId::Gemv, a.kernel.variant_id), ErrorCode::Config, "MATMUL: unknown kernel variant id %u",
              a.kernel.variant_id);
        CHECK(a.gates.n_v == 0, ErrorCode::Unsupported, "MATMUL: the GDN gates epilogue (GemvArgs::gates) is Vulkan-only");
        const Resolver r(this, "MATMUL");
        const auto t = static_cast<std::uint32_t>(a.wtype);
        const std::uint64_t rb = row_bytes(a.wtype, a.cols, r.op());
        const bool slab = is_slab(a.w);
        std::uint32_t variant = a.kernel.variant_id;
        if (variant == 0) variant = slab ? kGemvSlabAuto : kGemvGgufRef;
        // rows must not depend on the batch unless the caller accepts the GEMM's numerics: the
        // backend's batch-invariant family
        if (variant == kGemvSlabAuto && !a.allow_gemm) variant = invariant_gemv_;
        CHECK(slab == (variant != kGemvGgufRef), ErrorCode::Config, "MATMUL: variant %u does not read the %s layout", variant,
              slab ? "SLAB" : "GGUF");
        const Operand w = slab ? r.slab(a.w, a.wtype, a.rows, a.cols, "w")
                               : r.get(a.w, a.rows, rb, a.wtype == DType::F32 ? kF32 : 1, Access::Read, "w");
        const Operand x = r.f32(a.x, a.n_vec, a.cols, Access::Read, "x");
        const Operand y = r.f32(a.y, a.n_vec, a.rows, Access::Write, "y");
        r.no_overlap(y, x);
        r.no_overlap(y, w);
        const Operand nw = a.norm_w.empty() ? Operand{} : r.f32(a.norm_w, 1, a.cols, Access::Read, "norm_w");
        r.no_overlap(y, nw);
        if (a.n_vec == 0 || a.rows == 0) return;
        const bool gemm = variant == kGemmSlabBf16 || variant == kGemmSlabBf16M512 || variant == kGemmSlabBf16SmallM ||
                          (variant == kGemvSlabAuto && a.n_vec > 8);
        if (gemm)
            CHECK(reinterpret_cast<std::uintptr_t>(x.base) % 16 == 0 && x.stride % 16 == 0, ErrorCode::Kernel,
                  "MATMUL: the MFMA GEMM needs 16-byte aligned x rows");
        halo_mi_gemv_params p{t,      slab ? (std::uint32_t)HALO_MI_LAYOUT_SLAB : (std::uint32_t)HALO_MI_LAYOUT_GGUF,
                              w.base, slab ? 0 : w.stride,
                              reinterpret_cast<const float*>(x.base), x.stride / kF32,
                              reinterpret_cast<float*>(y.base), y.stride / kF32,
                              a.rows, a.cols, a.n_vec, abi_gemv_variant(variant),
                              reinterpret_cast<const float*>(nw.base), a.norm_eps};
        check_abi(halo_mi_gemv(&p, st.native()));
    }

    void swiglu(Stream& s, const EltwiseArgs& a) override {
        HipStream& st = stream(s, "SWIGLU");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kSwiglu, ErrorCode::Config, "SWIGLU: unknown kernel variant id %u",
              a.kernel.variant_id);
        const Resolver r(this, "SWIGLU");
        const Operand g = r.f32(a.a, a.rows, a.cols, Access::Read, "a");
        const Operand u = r.f32(a.b, a.rows, a.cols, Access::Read, "b");
        const Operand out = r.f32(a.out, a.rows, a.cols, Access::Write, "out");
        r.no_overlap(out, g);
        r.no_overlap(out, u);
        if (a.rows == 0 || a.cols == 0) return;
        check_abi(halo_mi_swiglu(reinterpret_cast<const float*>(g.base), g.stride / kF32, reinterpret_cast<const float*>(u.base),
                                 u.stride / kF32, reinterpret_cast<float*>(out.base), out.stride / kF32, a.rows, a.cols,
                                 st.native()));
    }

    void gate_up_swiglu(Stream& s, const GateUpArgs& a) override {
        HipStream& st = stream(s, "GATE_UP_SWIGLU");
        CHECK(has_variant(OpId::GateUpSwiglu, a.kernel.variant_id), ErrorCode::Config,
              "GATE_UP_SWIGLU: unknown kernel variant id %u", a.kernel.variant_id);
        const Resolver r(this, "GATE_UP_SWIGLU");
        (void)row_bytes(a.wtype, a.cols, r.op());
        const Operand wg = r.slab(a.w_gate, a.wtype, a.rows, a.cols, "w_gate");
        const Operand wu = r.slab(a.w_up, a.wtype, a.rows, a.cols, "w_up");
        const Operand x = r.f32(a.x, a.n_vec, a.cols, Access::Read, "x");
        const Operand out = r.f32(a.out, a.n_vec, a.rows, Access::Write, "out");
        r.no_overlap(out, x);
        r.no_overlap(out, wg);
        r.no_overlap(out, wu);
        const Operand nw = a.norm_w.empty() ? Operand{} : r.f32(a.norm_w, 1, a.cols, Access::Read, "norm_w");
        r.no_overlap(out, nw);
        if (a.n_vec == 0 || a.rows == 0) return;
        const std::uint32_t id = a.kernel.variant_id;
        const std::uint32_t variant = id == kGateUpGemv         ? HALO_MI_GEMV_SLAB
                                      : id == kGateUpGemm       ? HALO_MI_GEMM_SLAB_BF16
                                      : id == kGateUpGemmM512   ? HALO_MI_GEMM_SLAB_BF16_M512
                                      : id == kGateUpGemmSmallM ? HALO_MI_GEMM_SLAB_BF16_SMALL_M
                                      : id == kGateUpExactSmallM ? HALO_MI_GEMM_SLAB_EXACT_SMALL_M
                                      : id == kGateUpExactInvariant ? HALO_MI_GEMM_SLAB_EXACT_INVARIANT
                                      : a.allow_gemm            ? HALO_MI_GEMV_SLAB_AUTO
                                                                : abi_gemv_variant(invariant_gemv_);
        halo_mi_gate_up_params p{static_cast<std::uint32_t>(a.wtype), HALO_MI_LAYOUT_SLAB, wg.base, wu.base,
                                 reinterpret_cast<const float*>(x.base), x.stride / kF32, reinterpret_cast<float*>(out.base),
                                 out.stride / kF32, a.rows, a.cols, a.n_vec, variant,
                                 reinterpret_cast<const float*>(nw.base), a.norm_eps};
        check_abi(halo_mi_gate_up_swiglu(&p, st.native()));
    }

    // LM_HEAD (CpuBackend::lm_head, src/backend/cpu_backend.cpp:669-770): the operands of the
    // gemv (y optional), result and the optional ids, checked before anything is enqueued. The
    // gemv's kernel choice picks the path: the default fuses the argmax into the slab gemv
    // (SLAB weights) or ranks the logits after the reference-order gemv (GGUF weights, which
    // then need gemv.y); an explicit gemv variant keeps its meaning.
    void lm_head(Stream& s, const LmHeadArgs& a) override {
        HipStream& st = stream(s, "LM_HEAD");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kLmHeadFused, ErrorCode::Config,
              "LM_HEAD: unknown kernel variant id %u", a.kernel.variant_id);
        check_no_status(a.status, "LM_HEAD");
        const GemvArgs& g = a.gemv;
        CHECK(has_variant(OpId::Gemv, g.kernel.variant_id), ErrorCode::Config, "LM_HEAD: unknown gemv variant id %u",
              g.kernel.variant_id);
        CHECK(a.ids_slots.empty() == a.ids_scatter.empty() && (a.ids_scatter.empty() || !a.ids.empty()), ErrorCode::Api,
              "LM_HEAD: ids_slots and ids_scatter go together, and only with ids");
        const Resolver r(this, "LM_HEAD");
        const auto t = static_cast<std::uint32_t>(g.wtype);
        const std::uint64_t rb = row_bytes(g.wtype, g.cols, r.op());
        const bool slab = is_slab(g.w);
        std::uint32_t variant = g.kernel.variant_id;
        if (variant == 0) variant = slab ? kGemvSlab : kGemvGgufRef;
        CHECK(slab == (variant != kGemvGgufRef), ErrorCode::Config, "LM_HEAD: variant %u does not read the %s layout",
              variant, slab ? "SLAB" : "GGUF");
        const Operand w = slab ? r.slab(g.w, g.wtype, g.rows, g.cols, "w")
                               : r.get(g.w, g.rows, rb, g.wtype == DType::F32 ? kF32 : 1, Access::Read, "w");
        const Operand x = r.f32(g.x, g.n_vec, g.cols, Access::Read, "x");
        const bool logits = !g.y.empty();
        const Operand y = logits ? r.f32(g.y, g.n_vec, g.rows, Access::Write, "logits") : Operand{};
        const Operand res = r.get(a.result, 1, mul_u64(g.n_vec, kArgmaxResultBytes, r.op(), "result"), 4, Access::Write,
                                  "result");
        for (const Operand* o : {&y, &res}) {
            r.no_overlap(*o, x);
            r.no_overlap(*o, w);
        }
        r.no_overlap(res, y);
        const Operand nw = g.norm_w.empty() ? Operand{} : r.f32(g.norm_w, 1, g.cols, Access::Read, "norm_w");
        r.no_overlap(y, nw);
        r.no_overlap(res, nw);
        Operand ids{}, slots{}, scat{};
        if (!a.ids.empty()) {
            ids = r.get(a.ids, 1, mul_u64(g.n_vec, 4, r.op(), "ids"), 4, Access::Write, "ids");
            for (const Operand* o : std::initializer_list<const Operand*>{&x, &w, &y, &res}) r.no_overlap(ids, *o);
        }
        std::uint64_t scat_len = 0;
        if (!a.ids_scatter.empty()) {
            slots = r.get(a.ids_slots, 1, mul_u64(g.n_vec, 4, r.op(), "ids_slots"), 4, Access::Read, "ids_slots");
            scat_len = a.ids_scatter.view_bytes() / 4;
            CHECK(scat_len >= 1, ErrorCode::Api, "LM_HEAD: ids_scatter holds no int32");
            scat = r.get(a.ids_scatter, 1, scat_len * 4, 4, Access::Write, "ids_scatter");
            for (const Operand* o : std::initializer_list<const Operand*>{&x, &w, &y, &res, &ids, &slots})
                r.no_overlap(scat, *o);
            for (const Operand* o : std::initializer_list<const Operand*>{&y, &res, &ids}) r.no_overlap(*o, slots);
        }
        if (g.n_vec == 0) return;
        halo_mi_lm_head_params p{};
        p.gemv = halo_mi_gemv_params{t,      slab ? (std::uint32_t)HALO_MI_LAYOUT_SLAB : (std::uint32_t)HALO_MI_LAYOUT_GGUF,
                                     w.base, slab ? 0 : w.stride,
                                     reinterpret_cast<const float*>(x.base), x.stride / kF32,
                                     logits ? reinterpret_cast<float*>(y.base) : nullptr, logits ? y.stride / kF32 : 0,
                                     g.rows, g.cols, g.n_vec, abi_gemv_variant(variant),
                                     reinterpret_cast<const float*>(nw.base), g.norm_eps};
        p.result = res.base;
        p.valid_rows = a.valid_rows;
        p.ids = reinterpret_cast<std::int32_t*>(ids.base);
        p.ids_slots = reinterpret_cast<const std::uint32_t*>(slots.base);
        p.ids_scatter = reinterpret_cast<std::int32_t*>(scat.base);
        p.ids_scatter_len = scat_len;
        check_abi(halo_mi_lm_head(&p, st.native()));
    }

    // ARGMAX (CpuBackend::argmax, src/backend/cpu_backend.cpp:772-783): the result words of each
    // vector; a NaN logit poisons its vector's words (the reference HIP backend's device form of
    // the CPU's Error(Kernel); decode_argmax reports it).
    void argmax(Stream& s, const ArgmaxArgs& a) override {
        HipStream& st = stream(s, "ARGMAX_FUSED");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kArgmax, ErrorCode::Config,
              "ARGMAX_FUSED: unknown kernel variant id %u", a.kernel.variant_id);
        check_no_status(a.status, "ARGMAX_FUSED");
        const Resolver r(this, "ARGMAX_FUSED");
        const Operand l = r.f32(a.logits, a.n_vec, a.n, Access::Read, "logits");
        const Operand res = r.get(a.result, 1, mul_u64(a.n_vec, kArgmaxResultBytes, r.op(), "result"), 4, Access::Write, "result");
        r.no_overlap(res, l);
        if (a.n_vec == 0) return;
        CHECK(a.n > 0, ErrorCode::Kernel, "ARGMAX_FUSED: empty row");
        check_abi(halo_mi_argmax(reinterpret_cast<const float*>(l.base), l.stride / kF32, a.n, a.n_vec, res.base, st.native()));
    }

    // COPY (CpuBackend::copy): bytes from src to dst, in stream order; the ranges must not overlap.
    void copy(Stream& s, const CopyArgs& a) override {
        HipStream& st = stream(s, "COPY");
        CHECK(a.kernel.variant_id == 0 || a.kernel.variant_id == kCopy, ErrorCode::Config, "COPY: unknown kernel variant id %u",
              a.kernel.variant_id);
        const Resolver r(this, "COPY");
        const Operand src = r.get(a.src, 1, a.bytes, 1, Access::Read, "src");
        const Operand dst = r.get(a.dst, 1, a.bytes, 1, Access::Write, "dst");
        r.no_overlap(dst, src);
        if (a.bytes == 0) return;
        CHECK(hipMemcpyAsync(dst.base, src.base, a.bytes, hipMemcpyDeviceToDevice, (hipStream_t)st.native()) == hipSuccess,
              ErrorCode::Device, "COPY: hipMemcpyAsync failed");
    }

    // The ops of the reference interface outside this path.
    void add_rms_norm(Stream&, const AddRmsNormArgs&) override { unsupported(OpId::AddRmsNorm); }
    void gdn_gates(Stream&, const GdnGateArgs&) override { unsupported(OpId::GdnGates); }
    void conv1d_silu(Stream&, const Conv1dArgs&) override { unsupported(OpId::Conv1dSilu); }
    void gated_delta_rule(Stream&, const GdnArgs&) override { unsupported(OpId::GatedDeltaRule); }
    void gated_rms_norm(Stream&, const GatedNormArgs&) override { unsupported(OpId::GatedRmsNorm); }
    void partial_rope(Stream&, const RopeArgs&) override { unsupported(OpId::PartialRope); }
    void kv_write(Stream&, const KvWriteArgs&) override { unsupported(OpId::KvWrite); }
    void attention(Stream&, const AttentionArgs&) override { unsupported(OpId::Attention); }
    void mul_sigmoid(Stream&, const EltwiseArgs&) override { unsupported(OpId::MulSigmoid); }
    void add(Stream&, const EltwiseArgs&) override { unsupported(OpId::Add); }
    void top_k(Stream&, const TopKArgs&) override { unsupported(OpId::TopK); }

private:
    [[noreturn]] static void unsupported(OpId op) {
        fail(ErrorCode::Unsupported, "%.*s is not implemented by the mi355x backend (quantized matmul path only)",
             (int)op_name(op).size(), op_name(op).data());
    }

    static bool is_slab(const TensorRef& t) {
        const auto* b = dynamic_cast<const DeviceBuffer*>(t.buffer);
        return b != nullptr && b->layout() == WeightLayout::Slab;
    }

    void check_alive(const char* op) const {
        CHECK(!lost_, ErrorCode::Device, "%s: the device behind this backend is lost", op);
        CHECK(!poisoned_, ErrorCode::Kernel, "%s: a previous kernel fault poisoned this backend", op);
    }

    HipStream& stream(Stream& s, const char* op) {
        check_alive(op);
        auto* hs = dynamic_cast<HipStream*>(&s);
        CHECK(hs != nullptr && hs->owner() == this, ErrorCode::Kernel, "%s: stream belongs to another backend", op);
        return *hs;
    }

    // The weight types of the reference HIP backend's GEMV, GET_ROWS and dequant ops
    // (backends/hip/src/ops.cpp:531-549): the library's GGUF-layout kernels also decode BF16,
    // Q4_1, Q5_0, Q5_1 and Q2_K, but this backend refuses them as the reference's does.
    static std::uint64_t row_bytes(DType t, std::uint32_t cols, const char* op) {
        switch (t) {
            case DType::F32: case DType::F16: case DType::Q4_0: case DType::Q8_0: case DType::Q3_K: case DType::Q4_K:
            case DType::Q5_K: case DType::Q6_K: case DType::IQ3_S: case DType::IQ4_NL: case DType::IQ4_XS: break;
            default:
                fail(ErrorCode::Unsupported,
                     "%s: weight type id %u has no HIP GEMV kernel (F32, F16, Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ3_S, "
                     "IQ4_NL, IQ4_XS)", op, static_cast<unsigned>(t));
        }
        const std::uint64_t rb = halo_mi_row_bytes(static_cast<std::uint32_t>(t), cols);
        if (rb == 0) {
            const std::uint64_t one = halo_mi_row_bytes(static_cast<std::uint32_t>(t), 256);
            CHECK(one == 0, ErrorCode::Kernel, "%s: %u elements is not a multiple of the %s block size", op, cols, type_name(t));
            fail(ErrorCode::Unsupported, "%s: no kernel for weight type %u", op, static_cast<unsigned>(t));
        }
        return rb;
    }

    int device_;
    std::uint32_t invariant_gemv_;  // MATMUL registry id of the batch-invariant family (MiOptions)
    int cus_ = 0;
    std::string name_;
    bool lost_ = false, poisoned_ = false;
};

void HipStream::wait() {
    const hipError_t e = hipStreamSynchronize(s_);
    if (e != hipSuccess) {
        const bool kernel_fault = e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorAssert;
        owner_->poison(kernel_fault);
        throw Error(kernel_fault ? ErrorCode::Kernel : ErrorCode::Device, std::string("stream wait: ") + hipGetErrorString(e));
    }
    // a split-K reduction that gave up waiting: the device did not finish its work in the wait budget
    if (halo_mi_stream_check(s_) != HALO_MI_OK) {
        owner_->poison(false);
        throw Error(ErrorCode::Device, std::string("stream wait: ") + halo_mi_last_error());
    }
    if (!status_used_) return;
    status_used_ = false;
    std::uint32_t word = 0;
    if (hipMemcpy(&word, status_, 4, hipMemcpyDeviceToHost) != hipSuccess ||
        (word != 0 && hipMemsetAsync(status_, 0, 4, s_) != hipSuccess) || hipStreamSynchronize(s_) != hipSuccess) {
        owner_->poison(false);
        throw Error(ErrorCode::Device, "stream wait: cannot read the status word");
    }
    CHECK(!(word & kStatusBadIndex), ErrorCode::Kernel, "GET_ROWS: an id lies outside the table (status 0x%x)", word);
}

}  // namespace

std::string_view to_string(ErrorCode c) noexcept {
    switch (c) {
        case ErrorCode::Model: return "MODEL_ERROR";
        case ErrorCode::Memory: return "MEMORY_ERROR";
        case ErrorCode::Backend: return "BACKEND_ERROR";
        case ErrorCode::Kernel: return "KERNEL_ERROR";
        case ErrorCode::Config: return "CONFIG_ERROR";
        case ErrorCode::Api: return "API_ERROR";
        case ErrorCode::Device: return "DEVICE_ERROR";
        case ErrorCode::Unsupported: return "UNSUPPORTED_ERROR";
        case ErrorCode::Io: return "IO_ERROR";
        case ErrorCode::Cancelled: return "CANCELLED";
    }
    return "UNKNOWN_ERROR";
}

Error::Error(ErrorCode code, const std::string& message)
    : std::runtime_error(std::string(to_string(code)) + ": " + message), code_(code) {}

std::string_view to_string(Kind k) noexcept {
    switch (k) {
        case Kind::Cpu: return "cpu";
        case Kind::Hip: return "hip";
        case Kind::HipEmulation: return "hip-emulation";
        case Kind::Vulkan: return "vulkan";
    }
    return "unknown";
}

// The op names of the reference's registry (src/backend/backend.cpp:22-46).
std::string_view op_name(OpId op) noexcept {
    switch (op) {
        case OpId::GetRows: return "GET_ROWS";
        case OpId::RmsNorm: return "RMS_NORM";
        case OpId::AddRmsNorm: return "ADD_RMS_NORM";
        case OpId::Gemv: return "MATMUL";
        case OpId::GdnGates: return "GDN_GATE";
        case OpId::Conv1dSilu: return "CONV1D_SHORT";
        case OpId::GatedDeltaRule: return "GATED_DELTANET";
        case OpId::GatedRmsNorm: return "GATED_NORM";
        case OpId::PartialRope: return "PARTIAL_ROPE";
        case OpId::KvWrite: return "KV_WRITE";
        case OpId::Attention: return "ATTENTION";
        case OpId::Swiglu: return "SWIGLU";
        case OpId::MulSigmoid: return "MUL_SIGMOID";
        case OpId::Add: return "ADD";
        case OpId::LmHead: return "LM_HEAD";
        case OpId::Argmax: return "ARGMAX_FUSED";
        case OpId::TopK: return "TOP_K";
        case OpId::Copy: return "COPY";
        case OpId::GateUpSwiglu: return "GATE_UP_SWIGLU";
    }
    return "UNKNOWN";
}

TensorRef TensorRef::shifted(std::uint64_t delta) const {
    CHECK(bytes == 0 || delta < bytes, ErrorCode::Kernel, "TensorRef::shifted: %llu bytes past a %llu-byte view",
          (unsigned long long)delta, (unsigned long long)bytes);
    CHECK(offset <= std::numeric_limits<std::uint64_t>::max() - delta, ErrorCode::Kernel, "TensorRef::shifted: offset overflow");
    return {buffer, offset + delta, bytes == 0 ? 0 : bytes - delta, row_stride};
}

namespace {
template <class A>
const A& args_of(const OpInvocation& inv) {
    const A* a = std::get_if<A>(&inv.args);
    if (a == nullptr) {
        const std::string_view n = op_name(inv.op);
        fail(ErrorCode::Api, "run_op: %.*s called with the args of another op", (int)n.size(), n.data());
    }
    return *a;
}
}  // namespace

// Backend::run_op (src/backend/backend.cpp:57-81 of the reference): the typed method of inv.op.
void Backend::run_op(Stream& s, const OpInvocation& inv) {
    switch (inv.op) {
        case OpId::GetRows: return get_rows(s, args_of<GetRowsArgs>(inv));
        case OpId::RmsNorm: return rms_norm(s, args_of<RmsNormArgs>(inv));
        case OpId::AddRmsNorm: return add_rms_norm(s, args_of<AddRmsNormArgs>(inv));
        case OpId::Gemv: return gemv(s, args_of<GemvArgs>(inv));
        case OpId::GdnGates: return gdn_gates(s, args_of<GdnGateArgs>(inv));
        case OpId::Conv1dSilu: return conv1d_silu(s, args_of<Conv1dArgs>(inv));
        case OpId::GatedDeltaRule: return gated_delta_rule(s, args_of<GdnArgs>(inv));
        case OpId::GatedRmsNorm: return gated_rms_norm(s, args_of<GatedNormArgs>(inv));
        case OpId::PartialRope: return partial_rope(s, args_of<RopeArgs>(inv));
        case OpId::KvWrite: return kv_write(s, args_of<KvWriteArgs>(inv));
        case OpId::Attention: return attention(s, args_of<AttentionArgs>(inv));
        case OpId::Swiglu: return swiglu(s, args_of<EltwiseArgs>(inv));
        case OpId::MulSigmoid: return mul_sigmoid(s, args_of<EltwiseArgs>(inv));
        case OpId::Add: return add(s, args_of<EltwiseArgs>(inv));
        case OpId::LmHead: return lm_head(s, args_of<LmHeadArgs>(inv));
        case OpId::Argmax: return argmax(s, args_of<ArgmaxArgs>(inv));
        case OpId::TopK: return top_k(s, args_of<TopKArgs>(inv));
        case OpId::Copy: return copy(s, args_of<CopyArgs>(inv));
        case OpId::GateUpSwiglu: break;  // an addition with no args type in OpInvocation
    }
    fail(ErrorCode::Api, "run_op: unknown op id %u", static_cast<unsigned>(inv.op));
}

// decode_argmax (src/backend/backend.cpp:83-99 of the reference): a poisoned vector decodes as
// {-1, NaN} and does not stop the others.
std::vector<ArgmaxResult> decode_argmax(std::span<const std::byte> words) {
    CHECK(words.size() % kArgmaxResultBytes == 0, ErrorCode::Kernel, "decode_argmax: %zu bytes is not a multiple of %u",
          words.size(), kArgmaxResultBytes);
    const std::size_t n = words.size() / kArgmaxResultBytes;
    std::vector<ArgmaxResult> out(n);
    for (std::size_t i = 0; i < n; ++i) {
        std::array<std::uint32_t, 3> w{};
        std::memcpy(w.data(), words.data() + i * kArgmaxResultBytes, sizeof(w));
        out[i] = w[2] != 0 ? ArgmaxResult{-1, std::numeric_limits<float>::quiet_NaN()}
                           : ArgmaxResult{static_cast<std::int32_t>(w[0]), std::bit_cast<float>(w[1])};
    }
    return out;
}

std::unique_ptr<MiBackend> make_mi355x_backend(int device, MiOptions options) {
    return std::make_unique<Mi355xBackend>(device, options);
}

}  // namespace halo_mi::backend
