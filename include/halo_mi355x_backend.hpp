// halo_mi355x C++ backend: the host-side mirror of the reference's ADR-001 Backend interface
// (include/halo/backend/backend.h:104-584) for the quantized matrix-multiply path, built on
// the C ABI of halo_mi355x.h.
//
// Contract kept from the reference:
//  - every op validates all operands on the host and throws before anything is enqueued
//    (backend.h:5-9); work then runs in stream order; results are read after Stream::wait();
//  - error mapping (backend.h:24-26): shape / alias / range / alignment -> Error(Kernel);
//    dtype or limit -> Error(Unsupported); unknown variant id -> Error(Config); allocation ->
//    Error(Memory); a device fault at wait() -> Error(Kernel) and a poisoned backend, device
//    loss -> Error(Device) and a sticky lost() (ADR-001:402-414);
//  - aliasing (backend.h:15-19): an output may not overlap any operand;
//  - kernel selection by an explicit, append-only variant id (KernelChoice, 0 = default);
//  - one thread drives a Backend and its Streams.
// Ops of the reference interface outside this path throw Error(Unsupported).
//
// Additions (no counterpart in the reference): weights can be imported straight into the
// SLAB device layout (import_weights), and the FFN's gate/up/SwiGLU composition
// (src/models/qwen35.cpp:789-805) is one op, gate_up_swiglu.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>

namespace halo_mi::backend {

// ---- errors (include/halo/core/error.h:13-51) --------------------------------------------

enum class ErrorCode { Model, Memory, Backend, Kernel, Config, Api, Device, Unsupported, Io, Cancelled };

[[nodiscard]] std::string_view to_string(ErrorCode c) noexcept;

class Error : public std::runtime_error {
public:
    Error(ErrorCode code, const std::string& message);
    [[nodiscard]] ErrorCode code() const noexcept { return code_; }

private:
    ErrorCode code_;
};

// ---- types (backend.h:60-314) -------------------------------------------------------------

enum class DType : std::uint32_t { F32 = 0, Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ4_XS = 23 };
enum class Kind : std::uint8_t { Cpu, Hip, HipEmulation, Vulkan };
enum class Tier : std::uint8_t { Vram, Gtt, Host };
// How the bytes of a weight buffer are laid out (an addition of this backend).
enum class WeightLayout : std::uint8_t { Gguf, Slab };

class Backend;

class Buffer {
public:
    virtual ~Buffer() = default;
    [[nodiscard]] virtual std::uint64_t bytes() const noexcept = 0;
    [[nodiscard]] virtual Tier tier() const noexcept = 0;
    [[nodiscard]] virtual const Backend* backend() const noexcept = 0;
    [[nodiscard]] virtual bool writable() const noexcept = 0;
    /// Host address of byte 0, or null (device memory is never host-mapped; ADR A-4).
    [[nodiscard]] virtual const std::byte* host_data() const noexcept = 0;
    [[nodiscard]] virtual std::byte* host_ptr() const noexcept = 0;
    /// Device address of byte 0 (this backend's addition).
    [[nodiscard]] virtual void* device_ptr() const noexcept = 0;
    [[nodiscard]] virtual WeightLayout layout() const noexcept = 0;

protected:
    Buffer() = default;
    Buffer(const Buffer&) = default;
    Buffer& operator=(const Buffer&) = default;
};

struct TensorRef {
    const Buffer* buffer = nullptr;
    std::uint64_t offset = 0;
    std::uint64_t bytes = 0;
    std::uint64_t row_stride = 0;

    [[nodiscard]] bool empty() const noexcept { return buffer == nullptr; }
    [[nodiscard]] static TensorRef of(const Buffer& b) noexcept { return {&b, 0, 0, 0}; }
    [[nodiscard]] std::uint64_t view_bytes() const noexcept {
        if (bytes != 0 || buffer == nullptr) return bytes;
        return buffer->bytes() > offset ? buffer->bytes() - offset : 0;
    }
    [[nodiscard]] TensorRef with_stride(std::uint64_t s) const noexcept { return {buffer, offset, bytes, s}; }
};

struct KernelChoice {
    std::uint32_t variant_id = 0;
};

// Operator ids: the reference's values (backend.h:187-206), plus this backend's fused FFN op.
enum class OpId : std::uint16_t {
    GetRows = 0, RmsNorm = 1, AddRmsNorm = 2, Gemv = 3, GdnGates = 4, Conv1dSilu = 5, GatedDeltaRule = 6,
    GatedRmsNorm = 7, PartialRope = 8, KvWrite = 9, Attention = 10, Swiglu = 11, MulSigmoid = 12, Add = 13,
    LmHead = 14, Argmax = 15, TopK = 16, Copy = 17,
    GateUpSwiglu = 18,  // addition: gemv(gate) + gemv(up) + swiglu in one launch
};

struct VariantInfo {
    std::uint32_t id = 0;
    std::string_view name;
    OpId op = OpId::GetRows;
    std::string_view form;
};

struct Limits {
    std::uint32_t max_gdn_dk = 0, max_gdn_chunk = 0, max_head_dim = 0, max_conv_k = 0, max_top_k = 0, max_rope_dims = 0;
    bool gdn_chunked = false;
    std::uint64_t max_import_bytes = 0;
    std::uint64_t max_pool_buffer_bytes = 0;
    bool lm_head_ids = false;
    std::uint32_t max_fused_norm_cols = 0;
    bool gemv_gdn_gates = false;
    /// Largest n_vec of one gemv / gate_up_swiglu call (this backend's addition; 0 = none).
    std::uint32_t max_n_vec = 0;
};

/// GET_ROWS restricted to a contiguous row range (backend.h:254-263): out rows = dequantized
/// W rows [first_row, first_row + n_rows), bit-identical to tensor::dequantize_row.
struct DequantRowsArgs {
    DType type = DType::F32;
    TensorRef table{}, out{};
    std::uint32_t n_rows_table = 0, cols = 0, first_row = 0, n_rows = 0;
    KernelChoice kernel{};
};

/// GET_ROWS (backend.h:254-263): out[i] = dequant(table row ids[i]), bit-identical to
/// tensor::dequantize_row. ids: n_ids int32 in device memory. status (optional, one uint32 of
/// device memory; the reference's StatusRef): cleared, then kStatusBadIndex when an id lies
/// outside [0, n_rows) - that output row is not written. The CPU backend throws Error(Kernel)
/// instead (cpu_backend.cpp:296-299); ids on the device are only known to the kernel.
struct GetRowsArgs {
    DType type = DType::F32;
    TensorRef table{}, ids{}, out{};
    std::uint32_t n_rows = 0, cols = 0, n_ids = 0;
    KernelChoice kernel{};
    TensorRef status{};
};
/// The status bit of a GET_ROWS id outside the table (backends/hip/kernels/hd.h:156).
inline constexpr std::uint32_t kStatusBadIndex = 8u;

/// RMS_NORM (backend.h:267-272; cpu::rms_norm): rows x cols; w: [cols]. out may be x itself
/// (same stride), else must not overlap x. Bitwise equal to the CPU.
struct RmsNormArgs {
    TensorRef x{}, w{}, out{};
    std::uint32_t rows = 0, cols = 0;
    float eps = 1e-6f;
    KernelChoice kernel{};
};

/// MATMUL / QUANT_GEMV (backend.h:283-314): y[t][n] = sum_i x[t][i] W[n][i].
struct GemvArgs {
    DType wtype = DType::F32;
    TensorRef w{}, x{}, y{};
    std::uint32_t rows = 0, cols = 0, n_vec = 1;
    KernelChoice kernel{};
    /// Fused input norm (backend.h:292-299): y = W (rms_norm(x) * norm_w) with eps = norm_eps,
    /// x the raw rows; norm_w: [cols] fp32. Every variant and n_vec here (the reference takes it
    /// on one Vulkan path); its numerics per variant are halo_mi_gemv's (include/halo_mi355x.h).
    TensorRef norm_w{};
    float norm_eps = 1e-6f;
    /// As in the reference: off (the default), every row of y is bitwise the row an n_vec == 1 call
    /// gives, whatever n_vec (the SLAB default then runs the GEMV kernel at every n_vec). On, the
    /// SLAB default may run the bf16 MFMA GEMM for n_vec > 8 (its own tolerance, not batch-invariant).
    bool allow_gemm = false;
    struct Gates {
        TensorRef dt_bias{}, a{};
        std::uint32_t n_v = 0;
    } gates{};
};

/// ARGMAX result words of one vector: {index u32, value (f32 bits), nan (0/1)} (backend.h:430-431).
inline constexpr std::uint32_t kArgmaxResultBytes = 12;

/// LM_HEAD (backend.h:433-460): the gemv over the vocabulary + fused argmax (ties to the lowest
/// index; a NaN logit poisons its own vector; rows at or past valid_rows, when not 0, are not
/// ranked). gemv.y is optional (the full logits). result: n_vec * kArgmaxResultBytes. ids,
/// ids_slots / ids_scatter: optional, as in the reference (Limits::lm_head_ids); a slot past
/// ids_scatter's end is dropped (the reference's Vulkan behaviour, backend.h:453-457).
struct LmHeadArgs {
    GemvArgs gemv{};
    TensorRef result{};
    std::uint32_t valid_rows = 0;
    KernelChoice kernel{};
    TensorRef ids{};
    TensorRef ids_slots{};
    TensorRef ids_scatter{};
};

/// SWIGLU (backend.h:420-427): out = silu(a) * b, rows x cols.
struct EltwiseArgs {
    TensorRef a{}, b{}, out{};
    std::uint32_t rows = 0, cols = 0;
    KernelChoice kernel{};
};

/// Addition: out[t][n] = silu((Wg x_t)[n]) * (Wu x_t)[n]; Wg, Wu SLAB weights of one shape.
struct GateUpArgs {
    DType wtype = DType::Q4_K;
    TensorRef w_gate{}, w_up{}, x{}, out{};
    std::uint32_t rows = 0, cols = 0, n_vec = 1;
    KernelChoice kernel{};
    bool allow_gemm = false;  ///< same meaning as GemvArgs::allow_gemm
    TensorRef norm_w{};       ///< fused input norm, as GemvArgs::norm_w
    float norm_eps = 1e-6f;
};

class Stream {
public:
    virtual ~Stream() = default;
    virtual void submit() = 0;
    virtual void wait() = 0;  ///< throws the translated device error
    virtual void abort() noexcept = 0;
    /// The hipStream_t (this backend's addition).
    [[nodiscard]] virtual void* native() const noexcept = 0;

protected:
    Stream() = default;
};

class Backend {
public:
    virtual ~Backend() = default;
    Backend(const Backend&) = delete;
    Backend& operator=(const Backend&) = delete;

    [[nodiscard]] virtual Kind kind() const noexcept = 0;
    [[nodiscard]] virtual std::string describe() const = 0;
    [[nodiscard]] virtual Limits limits() const noexcept = 0;
    [[nodiscard]] virtual bool lost() const noexcept = 0;

    [[nodiscard]] virtual std::unique_ptr<Buffer> allocate(std::uint64_t bytes, Tier tier) = 0;
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_host(std::span<std::byte> bytes) = 0;
    /// Read-only import: the bytes are copied into VRAM as they are (GGUF layout).
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_host_readonly(std::span<const std::byte> bytes) = 0;
    /// Addition: read-only import of a rows x cols GGUF weight matrix (rows `row_stride` bytes
    /// apart, 0 = dense) into the SLAB layout, repacked on the device chunk by chunk.
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_weights(std::span<const std::byte> gguf, DType type,
                                                                 std::uint32_t rows, std::uint32_t cols,
                                                                 std::uint64_t row_stride = 0) = 0;
    [[nodiscard]] virtual std::unique_ptr<Stream> create_stream() = 0;
    virtual void upload(Stream& s, TensorRef dst, std::span<const std::byte> src) = 0;
    virtual void download(Stream& s, TensorRef src, std::span<std::byte> dst) = 0;

    [[nodiscard]] virtual std::span<const VariantInfo> variants(OpId op, std::string_view form = {}) const = 0;

    virtual void dequant_rows(Stream&, const DequantRowsArgs&) = 0;
    virtual void get_rows(Stream&, const GetRowsArgs&) = 0;
    virtual void rms_norm(Stream&, const RmsNormArgs&) = 0;
    virtual void gemv(Stream&, const GemvArgs&) = 0;
    virtual void swiglu(Stream&, const EltwiseArgs&) = 0;
    virtual void gate_up_swiglu(Stream&, const GateUpArgs&) = 0;
    virtual void lm_head(Stream&, const LmHeadArgs&) = 0;
    /// Any other op of the reference interface: Error(Unsupported) on this backend.
    [[noreturn]] void unsupported(OpId op) const;

protected:
    Backend() = default;
};

/// The MI355X backend on HIP device `device` (default 0). Error(Device) without a GPU.
[[nodiscard]] std::unique_ptr<Backend> make_mi355x_backend(int device = 0);

/// Registered variant ids (append-only; never renumbered).
inline constexpr std::uint32_t kGemvGgufRef = 1;   // == HALO_MI_GEMV_GGUF_REF
inline constexpr std::uint32_t kGemvSlab = 2;      // == HALO_MI_GEMV_SLAB
inline constexpr std::uint32_t kGemmSlabBf16 = 3;  // == HALO_MI_GEMM_SLAB_BF16
inline constexpr std::uint32_t kGemvSlabAuto = 4;  // == HALO_MI_GEMV_SLAB_AUTO
inline constexpr std::uint32_t kDequantRows = 5;
inline constexpr std::uint32_t kSwiglu = 6;
inline constexpr std::uint32_t kGateUpGemv = 7;
inline constexpr std::uint32_t kGateUpGemm = 8;
inline constexpr std::uint32_t kGemmSlabBf16M512 = 9;  // == HALO_MI_GEMM_SLAB_BF16_M512 (MATMUL)
inline constexpr std::uint32_t kGateUpGemmM512 = 10;   // GATE_UP_SWIGLU on the 512-row-tile GEMM
inline constexpr std::uint32_t kLmHeadFused = 11;      // LM_HEAD: argmax fused into the slab gemv
inline constexpr std::uint32_t kRmsNorm = 12;          // RMS_NORM in cpu::rms_norm's order (bitwise)

}  // namespace halo_mi::backend
