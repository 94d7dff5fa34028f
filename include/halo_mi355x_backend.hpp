// halo_mi355x C++ backend: the host-side mirror of the reference's ADR-001 Backend interface
// (include/halo/backend/backend.h of the reference) for the quantized matrix-multiply path,
// built on the C ABI of halo_mi355x.h.
//
// `Backend`, `Stream`, `Buffer`, `TensorRef` and every args struct have the reference's members,
// types and virtual layout (backend.h:104-584), so a forward written against the reference's
// interface compiles against this one by namespace. The ops of the path (get_rows, rms_norm,
// gemv, swiglu, lm_head, argmax, copy) run on the GPU; the other op virtuals throw
// Error(Unsupported), as the reference allows for a backend of this scope.
//
// Contract kept from the reference:
//  - every op validates all operands on the host and throws before anything is enqueued
//    (backend.h:5-9); work then runs in stream order; results are read after Stream::wait();
//  - error mapping (backend.h:24-26): shape / alias / range / alignment -> Error(Kernel);
//    dtype or limit -> Error(Unsupported); unknown variant id -> Error(Config); allocation ->
//    Error(Memory); a device fault at wait() -> Error(Kernel) and a poisoned backend, device
//    loss -> Error(Device) and a sticky lost() (ADR-001:402-414); a GET_ROWS id outside the
//    table -> Error(Kernel) at wait() (the reference HIP backend's status word,
//    backends/hip/src/ops.cpp:982-1012; the CPU backend throws it synchronously);
//  - aliasing (backend.h:15-19): an output may not overlap any operand;
//  - kernel selection by an explicit, append-only variant id (KernelChoice, 0 = default);
//  - one thread drives a Backend and its Streams.
//
// Additions (no counterpart in the reference) live in the derived classes MiBuffer, MiStream and
// MiBackend, never in the reference's classes: weights imported straight into the SLAB device
// layout (MiBackend::import_weights), GET_ROWS over a contiguous row range
// (MiBackend::dequant_rows), the FFN's gate/up/SwiGLU composition (src/models/qwen35.cpp:789-805)
// as one op (MiBackend::gate_up_swiglu), device addresses and layouts of buffers, and the
// hipStream_t of a stream.
#pragma once

#include <cstddef>
#include <cstdint>
#include <limits>
#include <memory>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

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

// ---- element types (include/halo/tensor/dtype.h:18-49: ggml's ids) -----------------------

enum class DType : std::uint32_t {
    F32 = 0, F16 = 1, Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q8_1 = 9, Q2_K = 10, Q3_K = 11, Q4_K = 12,
    Q5_K = 13, Q6_K = 14, Q8_K = 15, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19, IQ4_NL = 20, IQ3_S = 21,
    IQ2_S = 22, IQ4_XS = 23, I8 = 24, I16 = 25, I32 = 26, I64 = 27, F64 = 28, IQ1_M = 29, BF16 = 30,
};

// ---- types (backend.h:60-247) ---------------------------------------------------------------

class Backend;

enum class Kind : std::uint8_t { Cpu, Hip, HipEmulation, Vulkan };
enum class Tier : std::uint8_t { Vram, Gtt, Host };

[[nodiscard]] std::string_view to_string(Kind k) noexcept;

/// Element format of a KV pool image (backend.h:68-75).
enum class KvType : std::uint8_t { F32, F16, Q8 };

/// Memory owned (or imported) by one Backend (backend.h:105-124).
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

protected:
    Buffer() = default;
    Buffer(const Buffer&) = default;
    Buffer& operator=(const Buffer&) = default;
};

/// An operand: bytes [offset, offset + bytes) of `buffer` (bytes 0 = to the end of the buffer);
/// row_stride = bytes between consecutive rows (0 = dense) (backend.h:128-155).
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
    /// The same buffer from offset + delta on; a bounded view shrinks by delta. Error(Kernel)
    /// when delta reaches past a bounded view's end, or on offset overflow.
    [[nodiscard]] TensorRef shifted(std::uint64_t delta) const;
    [[nodiscard]] TensorRef with_stride(std::uint64_t s) const noexcept { return {buffer, offset, bytes, s}; }
};

/// Status bits a device op sets when it detects a data error (backend.h:157-161).
inline constexpr std::uint32_t kStatusPositiveG = 1u;
inline constexpr std::uint32_t kStatusNaN = 2u;
inline constexpr std::uint32_t kStatusBadBlock = 4u;
inline constexpr std::uint32_t kStatusBadIndex = 8u;
inline constexpr std::uint32_t kBatchWide = std::numeric_limits<std::uint32_t>::max();
inline constexpr std::uint32_t kNoStatus = std::numeric_limits<std::uint32_t>::max();

/// One word of the step's status array and the sequence that owns it (backend.h:164-171);
/// must be empty, as on every reference backend (WS-BI-1).
struct StatusRef {
    std::uint32_t word = kNoStatus;
    std::uint32_t owner = kBatchWide;
    [[nodiscard]] bool empty() const noexcept { return word == kNoStatus; }
};

struct KernelChoice {
    std::uint32_t variant_id = 0;
};

/// Operator ids: the reference's values (backend.h:187-206), plus this backend's fused FFN op
/// (appended; the reference's kOpCount ops keep their values).
enum class OpId : std::uint16_t {
    GetRows = 0, RmsNorm = 1, AddRmsNorm = 2, Gemv = 3, GdnGates = 4, Conv1dSilu = 5, GatedDeltaRule = 6,
    GatedRmsNorm = 7, PartialRope = 8, KvWrite = 9, Attention = 10, Swiglu = 11, MulSigmoid = 12, Add = 13,
    LmHead = 14, Argmax = 15, TopK = 16, Copy = 17,
    GateUpSwiglu = 18,  // addition: gemv(gate) + gemv(up) + swiglu in one launch (MiBackend::gate_up_swiglu)
};
inline constexpr std::size_t kOpCount = 18;  // the reference's ops

[[nodiscard]] std::string_view op_name(OpId op) noexcept;

struct VariantInfo {
    std::uint32_t id = 0;
    std::string_view name;
    OpId op = OpId::GetRows;
    std::string_view form;
};

/// Operand limits of a backend (backend.h:219-247).
struct Limits {
    std::uint32_t max_gdn_dk = 0;
    std::uint32_t max_gdn_chunk = 0;
    std::uint32_t max_head_dim = 0;
    std::uint32_t max_conv_k = 0;
    std::uint32_t max_top_k = 0;
    std::uint32_t max_rope_dims = 0;
    bool gdn_chunked = false;
    std::uint64_t max_import_bytes = 0;
    std::uint64_t max_pool_buffer_bytes = 0;
    bool lm_head_ids = false;
    /// Largest cols of a gemv with GemvArgs::norm_w whose result is bit for bit rms_norm then
    /// this backend's own unfused gemv (backend.h:236-242).
    std::uint32_t max_fused_norm_cols = 0;
    bool gemv_gdn_gates = false;
};

// ---- args structs (backend.h:249-476) -------------------------------------------------------

/// GET_ROWS: out[i] = dequant(table row ids[i]), bit-identical to tensor::dequantize_row. An id
/// outside [0, n_rows) leaves its row unwritten and fails the stream's next wait() with
/// Error(Kernel).
struct GetRowsArgs {
    DType type = DType::F32;
    TensorRef table{}, ids{}, out{};
    std::uint32_t n_rows = 0, cols = 0, n_ids = 0;
    KernelChoice kernel{};
    StatusRef status{};
};

/// RMS_NORM (cpu::rms_norm): rows x cols; w: [cols]. out may be x itself (same stride), else
/// must not overlap x. Bitwise equal to the CPU.
struct RmsNormArgs {
    TensorRef x{}, w{}, out{};
    std::uint32_t rows = 0, cols = 0;
    float eps = 1e-6f;
    KernelChoice kernel{};
};

struct AddRmsNormArgs {
    TensorRef a{}, b{}, h{}, w{}, out{};
    std::uint32_t rows = 0, cols = 0;
    float eps = 1e-6f;
    KernelChoice kernel{};
};

/// MATMUL / QUANT_GEMV: y[t][n] = sum_i x[t][i] W[n][i].
struct GemvArgs {
    DType wtype = DType::F32;
    TensorRef w{}, x{}, y{};
    std::uint32_t rows = 0, cols = 0, n_vec = 1;
    KernelChoice kernel{};
    /// Fused input norm: y = W (rms_norm(x) * norm_w) with eps = norm_eps, x the raw rows;
    /// norm_w: [cols] fp32. Every variant and n_vec here; bitwise rms_norm then the same gemv.
    TensorRef norm_w{};
    float norm_eps = 1e-6f;
    /// Off (the default), every row of y is bitwise the row an n_vec == 1 call gives, whatever
    /// n_vec. On, the SLAB default may run the bf16 MFMA GEMM for n_vec > 8.
    bool allow_gemm = false;
    struct Gates {
        TensorRef dt_bias{}, a{};
        std::uint32_t n_v = 0;
    } gates{};
};

struct GdnGateArgs {
    TensorRef alpha{}, beta{}, dt_bias{}, a{}, g_out{}, beta_out{};
    std::uint32_t n_tokens = 0, n_heads = 0;
    KernelChoice kernel{};
};

struct StateRing {
    std::uint32_t p = 0;
    std::uint32_t live = 0;
};

struct Conv1dArgs {
    TensorRef x{}, weight{}, conv_state{}, out{}, state_slots{};
    std::uint32_t n_tokens = 0, channels = 0, kernel_size = 4, n_slots = 0;
    std::optional<StateRing> ring{};
    KernelChoice kernel{};
};

enum class GdnForm : std::uint8_t { Recurrent, Chunked };
enum class GdnHeadMapping : std::uint8_t { Tiled, Grouped };

struct GdnArgs {
    GdnForm form = GdnForm::Recurrent;
    TensorRef q{}, k{}, v{}, g{}, beta{}, state{}, state_slots{}, out{};
    std::uint32_t n_k = 0, n_v = 0, d_k = 0, d_v = 0, n_tokens = 0, n_slots = 0;
    GdnHeadMapping mapping = GdnHeadMapping::Tiled;
    bool qk_l2norm = true;
    std::optional<float> q_scale{};
    std::uint32_t chunk_size = 64;
    std::optional<StateRing> ring{};
    KernelChoice kernel{};
    StatusRef status{};
};

struct GatedNormArgs {
    TensorRef x{}, z{}, w{}, out{};
    std::uint32_t rows = 0, cols = 0;
    float eps = 1e-6f;
    KernelChoice kernel{};
};

struct RopeArgs {
    TensorRef x{}, positions{};
    std::uint32_t n_tokens = 0, n_heads = 0, head_dim = 0, rot_dims = 0;
    float theta = 10000.0f;
    std::uint32_t head_stride = 0;
    KernelChoice kernel{};
};

struct KvWriteArgs {
    TensorRef kv_pool{}, block_table{}, k{}, v{};
    std::uint32_t n_pool_blocks = 0, n_layers = 1, layer = 0, block_tokens = 16, kv_dim = 0;
    std::uint32_t n_block_table = 0;
    std::uint32_t start = 0, n_tokens = 1;
    KernelChoice kernel{};
    StatusRef status{};
    KvType kv_type = KvType::F32;
};

struct AttentionArgs {
    TensorRef q{}, kv_pool{}, block_table{}, out{};
    std::uint32_t q_head_stride = 0;
    std::uint32_t n_pool_blocks = 0, n_layers = 1, layer = 0, block_tokens = 16;
    std::uint32_t n_block_table = 0;
    std::uint32_t n_head = 0, n_kv_head = 0, head_dim = 0, n_tokens = 1, q_offset = 0;
    float scale = 1.0f;
    KernelChoice kernel{};
    StatusRef status{};
    KvType kv_type = KvType::F32;
    TensorRef tree_parent{};
};

/// SWIGLU out = silu(a) * b; MUL_SIGMOID out = a * sigmoid(b); ADD out = a + b.
struct EltwiseArgs {
    TensorRef a{}, b{}, out{};
    std::uint32_t rows = 0, cols = 0;
    KernelChoice kernel{};
};

/// ARGMAX result words of one vector: {index u32, value (f32 bits), nan (0/1)} (backend.h:430-431).
inline constexpr std::uint32_t kArgmaxResultBytes = 12;

/// LM_HEAD: the gemv over the vocabulary + fused argmax (ties to the lowest index; a NaN logit
/// poisons its own vector; rows at or past valid_rows, when not 0, are not ranked). gemv.y is
/// optional (the full logits). A slot past ids_scatter's end is dropped (the reference's Vulkan
/// behaviour, backend.h:453-457).
struct LmHeadArgs {
    GemvArgs gemv{};
    TensorRef result{};
    std::uint32_t valid_rows = 0;
    KernelChoice kernel{};
    StatusRef status{};
    TensorRef ids{};
    TensorRef ids_slots{};
    TensorRef ids_scatter{};
};

/// ARGMAX (cpu::argmax per vector): logits n_vec rows of [n]; result as LmHeadArgs.
struct ArgmaxArgs {
    TensorRef logits{}, result{};
    std::uint32_t n = 0, n_vec = 1;
    KernelChoice kernel{};
    StatusRef status{};
};

struct TopKArgs {
    TensorRef logits{}, ids{}, values{};
    std::uint32_t n = 0, k = 0, n_vec = 1;
    KernelChoice kernel{};
    StatusRef status{};
};

/// COPY: `bytes` bytes from src to dst (dense). Must not overlap.
struct CopyArgs {
    TensorRef src{}, dst{};
    std::uint64_t bytes = 0;
    KernelChoice kernel{};
};

/// A type-erased op call (backend.h:470-476).
struct OpInvocation {
    OpId op = OpId::Copy;
    std::variant<GetRowsArgs, RmsNormArgs, AddRmsNormArgs, GemvArgs, GdnGateArgs, Conv1dArgs, GdnArgs, GatedNormArgs,
                 RopeArgs, KvWriteArgs, AttentionArgs, EltwiseArgs, LmHeadArgs, ArgmaxArgs, TopKArgs, CopyArgs>
        args;
};

/// Ordered work queue (backend.h:495-506).
class Stream {
public:
    virtual ~Stream() = default;
    virtual void submit() = 0;
    virtual void wait() = 0;  ///< throws the translated device error
    virtual void abort() noexcept = 0;

protected:
    Stream() = default;
    Stream(const Stream&) = default;
    Stream& operator=(const Stream&) = default;
};

/// The reference's Backend (backend.h:508-584), virtual for virtual.
class Backend {
public:
    virtual ~Backend() = default;
    Backend(const Backend&) = delete;
    Backend& operator=(const Backend&) = delete;

    [[nodiscard]] virtual Kind kind() const noexcept = 0;
    [[nodiscard]] virtual std::string describe() const = 0;
    [[nodiscard]] virtual Limits limits() const noexcept = 0;
    [[nodiscard]] virtual bool lost() const noexcept { return false; }

    // ---- memory ----------------------------------------------------------------------
    [[nodiscard]] virtual std::unique_ptr<Buffer> allocate(std::uint64_t bytes, Tier tier) = 0;
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_host(std::span<std::byte> bytes) = 0;
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_host_writeonly(std::span<std::byte> bytes,
                                                                        std::uint64_t writeback_bytes) {
        (void)writeback_bytes;
        return import_host(bytes);
    }
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_host_readonly(std::span<const std::byte> bytes) = 0;
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_step_readonly(std::span<const std::byte> bytes) {
        return import_host_readonly(bytes);
    }
    [[nodiscard]] virtual std::unique_ptr<Stream> create_stream() = 0;
    virtual void upload(Stream& s, TensorRef dst, std::span<const std::byte> src) = 0;
    virtual void download(Stream& s, TensorRef src, std::span<std::byte> dst) = 0;

    // ---- registry --------------------------------------------------------------------
    [[nodiscard]] virtual std::span<const VariantInfo> variants(OpId op, std::string_view form = {}) const = 0;

    // ---- ops: validate on the host (throw before enqueuing), then enqueue --------------
    virtual void get_rows(Stream&, const GetRowsArgs&) = 0;
    virtual void rms_norm(Stream&, const RmsNormArgs&) = 0;
    virtual void add_rms_norm(Stream&, const AddRmsNormArgs&) = 0;
    virtual void gemv(Stream&, const GemvArgs&) = 0;
    virtual void gdn_gates(Stream&, const GdnGateArgs&) = 0;
    virtual void conv1d_silu(Stream&, const Conv1dArgs&) = 0;
    virtual void gated_delta_rule(Stream&, const GdnArgs&) = 0;
    virtual void gated_rms_norm(Stream&, const GatedNormArgs&) = 0;
    virtual void partial_rope(Stream&, const RopeArgs&) = 0;
    virtual void kv_write(Stream&, const KvWriteArgs&) = 0;
    virtual void attention(Stream&, const AttentionArgs&) = 0;
    virtual void swiglu(Stream&, const EltwiseArgs&) = 0;
    virtual void mul_sigmoid(Stream&, const EltwiseArgs&) = 0;
    virtual void add(Stream&, const EltwiseArgs&) = 0;
    virtual void lm_head(Stream&, const LmHeadArgs&) = 0;
    virtual void argmax(Stream&, const ArgmaxArgs&) = 0;
    virtual void top_k(Stream&, const TopKArgs&) = 0;
    virtual void copy(Stream&, const CopyArgs&) = 0;

    /// Dispatches to the typed method. Error(Api) if `inv.args` does not hold the args type of
    /// `inv.op` (backend.h:578-580).
    void run_op(Stream& s, const OpInvocation& inv);

protected:
    Backend() = default;
};

/// Decodes argmax result words (n_vec * 3 u32). Error(Kernel) naming the vector if its NaN word
/// is set (backend.h:590-595).
struct ArgmaxResult {
    std::int32_t index = -1;
    float value = 0.0f;
};
[[nodiscard]] std::vector<ArgmaxResult> decode_argmax(std::span<const std::byte> words);

// ---- this backend's additions ---------------------------------------------------------------

/// How the bytes of a weight buffer are laid out.
enum class WeightLayout : std::uint8_t { Gguf, Slab };

/// A buffer of the MI355X backend: its device address and the layout of its weights.
class MiBuffer : public Buffer {
public:
    [[nodiscard]] virtual void* device_ptr() const noexcept = 0;
    [[nodiscard]] virtual WeightLayout layout() const noexcept = 0;
};

/// A stream of the MI355X backend: its hipStream_t.
class MiStream : public Stream {
public:
    [[nodiscard]] virtual void* native() const noexcept = 0;
};

/// GET_ROWS restricted to a contiguous row range: out rows = dequantized W rows
/// [first_row, first_row + n_rows), bit-identical to tensor::dequantize_row.
struct DequantRowsArgs {
    DType type = DType::F32;
    TensorRef table{}, out{};
    std::uint32_t n_rows_table = 0, cols = 0, first_row = 0, n_rows = 0;
    KernelChoice kernel{};
};

/// out[t][n] = silu((Wg x_t)[n]) * (Wu x_t)[n]; Wg, Wu SLAB weights of one shape.
struct GateUpArgs {
    DType wtype = DType::Q4_K;
    TensorRef w_gate{}, w_up{}, x{}, out{};
    std::uint32_t rows = 0, cols = 0, n_vec = 1;
    KernelChoice kernel{};
    bool allow_gemm = false;  ///< same meaning as GemvArgs::allow_gemm
    TensorRef norm_w{};       ///< fused input norm, as GemvArgs::norm_w
    float norm_eps = 1e-6f;
};

/// The MI355X backend's own interface on top of the reference's.
class MiBackend : public Backend {
public:
    /// Read-only import of a rows x cols GGUF weight matrix (rows `row_stride` bytes apart, 0 =
    /// dense) into the SLAB layout, repacked on the device chunk by chunk.
    [[nodiscard]] virtual std::unique_ptr<Buffer> import_weights(std::span<const std::byte> gguf, DType type,
                                                                 std::uint32_t rows, std::uint32_t cols,
                                                                 std::uint64_t row_stride = 0) = 0;
    virtual void dequant_rows(Stream&, const DequantRowsArgs&) = 0;
    virtual void gate_up_swiglu(Stream&, const GateUpArgs&) = 0;
};

/// The kernel family a MATMUL or GATE_UP_SWIGLU call with `allow_gemm == false` and kernel
/// variant 0 runs on SLAB weights (GemvArgs::allow_gemm, backend.h:298-304: every row bitwise the
/// row of an n_vec == 1 call). Both families keep that for any n_vec; the choice is per backend,
/// so a decode at one vector and an MTP verify at K vectors always take the same one.
enum class BatchInvariantKernel : std::uint8_t {
    Gemv,   ///< the slab GEMV: fastest at 1-2 vectors, four vectors per pass over the weights
    Exact,  ///< the exact small-M GEMM with its K split fixed by the shape (HALO_MI_GEMM_SLAB_EXACT_INVARIANT):
            ///< fastest from 3 vectors, eight per pass; the slab GEMV where the split does not fit
};

struct MiOptions {
    BatchInvariantKernel batch_invariant = BatchInvariantKernel::Gemv;
};

/// The MI355X backend on HIP device `device` (default 0). Error(Device) without a GPU.
[[nodiscard]] std::unique_ptr<MiBackend> make_mi355x_backend(int device = 0, MiOptions options = {});

/// Registered variant ids (explicit and append-only; never renumbered, a retired id is never
/// reused). They start after the reference HIP backend's last id (29, copy_async;
/// src/backend/hip_adapter.cpp:68-96), so one registry can hold both.
inline constexpr std::uint32_t kGemvGgufRef = 30;       // C ABI HALO_MI_GEMV_GGUF_REF
inline constexpr std::uint32_t kGemvSlab = 31;          // HALO_MI_GEMV_SLAB
inline constexpr std::uint32_t kGemmSlabBf16 = 32;      // HALO_MI_GEMM_SLAB_BF16
inline constexpr std::uint32_t kGemvSlabAuto = 33;      // HALO_MI_GEMV_SLAB_AUTO
inline constexpr std::uint32_t kGemmSlabBf16M512 = 34;  // HALO_MI_GEMM_SLAB_BF16_M512
inline constexpr std::uint32_t kGemvSlabValu = 35;      // HALO_MI_GEMV_SLAB_VALU
inline constexpr std::uint32_t kGemmSlabBf16SmallM = 36;  // HALO_MI_GEMM_SLAB_BF16_SMALL_M
inline constexpr std::uint32_t kDequantRows = 37;       // GET_ROWS
inline constexpr std::uint32_t kRmsNorm = 38;           // RMS_NORM in cpu::rms_norm's order (bitwise)
inline constexpr std::uint32_t kSwiglu = 39;            // SWIGLU
inline constexpr std::uint32_t kLmHeadFused = 40;       // LM_HEAD: the argmax stage 2 (stage 1: the gemv variant)
inline constexpr std::uint32_t kArgmax = 41;            // ARGMAX: 64-row parts, then the same stage 2
inline constexpr std::uint32_t kCopy = 42;              // COPY: hipMemcpyAsync
inline constexpr std::uint32_t kGateUpGemv = 43;        // GATE_UP_SWIGLU on the GEMV pair
inline constexpr std::uint32_t kGateUpGemm = 44;        // ... on the 64..256-row-tile GEMM
inline constexpr std::uint32_t kGateUpGemmM512 = 45;    // ... on the 512-row-tile GEMM
inline constexpr std::uint32_t kGateUpGemmSmallM = 46;  // ... on the small-M GEMM
inline constexpr std::uint32_t kGemmSlabExactSmallM = 47;  // HALO_MI_GEMM_SLAB_EXACT_SMALL_M
inline constexpr std::uint32_t kGateUpExactSmallM = 48;    // GATE_UP_SWIGLU on the exact small-M GEMM
inline constexpr std::uint32_t kGemmSlabExactInvariant = 49;  // HALO_MI_GEMM_SLAB_EXACT_INVARIANT
inline constexpr std::uint32_t kGateUpExactInvariant = 50;    // GATE_UP_SWIGLU on it

}  // namespace halo_mi::backend
