// Load-time upload of GGUF weights into SLAB images (halo_mi_upload_tensors, halo_mi_upload_slab):
// the device half of the reference's loader, Qwen35::Impl::make_mat / try_make_fused
// (src/models/qwen35.cpp:253-313) over Backend::import_host_readonly / upload.
//
// A three-stage pipeline over a ring of chunk slots, each a pinned host buffer and a device
// staging buffer of one chunk (whole slabs of one tensor):
//   host     the calling thread gathers the chunk's rows (from every part of a row-fused tensor,
//            at any row stride, typically an mmap'd GGUF) into the slot's pinned buffer, split
//            over host threads;
//   copy     the copy stream moves the pinned buffer to the slot's device buffer;
//   repack   `stream` repacks the device buffer into the chunk's slabs of the destination.
// Events chain the stages: the copy of a slot waits for that slot's previous repack, the repack
// for its copy, and the host refills a pinned buffer only after its copy has completed. So the
// host gather of chunk i + 2, the DMA of chunk i + 1 and the repack of chunk i overlap.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <mutex>
#include <thread>
#include <vector>

#include "launch.h"

namespace halo_mi {
namespace {

constexpr uint32_t kRingSlots = 4;

// The staging ring of a device, kept between calls (allocating pinned memory costs about a
// millisecond per 64 MiB, more than a mid-size tensor's upload) and grown on demand. It is
// never freed: the process holds at most kRingSlots chunks of pinned and device memory.
struct Ring {
    uint8_t* host[kRingSlots] = {};
    uint8_t* dev[kRingSlots] = {};
    hipEvent_t copied[kRingSlots] = {}, repacked[kRingSlots] = {};
    bool used[kRingSlots] = {};
    hipStream_t cs = nullptr;
    uint64_t cap = 0;    // bytes per slot
    uint32_t slots = 0;  // slots allocated

    // every copy and repack of the last call has completed
    void drain() {
        if (cs) (void)hipStreamSynchronize(cs);
        for (uint32_t s = 0; s < slots; ++s)
            if (used[s]) (void)hipEventSynchronize(repacked[s]);
        for (bool& u : used) u = false;
    }

    int ensure(uint64_t bytes, uint32_t want) {
        if (!cs && hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) {
            cs = nullptr;
            return set_error(HALO_MI_E_DEVICE, "upload: cannot create the copy stream");
        }
        if (bytes > cap) {  // too small: release every slot, then allocate at the new size
            for (uint32_t s = 0; s < slots; ++s) {
                (void)hipHostFree(host[s]);
                (void)hipFree(dev[s]);
                host[s] = dev[s] = nullptr;
            }
            slots = 0;
            cap = bytes;
        }
        for (; slots < want; ++slots) {
            const uint32_t s = slots;
            if (hipHostMalloc(reinterpret_cast<void**>(&host[s]), cap, hipHostMallocDefault) != hipSuccess) {
                host[s] = nullptr;
                return set_error(HALO_MI_E_MEMORY, "upload: cannot allocate %llu bytes of pinned staging",
                                 (unsigned long long)cap);
            }
            if (hipMalloc(reinterpret_cast<void**>(&dev[s]), cap) != hipSuccess) {
                (void)hipHostFree(host[s]);
                host[s] = dev[s] = nullptr;
                return set_error(HALO_MI_E_MEMORY, "upload: cannot allocate %llu bytes of device staging",
                                 (unsigned long long)cap);
            }
            if ((!copied[s] && hipEventCreateWithFlags(&copied[s], hipEventDisableTiming) != hipSuccess) ||
                (!repacked[s] && hipEventCreateWithFlags(&repacked[s], hipEventDisableTiming) != hipSuccess)) {
                (void)hipHostFree(host[s]);
                (void)hipFree(dev[s]);
                host[s] = dev[s] = nullptr;
                return set_error(HALO_MI_E_DEVICE, "upload: cannot create events");
            }
        }
        return HALO_MI_OK;
    }
};

std::mutex g_ring_mu;
std::map<int, Ring*> g_rings;

// Whether p is pinned (page-locked) host memory, which the copy engine reads directly.
bool is_pinned(const void* p) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // pageable memory: not an error of this library
        return false;
    }
    return attr.type == hipMemoryTypeHost;
}

// One contiguous byte range to copy into the pinned buffer.
struct Piece {
    const uint8_t* src;
    uint64_t dst_off, bytes;
};

// The pieces of rows [r0, r0 + n) of a row-fused tensor: dense parts give one piece per part,
// strided ones one per row.
void gather_pieces(const halo_mi_upload_tensor& t, uint64_t rb, uint64_t r0, uint64_t n, std::vector<Piece>& out) {
    out.clear();
    uint64_t base = 0, off = 0;
    for (uint32_t p = 0; p < t.n_parts && off < n * rb; ++p) {
        const halo_mi_upload_part& part = t.parts[p];
        const uint64_t lo = std::max(r0, base), hi = std::min(r0 + n, base + part.rows);
        if (lo < hi) {
            const uint64_t stride = part.src_stride ? part.src_stride : rb;
            const auto* src = static_cast<const uint8_t*>(part.src) + (lo - base) * stride;
            if (stride == rb) {
                out.push_back({src, off, (hi - lo) * rb});
                off += (hi - lo) * rb;
            } else {
                for (uint64_t r = lo; r < hi; ++r, src += stride, off += rb) out.push_back({src, off, rb});
            }
        }
        base += part.rows;
    }
}

// memcpy of the pieces into dst, split by bytes over `threads` threads.
void copy_pieces(const std::vector<Piece>& pieces, uint8_t* dst, uint32_t threads) {
    uint64_t total = 0;
    for (const Piece& p : pieces) total += p.bytes;
    const uint64_t min_share = 4ull << 20;  // below this a thread costs more than it copies
    const uint32_t t = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(threads, total / min_share));
    auto run = [&](uint64_t b0, uint64_t b1) {  // byte range [b0, b1) of the concatenated pieces
        uint64_t pos = 0;
        for (const Piece& p : pieces) {
            const uint64_t lo = std::max(b0, pos), hi = std::min(b1, pos + p.bytes);
            if (lo < hi) std::memcpy(dst + p.dst_off + (lo - pos), p.src + (lo - pos), hi - lo);
            pos += p.bytes;
            if (pos >= b1) break;
        }
    };
    if (t <= 1) {
        run(0, total);
        return;
    }
    std::vector<std::thread> pool;
    const uint64_t share = (total + t - 1) / t;
    for (uint32_t i = 0; i < t; ++i) {
        const uint64_t b0 = std::min(total, (uint64_t)i * share), b1 = std::min(total, b0 + share);
        if (b0 < b1) pool.emplace_back(run, b0, b1);
    }
    for (auto& th : pool) th.join();
}

}  // namespace
}  // namespace halo_mi

using namespace halo_mi;

extern "C" {

int halo_mi_upload_tensors(const halo_mi_upload_tensor* tensors, uint32_t n, uint64_t chunk_bytes, uint32_t host_threads,
                           void* stream) {
    clear_error();
    const char* op = "upload_tensors";
    if (n == 0) return HALO_MI_OK;
    if (!tensors) return set_error(HALO_MI_E_KERNEL, "%s: null tensor list", op);
    if (chunk_bytes == 0) chunk_bytes = 64ull << 20;
    if (host_threads == 0) host_threads = std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
    // validation, and the largest chunk (whole slabs of one tensor)
    uint64_t slot_bytes = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const halo_mi_upload_tensor& t = tensors[i];
        int code;
        const uint64_t rb = row_bytes_checked(t.type, t.cols, &code, op);
        if (code) return code;
        if (!is_quant(t.type)) return set_error(HALO_MI_E_UNSUPPORTED, "%s: tensor %u: type %u has no SLAB layout", op, i, t.type);
        if (t.n_parts == 0 || !t.parts) return set_error(HALO_MI_E_KERNEL, "%s: tensor %u has no parts", op, i);
        uint64_t rows = 0;
        for (uint32_t p = 0; p < t.n_parts; ++p) {
            const halo_mi_upload_part& part = t.parts[p];
            if (part.rows && !part.src) return set_error(HALO_MI_E_KERNEL, "%s: tensor %u part %u has no source", op, i, p);
            if (part.rows > 1 && part.src_stride && part.src_stride < rb)
                return set_error(HALO_MI_E_KERNEL, "%s: tensor %u part %u: row stride < row bytes", op, i, p);
            rows += part.rows;
        }
        if (rows > 0xFFFFFFFFull) return set_error(HALO_MI_E_UNSUPPORTED, "%s: tensor %u has more than 2^32 rows", op, i);
        if (rows && !t.dst) return set_error(HALO_MI_E_KERNEL, "%s: tensor %u has no destination", op, i);
        if (reinterpret_cast<uintptr_t>(t.dst) % 16) return set_error(HALO_MI_E_KERNEL, "%s: tensor %u: SLAB images must be 16-byte aligned", op, i);
        if (rows == 0) continue;
        uint64_t chunk_rows = std::max<uint64_t>(chunk_bytes / rb / kSlabRows, 1) * kSlabRows;
        chunk_rows = std::min<uint64_t>(chunk_rows, (rows + kSlabRows - 1) / kSlabRows * kSlabRows);
        slot_bytes = std::max(slot_bytes, chunk_rows * rb);
    }
    if (slot_bytes == 0) return HALO_MI_OK;
    for (uint32_t i = 0; i < n; ++i)
        for (uint32_t j = 0; j < i; ++j) {
            uint64_t ri = 0, rj = 0;
            for (uint32_t p = 0; p < tensors[i].n_parts; ++p) ri += tensors[i].parts[p].rows;
            for (uint32_t p = 0; p < tensors[j].n_parts; ++p) rj += tensors[j].parts[p].rows;
            if (ranges_overlap(tensors[i].dst, halo_mi_slab_bytes(tensors[i].type, (uint32_t)ri, tensors[i].cols), tensors[j].dst,
                               halo_mi_slab_bytes(tensors[j].type, (uint32_t)rj, tensors[j].cols)))
                return set_error(HALO_MI_E_KERNEL, "%s: the destinations of tensors %u and %u overlap", op, j, i);
        }
    auto st = static_cast<hipStream_t>(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(HALO_MI_E_DEVICE, "%s: hipGetDevice failed", op);
    uint64_t total_chunks = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const uint64_t rb = halo_mi_row_bytes(tensors[i].type, tensors[i].cols);
        uint64_t rows = 0;
        for (uint32_t p = 0; p < tensors[i].n_parts; ++p) rows += tensors[i].parts[p].rows;
        const uint64_t cr = std::max<uint64_t>(slot_bytes / rb / kSlabRows, 1) * kSlabRows;
        total_chunks += (rows + cr - 1) / cr;
    }
    std::lock_guard<std::mutex> lock(g_ring_mu);
    Ring*& rp = g_rings[dev];
    if (!rp) rp = new Ring();
    Ring& ring = *rp;
    if (int rc = ring.ensure(slot_bytes, (uint32_t)std::min<uint64_t>(kRingSlots, total_chunks))) return rc;
    const uint32_t nslots = ring.slots;
    struct Drain {  // on every return: nothing of this call is still using the ring
        Ring& r;
        ~Drain() { r.drain(); }
    } drain{ring};
    std::vector<Piece> pieces;
    uint64_t chunk = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const halo_mi_upload_tensor& t = tensors[i];
        const uint64_t rb = halo_mi_row_bytes(t.type, t.cols);
        uint64_t rows = 0;
        for (uint32_t p = 0; p < t.n_parts; ++p) rows += t.parts[p].rows;
        const uint64_t chunk_rows = std::min<uint64_t>(std::max<uint64_t>(slot_bytes / rb / kSlabRows, 1) * kSlabRows,
                                                       (rows + kSlabRows - 1) / kSlabRows * kSlabRows);
        const SlabGeom g = slab_geom(t.type, t.cols);
        // a dense part in pinned memory is read by the copy engine directly
        std::vector<uint8_t> direct(t.n_parts);
        for (uint32_t p = 0; p < t.n_parts; ++p)
            direct[p] = t.parts[p].rows && (t.parts[p].src_stride == 0 || t.parts[p].src_stride == rb) &&
                        is_pinned(t.parts[p].src);
        for (uint64_t r0 = 0; r0 < rows; r0 += chunk_rows, ++chunk) {
            const uint32_t s = (uint32_t)(chunk % nslots);
            const uint64_t nr = std::min<uint64_t>(chunk_rows, rows - r0);
            gather_pieces(t, rb, r0, nr, pieces);
            const uint8_t* from = ring.host[s];
            if (pieces.size() == 1 && pieces[0].bytes == nr * rb) {  // the chunk lies in one dense part
                uint64_t base = 0;
                uint32_t p = 0;
                while (base + t.parts[p].rows <= r0) base += t.parts[p++].rows;
                if (direct[p]) from = pieces[0].src;
            }
            if (from == ring.host[s]) {
                // host: the pinned buffer is free once its previous copy has completed
                if (ring.used[s] && hipEventSynchronize(ring.copied[s]) != hipSuccess)
                    return set_error(HALO_MI_E_DEVICE, "%s: copy failed", op);
                copy_pieces(pieces, ring.host[s], host_threads);
            }
            // copy: the device buffer is free once its previous repack has completed
            hipError_t e = hipSuccess;
            if (ring.used[s]) e = hipStreamWaitEvent(ring.cs, ring.repacked[s], 0);
            if (e == hipSuccess) e = hipMemcpyAsync(ring.dev[s], from, nr * rb, hipMemcpyHostToDevice, ring.cs);
            if (e == hipSuccess) e = hipEventRecord(ring.copied[s], ring.cs);
            // repack on `stream` once the copy is in
            if (e == hipSuccess) e = hipStreamWaitEvent(st, ring.copied[s], 0);
            if (e != hipSuccess) return hip_status(e, "upload_tensors copy");
            if (int rc = launch_repack_slab(t.type, ring.dev[s], rb, (uint32_t)nr, t.cols,
                                            static_cast<uint8_t*>(t.dst) + (r0 / kSlabRows) * g.slab_bytes, st))
                return rc;
            if ((e = hipEventRecord(ring.repacked[s], st)) != hipSuccess) return hip_status(e, "upload_tensors repack");
            ring.used[s] = true;
        }
    }
    const hipError_t e = hipStreamSynchronize(st);
    return e == hipSuccess ? HALO_MI_OK : hip_status(e, "upload_tensors sync");
}

int halo_mi_upload_slab(uint32_t type, const void* host_src, uint64_t src_stride, uint32_t rows, uint32_t cols, void* dst,
                        uint64_t chunk_bytes, void* stream) {
    const halo_mi_upload_part part{host_src, src_stride, rows};
    const halo_mi_upload_tensor t{type, cols, &part, 1, dst};
    return halo_mi_upload_tensors(&t, 1, chunk_bytes, 0, stream);
}

}  // extern "C"
