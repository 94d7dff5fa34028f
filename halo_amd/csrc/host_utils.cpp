// Host side of the halo_mi355x library: error reporting, geometry, the host SLAB repack,
// and the synthetic-input generators (normal fill + GGUF quantizers).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "common.h"
#include "slab_layout.h"

namespace halo_mi {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

uint64_t row_bytes_checked(uint32_t type, uint32_t cols, int* code, const char* op) {
    const uint32_t be = block_elems(type);
    if (be == 0) {
        *code = set_error(HALO_MI_E_UNSUPPORTED, "%s: weight type %u is not supported", op, type);
        return 0;
    }
    if (cols % be != 0) {
        *code = set_error(HALO_MI_E_KERNEL, "%s: %u elements is not a multiple of the block size %u", op, cols, be);
        return 0;
    }
    *code = HALO_MI_OK;
    return (uint64_t)(cols / be) * block_bytes(type);
}

namespace {

// ---- threads ------------------------------------------------------------------------------

template <class Fn>
void parallel_rows(uint64_t n, uint32_t threads, Fn&& fn) {
    uint32_t t = threads ? threads : std::max(1u, std::thread::hardware_concurrency());
    if (t > n) t = static_cast<uint32_t>(std::max<uint64_t>(n, 1));
    if (t <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> pool;
    const uint64_t base = n / t, extra = n % t;
    uint64_t begin = 0;
    for (uint32_t i = 0; i < t; ++i) {
        const uint64_t len = base + (i < extra ? 1 : 0);
        pool.emplace_back([&fn, begin, len] { fn(begin, begin + len); });
        begin += len;
    }
    for (auto& th : pool) th.join();
}

// ---- fp32 -> fp16, round to nearest even ---------------------------------------------------

uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return static_cast<uint16_t>(sign | 0x7E00u);  // NaN
    if (ax >= 0x477FF000u) return static_cast<uint16_t>(sign | 0x7C00u);  // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {                                               // fp16 subnormal range or zero
        // value = ax_float; fp16 subnormal unit is 2^-24: round(value * 2^24) to nearest even.
        float v;
        std::memcpy(&v, &ax, 4);
        const float scaled = v * 16777216.0f;  // exact (power of two)
        const float r = std::nearbyint(scaled);  // default rounding mode: nearest even
        return static_cast<uint16_t>(sign | static_cast<uint32_t>(r));
    }
    // normal: rebias exponent, round mantissa 23 -> 10 bits to nearest even
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t exp = (ax >> 23) - 112u;
    uint32_t h = (exp << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1FFFu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;  // carry into exponent is correct
    return static_cast<uint16_t>(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) bits = sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u);
    else if (e) bits = sign | ((e + 112u) << 23) | (m << 13);
    else if (!m) bits = sign;
    else {
        const float v = (float)m * 0x1p-24f;
        std::memcpy(&bits, &v, 4);
        bits |= sign;
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = static_cast<uint8_t>(v & 0xFF);
    p[1] = static_cast<uint8_t>(v >> 8);
}

int nearest(float v) { return static_cast<int>(std::lrint(v)); }

// ---- quantizers (fp32 -> GGUF block); the reference ships none -----------------------------

// Q8_0: d = max|x| / 127, q = round(x / d).
void quant_q8_0(const float* x, uint8_t* blk) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(x[i]));
    const float d = amax / 127.0f;
    const uint16_t dh = f32_to_f16(d);
    const float dq = f16_to_f32(dh);
    put16(blk, dh);
    for (int i = 0; i < 32; ++i) {
        int q = dq > 0.0f ? nearest(x[i] / dq) : 0;
        q = std::clamp(q, -128, 127);
        blk[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(q));
    }
}

// Q4_0: the element of largest magnitude maps to q = 0 (value -8 d); q = round(x / d) + 8.
void quant_q4_0(const float* x, uint8_t* blk) {
    float vmax = 0.0f;
    for (int i = 0; i < 32; ++i)
        if (std::fabs(x[i]) > std::fabs(vmax)) vmax = x[i];
    const float d = vmax / -8.0f;
    const uint16_t dh = f32_to_f16(d);
    const float dq = f16_to_f32(dh);
    put16(blk, dh);
    uint8_t q[32];
    for (int i = 0; i < 32; ++i) q[i] = static_cast<uint8_t>(dq != 0.0f ? std::clamp(nearest(x[i] / dq) + 8, 0, 15) : 8);
    for (int i = 0; i < 16; ++i) blk[2 + i] = static_cast<uint8_t>(q[i] | (q[i + 16] << 4));
}

// Q4_K (QMAX 15) and Q5_K (QMAX 31): per 32-weight sub-block an affine fit w ~ s * q - m
// (q in 0..QMAX, m >= 0); the eight scales and eight mins are then quantized to 6 bits against
// fp16 d and dmin (the 12-byte scales field both formats share).
template <int QMAX>
void quant_k_affine(const float* x, uint8_t* blk) {
    float scale[8], minv[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) {
            lo = std::min(lo, x[32 * j + i]);
            hi = std::max(hi, x[32 * j + i]);
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[j] = (hi - lo) / (float)QMAX;
        minv[j] = -lo;
    }
    float smax = 0.0f, mmax = 0.0f;
    for (int j = 0; j < 8; ++j) {
        smax = std::max(smax, scale[j]);
        mmax = std::max(mmax, minv[j]);
    }
    const uint16_t dh = f32_to_f16(smax / 63.0f), mh = f32_to_f16(mmax / 63.0f);
    const float d = f16_to_f32(dh), dmin = f16_to_f32(mh);
    int sc[8], mq[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = d > 0.0f ? std::clamp(nearest(scale[j] / d), 0, 63) : 0;
        mq[j] = dmin > 0.0f ? std::clamp(nearest(minv[j] / dmin), 0, 63) : 0;
    }
    put16(blk, dh);
    put16(blk + 2, mh);
    uint8_t* s = blk + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = static_cast<uint8_t>((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
        s[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
        const float d1 = d * (float)sc[j], m1 = dmin * (float)mq[j];
        for (int i = 0; i < 32; ++i) {
            const int v = d1 > 0.0f ? nearest((x[32 * j + i] + m1) / d1) : 0;
            q[32 * j + i] = static_cast<uint8_t>(std::clamp(v, 0, QMAX));
        }
    }
    // group g of 32 bytes: low nibbles = sub-block 2g, high nibbles = sub-block 2g + 1; Q5_K
    // keeps the fifth bit of element l of sub-block j in bit j of qh[l] (bytes 16..47)
    uint8_t* qs = blk + (QMAX == 15 ? 16 : 48);
    for (int g = 0; g < 4; ++g)
        for (int l = 0; l < 32; ++l)
            qs[32 * g + l] = static_cast<uint8_t>((q[64 * g + l] & 15) | ((q[64 * g + 32 + l] & 15) << 4));
    if constexpr (QMAX == 31) {
        for (int l = 0; l < 32; ++l) {
            uint8_t h = 0;
            for (int j = 0; j < 8; ++j) h = static_cast<uint8_t>(h | ((q[32 * j + l] >> 4) << j));
            blk[16 + l] = h;
        }
    }
}

// The IQ4_NL code table of the GGUF format (ggml's kvalues_iq4nl).
constexpr int kIq4Values[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

// IQ4_XS: per 32-weight sub-block a scale s that maps the element of largest magnitude to the
// table's end -127; the eight scales are quantized to 6 bits (ls - 32 in -32..31) against
// fp16 d = -(the largest-magnitude scale) / 32; each weight takes the nearest table value.
void quant_iq4_xs(const float* x, uint8_t* blk) {
    float sv[8], smax = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float vmax = 0.0f;
        for (int i = 0; i < 32; ++i)
            if (std::fabs(x[32 * j + i]) > std::fabs(vmax)) vmax = x[32 * j + i];
        sv[j] = vmax / -127.0f;
        if (std::fabs(sv[j]) > std::fabs(smax)) smax = sv[j];
    }
    const uint16_t dh = f32_to_f16(smax / -32.0f);
    const float d = f16_to_f32(dh);
    put16(blk, dh);
    uint16_t sh = 0;
    for (int i = 0; i < 4; ++i) blk[4 + i] = 0;
    for (int j = 0; j < 8; ++j) {
        const int l = d != 0.0f ? std::clamp(nearest(sv[j] / d), -32, 31) : 0;
        const int ls = l + 32;
        blk[4 + j / 2] = static_cast<uint8_t>(blk[4 + j / 2] | ((ls & 15) << (4 * (j % 2))));
        sh = static_cast<uint16_t>(sh | ((ls >> 4) << (2 * j)));
        const float dl = d * (float)l;
        uint8_t q[32];
        for (int i = 0; i < 32; ++i) {
            int best = 8;
            if (dl != 0.0f) {
                const float t = x[32 * j + i] / dl;
                float err = std::fabs(t - (float)kIq4Values[0]);
                best = 0;
                for (int k = 1; k < 16; ++k) {
                    const float e = std::fabs(t - (float)kIq4Values[k]);
                    if (e < err) {
                        err = e;
                        best = k;
                    }
                }
            }
            q[i] = static_cast<uint8_t>(best);
        }
        for (int i = 0; i < 16; ++i) blk[8 + 16 * j + i] = static_cast<uint8_t>(q[i] | (q[i + 16] << 4));
    }
    put16(blk + 2, sh);
}

// Q6_K: per 16-weight sub-block a symmetric scale s = max|x| / 31 (q in -32..31); the sixteen
// scales are quantized to int8 against fp16 d = max|s| / 127.
void quant_q6_k(const float* x, uint8_t* blk) {
    float scale[16];
    float smax = 0.0f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(x[16 * j + i]));
        scale[j] = amax / 31.0f;
        smax = std::max(smax, scale[j]);
    }
    const uint16_t dh = f32_to_f16(smax / 127.0f);
    const float d = f16_to_f32(dh);
    int sc[16];
    for (int j = 0; j < 16; ++j) sc[j] = d > 0.0f ? std::clamp(nearest(scale[j] / d), -128, 127) : 0;
    uint8_t q[256];
    for (int j = 0; j < 16; ++j) {
        const float ds = d * (float)sc[j];
        for (int i = 0; i < 16; ++i) {
            const int v = ds != 0.0f ? nearest(x[16 * j + i] / ds) : 0;
            q[16 * j + i] = static_cast<uint8_t>(std::clamp(v, -32, 31) + 32);
        }
    }
    std::memset(blk, 0, 210);
    // element e: half n, quarter k, lane l (the layout dequantized by quant.cpp:302-327)
    for (int e = 0; e < 256; ++e) {
        const int n = e / 128, r = e % 128, k = r / 32, l = r % 32;
        const int lo4 = q[e] & 15, hi2 = q[e] >> 4;
        blk[64 * n + l + 32 * (k & 1)] |= static_cast<uint8_t>(k >= 2 ? (lo4 << 4) : lo4);
        blk[128 + 32 * n + l] |= static_cast<uint8_t>(hi2 << (2 * k));
    }
    for (int j = 0; j < 16; ++j) blk[192 + j] = static_cast<uint8_t>(static_cast<int8_t>(sc[j]));
    put16(blk + 208, dh);
}

// ---- SplitMix64 + Box-Muller ---------------------------------------------------------------

uint64_t splitmix_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Pair p of standard normals from outputs 2p and 2p+1 (seekable, so any split of the fill
// over threads gives the same values).
void normal_pair(uint64_t seed, uint64_t p, double* z0, double* z1) {
    const double u1 = ((splitmix_at(seed, 2 * p) >> 11) + 1) * 0x1p-53;  // (0, 1]
    const double u2 = (splitmix_at(seed, 2 * p + 1) >> 11) * 0x1p-53;    // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = 6.283185307179586476925286766559 * u2;
    *z0 = r * std::cos(a);
    *z1 = r * std::sin(a);
}

}  // namespace
}  // namespace halo_mi

using namespace halo_mi;

extern "C" {

const char* halo_mi_last_error(void) { return g_last_error.c_str(); }

uint64_t halo_mi_row_bytes(uint32_t type, uint32_t cols) {
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "row_bytes");
    return code ? 0 : rb;
}

uint64_t halo_mi_slab_bytes(uint32_t type, uint32_t rows, uint32_t cols) {
    if (!is_quant(type) || cols % block_elems(type) != 0) return 0;
    const uint64_t slabs = (rows + kSlabRows - 1) / kSlabRows;
    return slabs * slab_geom(type, cols).slab_bytes;
}

int halo_mi_repack_slab_host(uint32_t type, const void* src, uint64_t src_stride, uint32_t rows, uint32_t cols,
                             void* dst) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "repack_slab_host");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "repack_slab_host: type %u has no SLAB layout", type);
    if (src_stride == 0) src_stride = rb;
    if (rows > 1 && src_stride < rb)
        return set_error(HALO_MI_E_KERNEL, "repack_slab_host: row stride %llu < row bytes %llu",
                         (unsigned long long)src_stride, (unsigned long long)rb);
    const SlabGeom g = slab_geom(type, cols);
    const uint32_t nblk = cols / block_elems(type), S = cols / kSlot;
    const uint32_t slabs = (rows + kSlabRows - 1) / kSlabRows;
    auto* out = static_cast<uint8_t*>(dst);
    const auto* in = static_cast<const uint8_t*>(src);
    std::vector<uint8_t> zero(block_bytes(type), 0);
    parallel_rows((uint64_t)slabs * kSlabRows, 0, [&](uint64_t r0, uint64_t r1) {
        for (uint64_t row = r0; row < r1; ++row) {
            uint8_t* slab = out + (row / kSlabRows) * g.slab_bytes;
            const uint32_t lane = static_cast<uint32_t>(row % kSlabRows);
            for (uint32_t b = 0; b < nblk; ++b) {
                const uint8_t* blk = row < rows ? in + row * src_stride + (uint64_t)b * block_bytes(type) : zero.data();
                slab_pack_block(type, blk, slab, g, S, lane, b);
            }
        }
    });
    return HALO_MI_OK;
}

int halo_mi_unpack_slab_host(uint32_t type, const void* src, uint32_t rows, uint32_t cols, void* dst,
                             uint64_t dst_stride) {
    clear_error();
    int code;
    const uint64_t rb = row_bytes_checked(type, cols, &code, "unpack_slab_host");
    if (code) return code;
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "unpack_slab_host: type %u has no SLAB layout", type);
    if (dst_stride == 0) dst_stride = rb;
    if (rows > 1 && dst_stride < rb) return set_error(HALO_MI_E_KERNEL, "unpack_slab_host: row stride < row bytes");
    const SlabGeom g = slab_geom(type, cols);
    const uint32_t nblk = cols / block_elems(type), S = cols / kSlot;
    const auto* in = static_cast<const uint8_t*>(src);
    auto* out = static_cast<uint8_t*>(dst);
    parallel_rows(rows, 0, [&](uint64_t r0, uint64_t r1) {
        for (uint64_t row = r0; row < r1; ++row) {
            const uint8_t* slab = in + (row / kSlabRows) * g.slab_bytes;
            for (uint32_t b = 0; b < nblk; ++b)
                slab_unpack_block(type, slab, out + row * dst_stride + (uint64_t)b * block_bytes(type), g, S,
                                  static_cast<uint32_t>(row % kSlabRows), b);
        }
    });
    return HALO_MI_OK;
}

void halo_mi_fill_normal(uint64_t seed, float* out, uint64_t n, float mean, float std_) {
    const uint64_t pairs = (n + 1) / 2;
    parallel_rows(pairs, 0, [&](uint64_t p0, uint64_t p1) {
        for (uint64_t p = p0; p < p1; ++p) {
            double z0, z1;
            normal_pair(seed, p, &z0, &z1);
            out[2 * p] = static_cast<float>(mean + std_ * z0);
            if (2 * p + 1 < n) out[2 * p + 1] = static_cast<float>(mean + std_ * z1);
        }
    });
}

int halo_mi_quantize(uint32_t type, const float* src, uint64_t n, void* dst, uint32_t threads) {
    clear_error();
    if (!is_quant(type)) return set_error(HALO_MI_E_UNSUPPORTED, "quantize: type %u not supported", type);
    const uint32_t be = block_elems(type), bb = block_bytes(type);
    if (n % be) return set_error(HALO_MI_E_KERNEL, "quantize: %llu is not a multiple of %u", (unsigned long long)n, be);
    auto* out = static_cast<uint8_t*>(dst);
    parallel_rows(n / be, threads, [&](uint64_t b0, uint64_t b1) {
        for (uint64_t b = b0; b < b1; ++b) {
            const float* x = src + b * be;
            uint8_t* blk = out + b * bb;
            switch (type) {
                case kQ4_0: quant_q4_0(x, blk); break;
                case kQ8_0: quant_q8_0(x, blk); break;
                case kQ4_K: quant_k_affine<15>(x, blk); break;
                case kQ5_K: quant_k_affine<31>(x, blk); break;
                case kQ6_K: quant_q6_k(x, blk); break;
                case kIQ4_XS: quant_iq4_xs(x, blk); break;
            }
        }
    });
    return HALO_MI_OK;
}

}  // extern "C"
