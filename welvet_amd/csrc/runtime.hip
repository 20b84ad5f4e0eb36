// runtime.hip — C ABI of libwelvet_hip: device selection, resident blob
// table, upload-time re-layout and dispatch to the kernels in gemv.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/welvet_hip.h"
#include "wv_internal.h"

namespace wv {
namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
int hip_fail(hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return fail(WV_E_OOM, "%s: device memory exhausted (%s)", what, hipGetErrorString(e));
    return fail(WV_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

struct DeviceState {
    bool ready = false;
    hipStream_t stream = nullptr;
};

std::mutex g_mu;  // guards g_blobs, g_next, g_dev
std::unordered_map<uint64_t, DevBlob> g_blobs;
uint64_t g_next = 1;
DeviceState g_dev[64];
int g_current = -1;

int ensure_device_locked(int dev) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(WV_E_NODEV, "wv_init: no HIP device");
    if (dev < 0 || dev >= n || dev >= 64) return fail(WV_E_ARG, "wv_init: device %d out of range (count %d)", dev, n);
    hipError_t e = hipSetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "wv_init: hipSetDevice");
    if (!g_dev[dev].ready) {
        e = hipStreamCreateWithFlags(&g_dev[dev].stream, hipStreamNonBlocking);
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipStreamCreate");
        g_dev[dev].ready = true;
    }
    g_current = dev;
    return WV_OK;
}

int ensure_init() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_current >= 0) {
        hipSetDevice(g_current);
        return WV_OK;
    }
    return ensure_device_locked(0);
}

hipStream_t stream_or_default(void* s, int dev) {
    if (s) return static_cast<hipStream_t>(s);
    return g_dev[dev].stream;
}

bool force_raw() {
    const char* v = std::getenv("WV_FORCE_RAW");
    return v && v[0] == '1';
}

inline float f32_at(const uint8_t* p) { float v; std::memcpy(&v, p, 4); return v; }

// Host staging of a device image: byte buffer with 256-B aligned sections.
struct Image {
    std::vector<uint8_t> bytes;
    size_t add(size_t n) {
        size_t off = (bytes.size() + 255) & ~size_t(255);
        bytes.resize(off + n);
        return off;
    }
};

// Row-interleaved layout for the k-quants and the 32-block formats (requires cols % 256
// == 0): rows are grouped 64 at a time, one per lane of a wave, and every
// plane is stored [row group][chunk or super-block][lane][bytes] so that one
// wave-wide load reads contiguous memory. Byte count per 256 weights equals
// the reference blob's (Q2_K 104, Q3_K 136, Q4_K 168, Q5_K 200, Q6_K 216, Q8_0
// 288, Q4_0 160, Q4_1 / Q5_0 192, Q5_1 224); rows past
// `rows` in the last group are zero (d = 0 / scale = 0, contributing 0).
//   Q4_K: codes 16 B/chunk (LSB-first nibbles, as in the blob); meta per
//         super-block 8 words (u'(2p), u'(2p+1), m(2p), m(2p+1)); dd (d, dmin).
//         u' = max(u, 1): d*u/255 with u = 0 falls back to d/255
//         (quant/kquant.go:179-182), the value u = 1 gives.
//   Q5_K: low 4 code bits 16 B/chunk; fifth bits 4 B/chunk arranged for the
//         kernel's byte spread; meta and dd as Q4_K.
//   Q2_K / Q3_K: low 2 code bits 8 B/chunk (and Q3_K's third bits 4 B/chunk)
//         arranged for the kernel's byte spread; meta and dd as Q4_K.
//   Q6_K: low 4 code bits 16 B/chunk; high 2 bits 8 B/chunk arranged for
//         the kernel's byte spread; meta 8 u16 (u'(2p), u'(2p+1)); dd.
//   Q8_0 / Q4_0: codes 32 / 16 B per 32-block; meta 8 f32 block scales.
//   Q4_1 / Q5_0 / Q5_1: codes as Q4_0 (Q5_x: low 4 bits, plus the fifth
//         bits as Q5_K's); meta 8 f32 scales, then (Q4_1, Q5_1) 8 f32 mins.
// Code (and Q6_K high-bit) planes are chunk-step-major, [j][rg][sb][lane],
// j = chunk index inside the super-block; meta/dd are [rg][sb][lane].
struct RplOffsets {
    size_t codes = 0, hi = 0, meta = 0, dd = 0;
};
void build_rpl(int fmt, const uint8_t* raw, int64_t rows, int64_t cols, Image& img, RplOffsets& o) {
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256;
    const bool low2 = fmt == FMT_Q2_K || fmt == FMT_Q3_K;  // 2-bit plane (+ third bits)
    const bool bmin = fmt == FMT_Q4_1 || fmt == FMT_Q5_1;  // 32-blocks with a min
    const bool five = fmt == FMT_Q5_K || fmt == FMT_Q5_0 || fmt == FMT_Q5_1;
    const int cb = fmt == FMT_Q8_0 ? 32 : low2 ? 8 : 16, mb = fmt == FMT_Q6_K ? 16 : bmin ? 64 : 32;
    const bool kq = low2 || fmt == FMT_Q4_K || fmt == FMT_Q5_K || fmt == FMT_Q6_K;
    o.codes = img.add(size_t(rg * nch * 64 * cb));
    if (fmt == FMT_Q6_K) o.hi = img.add(size_t(rg * nch * 64 * 8));
    if (five || fmt == FMT_Q3_K) o.hi = img.add(size_t(rg * nch * 64 * 4));
    o.meta = img.add(size_t(rg * nsb * 64 * mb));
    if (kq) o.dd = img.add(size_t(rg * nsb * 64 * 8));
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* hi = base + o.hi;
    uint8_t* meta = base + o.meta;
    float* dd = reinterpret_cast<float*>(base + o.dd);
    KSpec ks;
    k_spec(fmt, ks);
    const int64_t sbb = kq ? k_super_bytes(ks) : 0;
    auto work = [&](int64_t g0, int64_t g1) {
        for (int64_t g = g0; g < g1; ++g)
            for (int lane = 0; lane < 64; ++lane) {
                const int64_t row = g * 64 + lane;
                if (row >= rows) continue;
                for (int64_t sb = 0; sb < nsb; ++sb) {
                    const int64_t mi = (g * nsb + sb) * 64 + lane;
                    uint8_t* m = meta + mi * mb;
                    if (kq) {
                        const uint8_t* o8 = raw + (row * nsb + sb) * sbb;
                        dd[2 * mi] = f32_at(o8);
                        dd[2 * mi + 1] = f32_at(o8 + 4);
                        for (int p = 0; p < 8; ++p) {
                            const int64_t ci = ((p * rg + g) * nsb + sb) * 64 + lane;  // [j][rg][sb][lane]
                            const uint8_t u0 = std::max<uint8_t>(o8[8 + 2 * p], 1), u1 = std::max<uint8_t>(o8[9 + 2 * p], 1);
                            if (fmt == FMT_Q4_K) {
                                m[4 * p] = u0;
                                m[4 * p + 1] = u1;
                                m[4 * p + 2] = o8[24 + 2 * p];
                                m[4 * p + 3] = o8[25 + 2 * p];
                                std::memcpy(codes + ci * 16, o8 + 40 + 16 * p, 16);
                            } else if (fmt == FMT_Q5_K || low2) {
                                m[4 * p] = u0;
                                m[4 * p + 1] = u1;
                                m[4 * p + 2] = o8[24 + 2 * p];
                                m[4 * p + 3] = o8[25 + 2 * p];
                                const int bits = ks.bits, qbytes = 32 * bits;  // 256*bits/8 bytes of codes
                                const uint8_t* q = o8 + 40;
                                uint8_t qv[32];
                                for (int k = 0; k < 32; ++k) {  // LSB-first stream (helpers.go:140-149)
                                    const int bit = (p * 32 + k) * bits;
                                    const uint32_t v = q[bit >> 3] | ((bit >> 3) + 1 < qbytes ? uint32_t(q[(bit >> 3) + 1]) << 8 : 0u);
                                    qv[k] = uint8_t((v >> (bit & 7)) & ((1u << bits) - 1));
                                }
                                // spread word s holds, in byte b, the code of column 8(s/2) + 2b + s%2
                                auto code = [&](int sw, int b) { return qv[8 * (sw >> 1) + 2 * b + (sw & 1)]; };
                                uint8_t* c = codes + ci * cb;
                                if (fmt == FMT_Q5_K) {
                                    for (int k = 0; k < 16; ++k) c[k] = uint8_t((qv[2 * k] & 15) | ((qv[2 * k + 1] & 15) << 4));
                                } else {  // dword s/4, byte b, bits 2(s%4): the low two bits
                                    std::memset(c, 0, 8);
                                    for (int sw = 0; sw < 8; ++sw)
                                        for (int b = 0; b < 4; ++b) c[4 * (sw >> 2) + b] |= uint8_t((code(sw, b) & 3) << (2 * (sw & 3)));
                                }
                                if (fmt != FMT_Q2_K) {  // byte b, bit s: the top bit (bit 4 of Q5_K, bit 2 of Q3_K)
                                    const int top = fmt == FMT_Q5_K ? 4 : 2;
                                    uint8_t* h = hi + ci * 4;
                                    std::memset(h, 0, 4);
                                    for (int sw = 0; sw < 8; ++sw)
                                        for (int b = 0; b < 4; ++b) h[b] |= uint8_t(((code(sw, b) >> top) & 1) << sw);
                                }
                            } else {
                                m[2 * p] = u0;
                                m[2 * p + 1] = u1;
                                const uint8_t* q = o8 + 24;  // 192 B of 6-bit codes
                                uint8_t qv[32];
                                for (int k = 0; k < 32; ++k) {  // LSB-first stream (helpers.go:140-149)
                                    const int bit = (p * 32 + k) * 6;
                                    const uint32_t v = q[bit >> 3] | ((bit >> 3) + 1 < 192 ? uint32_t(q[(bit >> 3) + 1]) << 8 : 0u);
                                    qv[k] = uint8_t((v >> (bit & 7)) & 63u);
                                }
                                uint8_t* c = codes + ci * 16;
                                for (int k = 0; k < 16; ++k) c[k] = uint8_t((qv[2 * k] & 15) | ((qv[2 * k + 1] & 15) << 4));
                                uint8_t* h = hi + ci * 8;
                                std::memset(h, 0, 8);
                                // spread word s = 2*w + half holds code 8w + 2b + half in byte b
                                for (int sw = 0; sw < 8; ++sw) {
                                    const int w = sw >> 1, half = sw & 1, t = sw >> 2, f = sw & 3;
                                    for (int b = 0; b < 4; ++b) h[t * 4 + b] |= uint8_t(((qv[8 * w + 2 * b + half] >> 4) & 3) << (2 * f));
                                }
                            }
                        }
                    } else {
                        // 32-blocks: [scale][min (Q4_1, Q5_1)][codes]; meta = 8 scales, then 8 mins
                        const int bb = fmt == FMT_Q8_0 ? 36 : fmt == FMT_Q4_0 ? 20 : fmt == FMT_Q5_1 ? 28 : 24;
                        const int hdr = bmin ? 8 : 4;
                        for (int p = 0; p < 8; ++p) {
                            const uint8_t* blk = raw + (row * nch + sb * 8 + p) * bb;
                            const int64_t ci = ((p * rg + g) * nsb + sb) * 64 + lane;
                            std::memcpy(m + 4 * p, blk, 4);
                            if (bmin) std::memcpy(m + 32 + 4 * p, blk + 4, 4);
                            if (!five) {
                                std::memcpy(codes + ci * cb, blk + hdr, size_t(cb));
                                continue;
                            }
                            uint8_t qv[32];
                            for (int k = 0; k < 32; ++k) {  // 20 B LSB-first stream of 5-bit codes
                                const int bit = k * 5;
                                const uint32_t v = blk[hdr + (bit >> 3)] | ((bit >> 3) + 1 < 20 ? uint32_t(blk[hdr + (bit >> 3) + 1]) << 8 : 0u);
                                qv[k] = uint8_t((v >> (bit & 7)) & 31u);
                            }
                            uint8_t* c = codes + ci * 16;
                            for (int k = 0; k < 16; ++k) c[k] = uint8_t((qv[2 * k] & 15) | ((qv[2 * k + 1] & 15) << 4));
                            uint8_t* h = hi + ci * 4;
                            std::memset(h, 0, 4);
                            for (int sw = 0; sw < 8; ++sw)
                                for (int b = 0; b < 4; ++b) h[b] |= uint8_t(((qv[8 * (sw >> 1) + 2 * b + (sw & 1)] >> 4) & 1) << sw);
                        }
                    }
                }
            }
    };
    const int64_t nthreads = std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), std::max<int64_t>(1, rg / 4));
    std::vector<std::thread> th;
    const int64_t per = (rg + nthreads - 1) / nthreads;
    for (int64_t t = 0; t < nthreads; ++t) {
        const int64_t g0 = t * per, g1 = std::min(rg, g0 + per);
        if (g0 < g1) th.emplace_back(work, g0, g1);
    }
    for (auto& t : th) t.join();
}

// Row-interleaved layout for the linear IQ formats (iq_rpl_spec): the codes
// come from Raw, one flat LSB-first stream over the whole matrix (element
// r*cols + c at bit (r*cols + c)*bits, quant/iq.go:182-207), and the group
// scales from Scales. Planes per 32-column chunk and lane: 4-bit codes as
// nibbles (16 B); 2- and 3-bit codes as Q2_K / Q3_K (8 B + 4 B of third
// bits); 1-bit codes as one 32-bit word holding at bit s of byte b the code
// of column 8(s/2) + 2b + s%2. Meta: per super-block 8 (group 32) or 16
// (group 16) f32 scales.
void build_rpl_lin(const LinCodes& lc, const uint8_t* raw, size_t raw_len, const float* scales, size_t n_scales,
                   int64_t rows, int64_t cols, Image& img, RplOffsets& o) {
    const int bits = lc.bits, sg = lc.sg;
    auto scale_at = [&](int64_t g) { return size_t(g) < n_scales && scales ? scales[g] : 1.0f; };
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256;
    const int cb = bits == 4 ? 16 : bits >= 2 ? 8 : 4, mb = sg == 16 ? 64 : 32;
    o.codes = img.add(size_t(rg * nch * 64 * cb));
    if (bits == 3) o.hi = img.add(size_t(rg * nch * 64 * 4));
    o.meta = img.add(size_t(rg * nsb * 64 * mb));
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* hi = base + o.hi;
    uint8_t* meta = base + o.meta;
    auto work = [&](int64_t g0, int64_t g1) {
        for (int64_t g = g0; g < g1; ++g)
            for (int lane = 0; lane < 64; ++lane) {
                const int64_t row = g * 64 + lane;
                if (row >= rows) continue;
                for (int64_t sb = 0; sb < nsb; ++sb) {
                    float* m = reinterpret_cast<float*>(meta + ((g * nsb + sb) * 64 + lane) * mb);
                    for (int p = 0; p < 8; ++p) {
                        const int64_t i0 = row * cols + sb * 256 + p * 32;
                        if (sg == 16) {
                            m[2 * p] = scale_at(i0 / 16);
                            m[2 * p + 1] = scale_at(i0 / 16 + 1);
                        } else {
                            m[p] = scale_at(i0 / 32);
                        }
                        uint8_t qv[32];
                        for (int k = 0; k < 32; ++k) {
                            const int64_t bit = (i0 + k) * bits;
                            const int64_t by = bit >> 3;
                            const uint32_t v = raw[by] | (size_t(by + 1) < raw_len ? uint32_t(raw[by + 1]) << 8 : 0u);
                            qv[k] = uint8_t((v >> (bit & 7)) & ((1u << bits) - 1));
                            if (lc.remap3 && qv[k] == 3) qv[k] = 1;  // TernaryPacked: code 3 decodes as 0
                        }
                        auto code = [&](int sw, int b) { return qv[8 * (sw >> 1) + 2 * b + (sw & 1)]; };
                        const int64_t ci = ((p * rg + g) * nsb + sb) * 64 + lane;
                        uint8_t* c = codes + ci * cb;
                        std::memset(c, 0, size_t(cb));
                        if (bits == 4) {
                            for (int k = 0; k < 16; ++k) c[k] = uint8_t(qv[2 * k] | (qv[2 * k + 1] << 4));
                        } else if (bits == 1) {
                            for (int sw = 0; sw < 8; ++sw)
                                for (int b = 0; b < 4; ++b) c[b] |= uint8_t((code(sw, b) & 1) << sw);
                        } else {
                            for (int sw = 0; sw < 8; ++sw)
                                for (int b = 0; b < 4; ++b) c[4 * (sw >> 2) + b] |= uint8_t((code(sw, b) & 3) << (2 * (sw & 3)));
                            if (bits == 3) {
                                uint8_t* h = hi + ci * 4;
                                std::memset(h, 0, 4);
                                for (int sw = 0; sw < 8; ++sw)
                                    for (int b = 0; b < 4; ++b) h[b] |= uint8_t(((code(sw, b) >> 2) & 1) << sw);
                            }
                        }
                    }
                }
            }
    };
    const int64_t nthreads = std::min<int64_t>(std::max(1u, std::thread::hardware_concurrency()), std::max<int64_t>(1, rg / 4));
    std::vector<std::thread> th;
    const int64_t per = (rg + nthreads - 1) / nthreads;
    for (int64_t t = 0; t < nthreads; ++t) {
        const int64_t g0 = t * per, g1 = std::min(rg, g0 + per);
        if (g0 < g1) th.emplace_back(work, g0, g1);
    }
    for (auto& t : th) t.join();
}

// AffinePacked with 64-column groups (affine_g64.go:124-161): 4-bit codes,
// element i at nibble i of Raw (low nibble first), as Q4_K's planes; meta per
// super-block and lane: the 4 group scales, then the 4 group mins (f32).
void build_rpl_affine(const uint8_t* raw, const float* scales, const float* mins, int64_t rows, int64_t cols, Image& img,
                      RplOffsets& o) {
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256, gpr = cols / 64;
    o.codes = img.add(size_t(rg * nch * 64 * 16));
    o.meta = img.add(size_t(rg * nsb * 64 * 32));
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* meta = base + o.meta;
    for (int64_t g = 0; g < rg; ++g)
        for (int lane = 0; lane < 64; ++lane) {
            const int64_t row = g * 64 + lane;
            if (row >= rows) continue;
            for (int64_t sb = 0; sb < nsb; ++sb) {
                float* m = reinterpret_cast<float*>(meta + ((g * nsb + sb) * 64 + lane) * 32);
                for (int q = 0; q < 4; ++q) {
                    m[q] = scales[row * gpr + sb * 4 + q];
                    m[4 + q] = mins[row * gpr + sb * 4 + q];
                }
                for (int p = 0; p < 8; ++p)
                    std::memcpy(codes + (((p * rg + g) * nsb + sb) * 64 + lane) * 16, raw + (row * cols + sb * 256 + p * 32) / 2, 16);
            }
        }
}

int upload_image(const Image& img, DevBlob& b) {
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, std::max<size_t>(img.bytes.size(), 256));
    if (e != hipSuccess) return hip_fail(e, "wv_blob_upload: hipMalloc");
    e = hipMemcpy(d, img.bytes.data(), img.bytes.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        hipFree(d);
        return hip_fail(e, "wv_blob_upload: hipMemcpy");
    }
    b.base = d;
    b.device_bytes = img.bytes.size();
    return WV_OK;
}

bool lookup(uint64_t h, DevBlob& out) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_blobs.find(h);
    if (it == g_blobs.end()) return false;
    out = it->second;
    return true;
}

bool supported_format(int fmt) {
    return (fmt >= FMT_Q8_0 && fmt <= FMT_AFFINE) || fmt == FMT_NATIVE_TERNARY;
}

// InferAffineBlockWeights (affine_g64.go:99-122): keep BlockWeights when the
// scales fit it, else 64 when they fit that, else cols / (scales per row).
int32_t infer_affine_group(int64_t rows, int64_t cols, int32_t bw, size_t n_scales) {
    if (bw > 0 && cols % bw == 0 && int64_t(n_scales) == rows * (cols / bw)) return bw;
    if (cols % 64 == 0 && int64_t(n_scales) == rows * (cols / 64)) return 64;
    if (int64_t(n_scales) % rows == 0) {
        const int64_t gpr = int64_t(n_scales) / rows;
        if (gpr > 0 && cols % gpr == 0) return int32_t(cols / gpr);
    }
    return bw > 0 ? bw : 64;
}

const char* fmt_name(int f) {
    static const char* names[] = {"none", "Q8_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1", "Q2_K", "Q3_K",
                                  "Q4_K", "Q5_K", "Q6_K", "IQ1_S", "IQ2_XXS", "IQ2_XS", "IQ3_XXS",
                                  "IQ3_S", "IQ4_NL", "IQ4_XS", "TernaryPacked", "BinaryPacked", "AffinePacked"};
    if (f >= 0 && f <= 20) return names[f];
    if (f == FMT_NATIVE_TERNARY) return "native-ternary";
    return "unknown";
}

// Raw bytes a blob must hold (quant.Pack sizes), or -1 if the format cannot
// be sized from (rows, cols) alone.
int64_t need_raw(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t* meta, size_t n_meta,
                 int64_t* need_scales) {
    const int64_t n = rows * cols;
    *need_scales = 0;
    if (fmt == FMT_NATIVE_TERNARY) return (n + 3) / 4;
    if (fmt == FMT_AFFINE) {  // 4-bit codes, groups of bw along each row (affine_g64.go:34-47)
        if (bw <= 0 || bw % 8 || cols % bw) return -1;
        *need_scales = rows * (cols / bw);
        return n / 2;
    }
    if (fmt == FMT_BINARY && bw == 128) {
        if (cols % 128 != 0) return -1;
        *need_scales = rows * (cols / 128);
        return rows * (cols / 32) * 4;
    }
    IQSpec is;
    if (iq_spec(fmt, is)) {
        if (n_meta >= 2) { is.bits = meta[0]; is.sg = meta[1]; }
        if (is.bits <= 0 || is.bits > 8 || is.sg <= 0) return -1;
        const int64_t padn = (n + is.sg - 1) / is.sg * is.sg;
        *need_scales = padn / is.sg;
        return (padn * is.bits + 7) / 8;
    }
    PackSizes ps;
    if (!pack_sizes(fmt, rows, cols, ps)) return -1;
    *need_scales = ps.scales;
    return ps.raw;
}

}  // namespace

// Helpers shared with the other HIP translation units (rt_internal.h).
int rt_fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}
int rt_hip_fail(hipError_t e, const char* what) { return hip_fail(e, what); }
int rt_ensure_init() { return ensure_init(); }
bool rt_lookup(uint64_t h, DevBlob& out) { return lookup(h, out); }
int rt_current_device() {
    std::lock_guard<std::mutex> lk(g_mu);
    return g_current;
}
}  // namespace wv

using namespace wv;

extern "C" {

int wv_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return ensure_device_locked(device);
}

const char* wv_last_error(void) { return g_err.c_str(); }

const char* wv_version(void) { return "welvet_hip 0.1 gfx950"; }

int wv_pack_sizes(int format, int64_t rows, int64_t cols, size_t* raw_len, size_t* n_scales, size_t* n_mins,
                  size_t* n_meta, int32_t* block_weights) {
    PackSizes ps;
    if (rows <= 0 || cols <= 0) return fail(WV_E_SHAPE, "PackSizes: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
    if (!pack_sizes(format, rows, cols, ps))
        return fail(WV_E_FORMAT, "quant: Pack not implemented for %s (native path TBD — no QAT fallback)", fmt_name(format));
    if (raw_len) *raw_len = size_t(ps.raw);
    if (n_scales) *n_scales = size_t(ps.scales);
    if (n_mins) *n_mins = size_t(ps.mins);
    if (n_meta) *n_meta = size_t(ps.meta);
    if (block_weights) *block_weights = ps.block_weights;
    return WV_OK;
}

int wv_pack(int format, const float* weights, int64_t rows, int64_t cols, uint8_t* raw, float* scales, float* mins,
            uint8_t* meta) {
    PackSizes ps;
    if (!weights || !raw) return fail(WV_E_ARG, "Pack: nil buffer");
    if (rows <= 0 || cols <= 0) return fail(WV_E_SHAPE, "Pack: bad shape rows=%lld cols=%lld len=0", (long long)rows, (long long)cols);
    if (!pack_sizes(format, rows, cols, ps))
        return fail(WV_E_FORMAT, "quant: Pack not implemented for %s (native path TBD — no QAT fallback)", fmt_name(format));
    if ((ps.scales && !scales) || (ps.mins && !mins) || (ps.meta && !meta))
        return fail(WV_E_ARG, "Pack: %s needs scales/mins/meta buffers", fmt_name(format));
    if (!pack(format, weights, rows, cols, raw, scales, mins, meta)) return fail(WV_E_FORMAT, "Pack: %s failed", fmt_name(format));
    return WV_OK;
}

int wv_pack_native_ternary(const float* weights, int64_t n, uint8_t* codes, float* scale) {
    if (!weights || !codes || !scale) return fail(WV_E_ARG, "packTernary: nil buffer");
    if (n <= 0) return fail(WV_E_SHAPE, "packTernary: empty tensor");
    pack_native_ternary(weights, n, codes, scale);
    return WV_OK;
}

int wv_blob_upload(int format, int64_t rows, int64_t cols, int32_t block_weights, const uint8_t* raw, size_t raw_len,
                   const float* scales, size_t n_scales, const float* mins, size_t n_mins, const uint8_t* meta,
                   size_t n_meta, float tensor_scale, uint64_t* handle) {
    if (!handle || !raw) return fail(WV_E_ARG, "wv_blob_upload: nil blob");
    if (rows <= 0 || cols <= 0)
        return fail(WV_E_SHAPE, "wv_blob_upload: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
    if (!supported_format(format))
        return fail(WV_E_FORMAT, "quant: MatVec not implemented for %s (native path TBD — no QAT fallback)", fmt_name(format));
    if (format == FMT_AFFINE) {
        // The fused path takes 4-bit codes only and every group's scale and
        // bias (EnsureAffineSIMDCache, k_iq_simd.go:187-215; simd_k_iq.go:57-67).
        const int bits = n_meta > 0 && meta[0] > 0 ? meta[0] : 4;
        if (bits != 4) return fail(WV_E_FORMAT, "wv_blob_upload: AffinePacked bits=%d not supported (want 4)", bits);
        block_weights = infer_affine_group(rows, cols, block_weights, n_scales);
        const int64_t groups = block_weights > 0 && cols % block_weights == 0 ? rows * (cols / block_weights) : 0;
        if (!mins || int64_t(n_mins) < groups)
            return fail(WV_E_SHAPE, "wv_blob_upload: AffinePacked needs %lld mins, got %zu", (long long)groups, n_mins);
    }
    int64_t need_sc = 0;
    const int64_t need = need_raw(format, rows, cols, block_weights, meta, n_meta, &need_sc);
    if (need < 0) return fail(WV_E_SHAPE, "wv_blob_upload: %s cannot hold rows=%lld cols=%lld", fmt_name(format), (long long)rows, (long long)cols);
    if (int64_t(raw_len) < need)
        return fail(WV_E_SHAPE, "wv_blob_upload: %s raw short: %zu bytes, need %lld", fmt_name(format), raw_len, (long long)need);
    if (need_sc > 0 && (!scales || int64_t(n_scales) < need_sc)) {
        // The reference substitutes scale 1 for missing ternary/binary scales
        // (ternary.go:69-72); IQ needs every scale (iq.go:193-195).
        if (format != FMT_TERNARY && format != FMT_BINARY)
            return fail(WV_E_SHAPE, "wv_blob_upload: %s needs %lld scales, got %zu", fmt_name(format), (long long)need_sc, n_scales);
    }
    int rc = ensure_init();
    if (rc) return rc;

    DevBlob b;
    b.fmt = format;
    b.rows = rows;
    b.cols = cols;
    b.block_weights = block_weights;
    b.tensor_scale = tensor_scale == 0.0f ? 1.0f : tensor_scale;  // expandNarrowToI8 (simd.go:153-156)
    b.device = g_current;
    Image img;
    const bool raw_only = force_raw();
    RplOffsets ro;
    IQSpec iqs;
    if (iq_spec(format, iqs)) {
        if (n_meta >= 2) { iqs.bits = meta[0]; iqs.sg = meta[1]; }
        b.iq_bits = iqs.bits;
        b.iq_sg = iqs.sg;
    }
    size_t o_codes = 0, o_raw = 0, o_sc = 0, o_mn = 0;
    if (format == FMT_NATIVE_TERNARY) {
        b.layout = LAYOUT_TERNARY_I8;
        if (cols > 32768) return fail(WV_E_SHAPE, "wv_blob_upload: native ternary cols %lld > 32768", (long long)cols);
        o_codes = img.add(size_t(need));
        std::memcpy(img.bytes.data() + o_codes, raw, size_t(need));
    } else if (!raw_only &&
               (format == FMT_Q2_K || format == FMT_Q3_K || format == FMT_Q4_K || format == FMT_Q5_K ||
                format == FMT_Q6_K || format == FMT_Q8_0 || format == FMT_Q4_0 || format == FMT_Q4_1 ||
                format == FMT_Q5_0 || format == FMT_Q5_1) &&
               cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl(format, raw, rows, cols, img, ro);
    } else if (LinCodes lc; !raw_only && rpl_lin_spec(format, block_weights, b.iq_bits, b.iq_sg, lc) && cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl_lin(lc, raw, raw_len, scales, n_scales, rows, cols, img, ro);
    } else if (!raw_only && format == FMT_AFFINE && block_weights == 64 && cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl_affine(raw, scales, mins, rows, cols, img, ro);
    } else {
        b.layout = LAYOUT_RAW;
        // 16 bytes of padding: the vectorized decoder reads whole aligned
        // dwords around each run of codes, up to 4 bytes past the last one.
        o_raw = img.add(size_t(need) + 16);
        std::memcpy(img.bytes.data() + o_raw, raw, size_t(need));
        b.raw_len = need;
        if (format == FMT_AFFINE) {
            b.n_mins = rows * (cols / block_weights);
            o_mn = img.add(size_t(b.n_mins) * 4);
            std::memcpy(img.bytes.data() + o_mn, mins, size_t(b.n_mins) * 4);
        }
        if (scales && n_scales) {
            o_sc = img.add(n_scales * 4);
            std::memcpy(img.bytes.data() + o_sc, scales, n_scales * 4);
            b.n_scales = int64_t(n_scales);
        }
    }
    // K-split scratch for the row-interleaved path: forward partial sums
    // [batch][split][rows] and MatVecT slice partials.
    size_t o_part = 0, o_tpart = 0, weight_bytes = img.bytes.size();
    if (b.layout == LAYOUT_RPL) {
        const int64_t rg = (rows + 63) / 64, nsb = cols / 256;
        b.rpl_max_batch = 8;
        b.rpl_max_split = int(std::max<int64_t>(1, (nsb + 3) / 4));
        o_part = img.add(size_t(b.rpl_max_batch) * b.rpl_max_split * rg * 64 * sizeof(float));
        RplArgs shape{};
        shape.rows = int(rows);
        shape.nsb = int(nsb);
        shape.rg_count = int(rg);
        const size_t tf = rpl_t_scratch_floats(shape);
        if (tf) {
            o_tpart = img.add(tf * sizeof(float));
        }
    }
    rc = upload_image(img, b);
    if (rc) return rc;
    b.device_bytes = weight_bytes;
    uint8_t* base = static_cast<uint8_t*>(b.base);
    if (b.layout == LAYOUT_RAW) {
        b.raw = base + o_raw;
        b.scales = b.n_scales ? reinterpret_cast<const float*>(base + o_sc) : nullptr;
        b.mins = b.n_mins ? reinterpret_cast<const float*>(base + o_mn) : nullptr;
    } else if (b.layout == LAYOUT_TERNARY_I8) {
        b.codes = base + o_codes;
    } else {
        RplArgs& r = b.rpl;
        r.codes = base + ro.codes;
        r.hi = ro.hi ? base + ro.hi : nullptr;
        r.meta = base + ro.meta;
        r.dd = ro.dd ? reinterpret_cast<const float2_t*>(base + ro.dd) : nullptr;
        r.partial = reinterpret_cast<float*>(base + o_part);
        r.rows = int(rows);
        r.nsb = int(cols / 256);
        r.rg_count = int((rows + 63) / 64);
        r.ksplit = 1;
        if (o_tpart) {
            b.rpl_t_partial = reinterpret_cast<float*>(base + o_tpart);
        }
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const uint64_t h = g_next++;
    g_blobs[h] = b;
    *handle = h;
    return WV_OK;
}

int wv_blob_upload_wire(int format, int64_t rows, int64_t cols, const uint8_t* wire, size_t wire_len,
                        uint64_t* handle) {
    if (!handle || !wire) return fail(WV_E_ARG, "wv_blob_upload_wire: nil wire");
    if (format == FMT_NONE || format == FMT_NATIVE_TERNARY)
        return fail(WV_E_FORMAT, "entity: not a packed quant blob (format=%s)", fmt_name(format));
    if (wire_len < 12) return fail(WV_E_SHAPE, "packed wire too short");
    uint32_t hdr[3];
    std::memcpy(hdr, wire, 12);
    const uint64_t ns = hdr[0], nm = hdr[1], nr = hdr[2];
    const uint64_t need = 12 + ns * 4 + nm * 4 + nr;
    if (wire_len < need)
        return fail(WV_E_SHAPE, "packed wire truncated (need %llu, have %zu)", (unsigned long long)need, wire_len);
    // The float arrays may sit at any byte offset of a mapped file: copy them out.
    std::vector<float> sc(ns), mn(nm);
    if (ns) std::memcpy(sc.data(), wire + 12, ns * 4);
    if (nm) std::memcpy(mn.data(), wire + 12 + ns * 4, nm * 4);
    const uint8_t* raw = wire + 12 + ns * 4 + nm * 4;
    int32_t bw = 0;
    if (format == FMT_BINARY) {
        bw = (cols % 128 == 0 && int64_t(ns) == rows * (cols / 128)) ? 128 : 32;
    } else if (format != FMT_AFFINE) {
        PackSizes ps;
        if (pack_sizes(format, rows, cols, ps)) bw = ps.block_weights;
    }
    return wv_blob_upload(format, rows, cols, bw, raw, size_t(nr), ns ? sc.data() : nullptr, size_t(ns),
                          nm ? mn.data() : nullptr, size_t(nm), nullptr, 0, 0.0f, handle);
}

int wv_blob_free(uint64_t handle) {
    DevBlob b;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_blobs.find(handle);
        if (it == g_blobs.end()) return fail(WV_E_HANDLE, "wv_blob_free: unknown handle %llu", (unsigned long long)handle);
        b = it->second;
        g_blobs.erase(it);
    }
    hipSetDevice(b.device);
    hipError_t e = hipFree(b.base);
    if (e != hipSuccess) return hip_fail(e, "wv_blob_free: hipFree");
    return WV_OK;
}

int wv_blob_info(uint64_t handle, int* format, int64_t* rows, int64_t* cols, size_t* device_bytes, int* layout) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "wv_blob_info: unknown handle %llu", (unsigned long long)handle);
    if (format) *format = b.fmt;
    if (rows) *rows = b.rows;
    if (cols) *cols = b.cols;
    if (device_bytes) *device_bytes = b.device_bytes;
    if (layout) *layout = b.layout;
    return WV_OK;
}

int wv_matvec_dev(uint64_t handle, const float* d_x, float* d_y, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVec: unknown handle %llu", (unsigned long long)handle);
    if (!d_x || !d_y) return fail(WV_E_ARG, "MatVec: nil x/y");
    if (batch < 0) return fail(WV_E_SHAPE, "MatVec: negative batch %d", batch);
    hipSetDevice(b.device);
    const int e = launch_matvec(b, d_x, d_y, batch, stream_or_default(stream, b.device));
    if (e != hipSuccess) return hip_fail(hipError_t(e), "MatVec: kernel launch");
    return WV_OK;
}

int wv_ternary_acc_dev(uint64_t handle, const float* d_x, int32_t* d_acc, float* d_act_scale, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "ternary acc: unknown handle %llu", (unsigned long long)handle);
    if (b.layout != LAYOUT_TERNARY_I8) return fail(WV_E_FORMAT, "ternary acc: blob is %s, not native ternary", fmt_name(b.fmt));
    if (!d_x || !d_acc) return fail(WV_E_ARG, "ternary acc: nil x/acc");
    hipSetDevice(b.device);
    const int e = launch_ternary_acc(b, d_x, d_acc, d_act_scale, batch, stream_or_default(stream, b.device));
    if (e != hipSuccess) return hip_fail(hipError_t(e), "ternary acc: kernel launch");
    return WV_OK;
}

int wv_matvec_t_dev(uint64_t handle, const float* d_gy, float* d_gx, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVecT: unknown handle %llu", (unsigned long long)handle);
    if (!d_gy || !d_gx) return fail(WV_E_ARG, "MatVecT: nil gy/gx");
    if (b.layout == LAYOUT_TERNARY_I8)
        return fail(WV_E_FORMAT, "quant: MatVecT not implemented for %s", fmt_name(b.fmt));
    if (batch <= 0) return WV_OK;
    hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    if (b.layout == LAYOUT_RPL) {
        const int k = launch_matvec_t(b, d_gy, d_gx, batch, s, nullptr);
        if (k != hipSuccess) return hip_fail(hipError_t(k), "MatVecT: kernel launch");
        return WV_OK;
    }
    float* part = nullptr;
    const size_t nf = matvec_t_scratch_floats(b, batch);
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&part), std::max<size_t>(nf, 1) * sizeof(float), s);
    if (e != hipSuccess) return hip_fail(e, "MatVecT: scratch");
    const int k = launch_matvec_t(b, d_gy, d_gx, batch, s, part);
    hipFreeAsync(part, s);
    if (k != hipSuccess) return hip_fail(hipError_t(k), "MatVecT: kernel launch");
    return WV_OK;
}

int wv_matmul_dev(uint64_t handle, const float* d_x, float* d_y, int32_t m, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatMul: unknown handle %llu", (unsigned long long)handle);
    if (!d_x || !d_y) return fail(WV_E_ARG, "MatMul: nil x/y");
    if (m < 0) return fail(WV_E_ARG, "MatMul: negative row count %d", m);
    if (m == 0) return WV_OK;
    hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    if (!gemm_supported(b, m)) {
        const int k = launch_matvec(b, d_x, d_y, m, s);
        if (k != hipSuccess) return hip_fail(hipError_t(k), "MatMul: kernel launch");
        return WV_OK;
    }
    float* part = nullptr;
    const size_t nf = gemm_scratch_floats(b, m);
    if (nf) {
        hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&part), nf * sizeof(float), s);
        if (e != hipSuccess) return hip_fail(e, "MatMul: split-K scratch");
    }
    const int k = launch_gemm(b, d_x, d_y, m, s, part);
    if (part) hipFreeAsync(part, s);
    if (k != hipSuccess) return hip_fail(hipError_t(k), "MatMul: kernel launch");
    return WV_OK;
}

int wv_matmul(uint64_t handle, const float* x, float* y, int32_t m) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatMul: unknown handle %llu", (unsigned long long)handle);
    if (!x || !y) return fail(WV_E_ARG, "MatMul: nil x/y");
    if (m <= 0) return m < 0 ? fail(WV_E_ARG, "MatMul: negative row count %d", m) : WV_OK;
    hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    const size_t nx = size_t(m) * size_t(b.cols), ny = size_t(m) * size_t(b.rows);
    float *dx = nullptr, *dy = nullptr;
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&dx), nx * 4, s);
    if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&dy), ny * 4, s);
    if (e != hipSuccess) return hip_fail(e, "MatMul: staging");
    int rc = WV_OK;
    e = hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) rc = hip_fail(e, "MatMul: copy x");
    if (!rc) rc = wv_matmul_dev(handle, dx, dy, m, s);
    if (!rc) {
        e = hipMemcpyAsync(y, dy, ny * 4, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) rc = hip_fail(e, "MatMul: copy y");
    }
    hipFreeAsync(dx, s);
    hipFreeAsync(dy, s);
    e = hipStreamSynchronize(s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "MatMul: sync");
    return rc;
}

int wv_matvec(uint64_t handle, const float* x, float* y, int32_t batch) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVec: unknown handle %llu", (unsigned long long)handle);
    if (!x || !y) return fail(WV_E_ARG, "MatVec: nil x/y");
    if (batch <= 0) return WV_OK;
    hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    const size_t nx = size_t(batch) * size_t(b.cols), ny = size_t(batch) * size_t(b.rows);
    float *dx = nullptr, *dy = nullptr;
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&dx), nx * 4, s);
    if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&dy), ny * 4, s);
    if (e != hipSuccess) return hip_fail(e, "MatVec: staging");
    e = hipMemcpyAsync(dx, x, nx * 4, hipMemcpyHostToDevice, s);
    int rc = WV_OK;
    if (e != hipSuccess) rc = hip_fail(e, "MatVec: copy x");
    if (!rc) {
        const int k = launch_matvec(b, dx, dy, batch, s);
        if (k != hipSuccess) rc = hip_fail(hipError_t(k), "MatVec: kernel launch");
    }
    if (!rc) {
        e = hipMemcpyAsync(y, dy, ny * 4, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) rc = hip_fail(e, "MatVec: copy y");
    }
    hipFreeAsync(dx, s);
    hipFreeAsync(dy, s);
    e = hipStreamSynchronize(s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "MatVec: sync");
    return rc;
}

int wv_matvec_t(uint64_t handle, const float* gy, float* gx, int32_t batch) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVecT: unknown handle %llu", (unsigned long long)handle);
    if (!gy || !gx) return fail(WV_E_ARG, "MatVecT: nil gy/gx");
    if (batch <= 0) return WV_OK;
    hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    const size_t ng = size_t(batch) * size_t(b.rows), nx = size_t(batch) * size_t(b.cols);
    float *dg = nullptr, *dx = nullptr;
    hipError_t e = hipMallocAsync(reinterpret_cast<void**>(&dg), ng * 4, s);
    if (e == hipSuccess) e = hipMallocAsync(reinterpret_cast<void**>(&dx), nx * 4, s);
    if (e != hipSuccess) return hip_fail(e, "MatVecT: staging");
    int rc = WV_OK;
    e = hipMemcpyAsync(dg, gy, ng * 4, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(dx, gx, nx * 4, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) rc = hip_fail(e, "MatVecT: copy in");
    if (!rc) rc = wv_matvec_t_dev(handle, dg, dx, batch, s);
    if (!rc) {
        e = hipMemcpyAsync(gx, dx, nx * 4, hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) rc = hip_fail(e, "MatVecT: copy out");
    }
    hipFreeAsync(dg, s);
    hipFreeAsync(dx, s);
    e = hipStreamSynchronize(s);
    if (!rc && e != hipSuccess) rc = hip_fail(e, "MatVecT: sync");
    return rc;
}

int wv_sync(void* stream) {
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(stream_or_default(stream, g_current));
    if (e != hipSuccess) return hip_fail(e, "wv_sync");
    return WV_OK;
}

}  // extern "C"
