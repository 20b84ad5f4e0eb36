// runtime.hip — C ABI of libwelvet_hip: device selection, resident blob
// table, upload-time re-layout and dispatch to the kernels in gemv.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
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

// Scratch of wv_matvec_dev_noalloc: a fixed device array, one copy per GPU
// the library runs on, held until the process ends. Host code never uses
// this name as an address: each device's address comes from
// hipGetSymbolAddress at initialisation (DeviceState::scratch).
constexpr size_t kNoAllocScratchFloats = size_t(1) << 20;  // 4 MiB
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

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
    float* scratch = nullptr;  // this device's address of the file-scope `scratch` array
    // The last wv_matvec_dev_noalloc call on this device: its stream and an
    // event recorded after its launches (created at initialisation), so that a
    // call on another stream while that one may still read or write `scratch`
    // is refused instead of racing (guarded by na_mu).
    std::mutex na_mu;
    hipEvent_t na_done = nullptr;
    hipStream_t na_stream = nullptr;
    bool na_pending = false;
    uint64_t resident = 0;  // device bytes of the uploaded blobs (g_mu)
    // Stream-ordered pool of the per-call buffers (K-split partials, host
    // staging). Its release threshold is unbounded, so memory freed by one
    // call stays in the pool for the next instead of going back to the driver
    // at each synchronization; the library's own pool leaves the device's
    // default pool as other users configured it.
    hipMemPool_t pool = nullptr;
};

std::mutex g_mu;  // guards g_blobs, g_next, g_dev, g_budget
std::unordered_map<uint64_t, DevBlob> g_blobs;
uint64_t g_next = 1;
DeviceState g_dev[64];
int g_current = -1;
uint64_t g_budget = 0;  // wv_set_weight_budget: per-device cap on blob bytes, 0 = none

int ensure_device_locked(int dev) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(WV_E_NODEV, "wv_init: no HIP device");
    if (dev < 0 || dev >= n || dev >= 64) return fail(WV_E_ARG, "wv_init: device %d out of range (count %d)", dev, n);
    hipError_t e = hipSetDevice(dev);
    if (e != hipSuccess) return hip_fail(e, "wv_init: hipSetDevice");
    if (!g_dev[dev].ready) {
        void* sp = nullptr;
        e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipGetSymbolAddress(scratch)");
        e = hipStreamCreateWithFlags(&g_dev[dev].stream, hipStreamNonBlocking);
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipStreamCreate");
        hipMemPoolProps props{};
        props.allocType = hipMemAllocationTypePinned;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = dev;
        e = hipMemPoolCreate(&g_dev[dev].pool, &props);
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipMemPoolCreate");
        uint64_t keep = UINT64_MAX;
        e = hipMemPoolSetAttribute(g_dev[dev].pool, hipMemPoolAttrReleaseThreshold, &keep);
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipMemPoolSetAttribute");
        e = hipEventCreateWithFlags(&g_dev[dev].na_done, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(e, "wv_init: hipEventCreate");
        g_dev[dev].scratch = static_cast<float*>(sp);
        g_dev[dev].ready = true;
    }
    g_current = dev;
    return WV_OK;
}

int ensure_init() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_current >= 0) {
        (void)hipSetDevice(g_current);
        return WV_OK;
    }
    return ensure_device_locked(0);
}

hipStream_t stream_or_default(void* s, int dev) {
    if (s) return static_cast<hipStream_t>(s);
    return g_dev[dev].stream;
}


// Allocation from the current device's library pool, in stream order (the
// staging buffers of the host entry points, which wait for their stream).
hipError_t pool_alloc(void** p, size_t bytes, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64 || !g_dev[dev].pool) return hipErrorNotInitialized;
    return hipMallocFromPoolAsync(p, bytes, g_dev[dev].pool, st);
}

// Scratch of the K-split / slice partials of one call. A call owns a slot of
// its device from before its first launch until its last launch is enqueued,
// under the device's slot lock; the slot's event, recorded after those
// launches, marks when the GPU is done with it. A call takes the slot last
// used on its own stream, else an idle slot, else the least recently used
// one, and unless the slot is idle its stream waits for the slot's event on
// the GPU (on the same stream that wait is already implied; it is kept so
// that a stream handle reused after a destroy cannot overlap the old
// stream's work). So two launches that could overlap never share partials,
// and steady-state calls allocate nothing (a stream-ordered allocation and
// free per call cost 4-10 us against 12-13 us of MatVecT). Slots only grow;
// they live as long as the process.
constexpr int kScratchSlots = 4;
struct ScratchSlot {
    float* p = nullptr;
    size_t floats = 0;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;  // stream of the last use
    uint64_t stamp = 0;
};
struct DeviceScratch {
    std::mutex mu;
    ScratchSlot slot[kScratchSlots];
    uint64_t clock = 0;
};
DeviceScratch g_scratch[64];

struct CallScratch {
    DeviceScratch* ds = nullptr;
    ScratchSlot* sl = nullptr;
    hipStream_t s = nullptr;
    std::unique_lock<std::mutex> lk;
    int get(size_t floats, hipStream_t st, const char* what) {
        if (!floats) return WV_OK;
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return hip_fail(e, what);
        if (dev < 0 || dev >= 64) return fail(WV_E_ARG, "%s: device %d", what, dev);
        ds = &g_scratch[dev];
        lk = std::unique_lock<std::mutex>(ds->mu);
        s = st;
        ScratchSlot* pick = nullptr;
        for (ScratchSlot& c : ds->slot)
            if (c.p && c.last == st) { pick = &c; break; }
        if (!pick)
            for (ScratchSlot& c : ds->slot)
                if (!c.p || hipEventQuery(c.done) == hipSuccess) { pick = &c; break; }
        if (!pick) {
            pick = &ds->slot[0];
            for (ScratchSlot& c : ds->slot)
                if (c.stamp < pick->stamp) pick = &c;
        }
        bool wait = pick->p && hipEventQuery(pick->done) != hipSuccess;
        // The event only orders later launches after the slot's last ones (and
        // tells the host when they are done); no data passes through it to
        // the host, so it skips the system-scope fence and its cache
        // writeback (with the fence each record cost 2-3 us of MatVecT).
        if (!pick->done &&
            (e = hipEventCreateWithFlags(&pick->done, hipEventDisableTiming | hipEventDisableSystemFence)) != hipSuccess) {
            pick->done = nullptr;
            return hip_fail(e, what);
        }
        if (pick->floats < floats) {  // grow: the old buffer may still be in use on the GPU
            if (pick->p) {
                if ((e = hipEventSynchronize(pick->done)) != hipSuccess) return hip_fail(e, what);
                (void)hipFree(pick->p);
                pick->p = nullptr;
                pick->floats = 0;
            }
            const size_t n = std::max<size_t>(floats, size_t(1) << 16);
            if ((e = hipMalloc(reinterpret_cast<void**>(&pick->p), n * sizeof(float))) != hipSuccess) {
                pick->p = nullptr;
                return hip_fail(e, what);
            }
            pick->floats = n;
            wait = false;
        }
        if (wait && (e = hipStreamWaitEvent(st, pick->done, 0)) != hipSuccess) return hip_fail(e, what);
        sl = pick;
        return WV_OK;
    }
    float* f() const { return sl ? sl->p : nullptr; }
    ~CallScratch() {
        if (!sl) return;
        (void)hipEventRecord(sl->done, s);
        sl->last = s;
        sl->stamp = ++ds->clock;
    }
};

// Device copies of a host call's buffers on stream s; finish() frees them in
// stream order and waits for the stream.
struct Staging {
    hipStream_t s;
    std::vector<void*> bufs;
    hipError_t err = hipSuccess;
    explicit Staging(hipStream_t st) : s(st) {}
    template <class T = float>
    T* out(size_t n) {
        void* p = nullptr;
        if (err == hipSuccess) err = pool_alloc(&p, std::max<size_t>(n, 1) * sizeof(T), s);
        if (err == hipSuccess) bufs.push_back(p);
        return static_cast<T*>(p);
    }
    template <class T>
    T* in(const T* h, size_t n) {
        T* p = out<T>(n);
        if (err == hipSuccess && n) err = hipMemcpyAsync(p, h, n * sizeof(T), hipMemcpyHostToDevice, s);
        return p;
    }
    int rc(const char* what) { return err == hipSuccess ? WV_OK : hip_fail(err, what); }
    template <class T>
    int back(T* h, const T* d, size_t n, const char* what) {
        const hipError_t e = n ? hipMemcpyAsync(h, d, n * sizeof(T), hipMemcpyDeviceToHost, s) : hipSuccess;
        return e == hipSuccess ? WV_OK : hip_fail(e, what);
    }
    int finish(int rc, const char* what) {
        for (void* p : bufs) (void)hipFreeAsync(p, s);
        bufs.clear();
        const hipError_t e = hipStreamSynchronize(s);
        if (!rc && e != hipSuccess) rc = hip_fail(e, what);
        return rc;
    }
    ~Staging() {
        for (void* p : bufs) (void)hipFreeAsync(p, s);
    }
};

inline float f32_at(const uint8_t* p) { float v; std::memcpy(&v, p, 4); return v; }

// Device order of the narrow DTypes' codes (LAYOUT_NARROW). The Store packs
// B-bit codes LSB-first, so a 32-bit word holds its E = 32/B elements j at
// bits B*j. The device word holds element j = 4k + b at bits 8b + B*k
// (k < 8/B, b < 4): then (w >> B*k) & mask gives, in byte b, the code of
// element 4k + b, so four consecutive elements meet four consecutive int8
// activations in one v_dot4 (native.hip). Int8 (B = 8) is unchanged.
void narrow_permute_words(uint8_t* p, size_t n, int B) {
    if (B >= 8) return;
    const int E = 32 / B;
    const uint32_t m = (1u << B) - 1u;
    for (size_t off = 0; off < n; off += 4) {
        uint32_t w = 0, o = 0;
        std::memcpy(&w, p + off, std::min<size_t>(4, n - off));  // the tail word's missing bytes read as 0
        for (int j = 0; j < E; ++j) o |= ((w >> (B * j)) & m) << (8 * (j & 3) + B * (j >> 2));
        std::memcpy(p + off, &o, 4);
    }
}

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
// Code (and high-bit) planes are in the chunk order rpl_strides gives (j =
// chunk index inside the super-block); meta/dd are [rg][sb][lane]. A last
// section holds one f32 per row (rg*64, 4 bytes per row beside the blob's
// bytes): the prefill GEMM's power-of-two row factor (gemm_row_factor).
struct RplOffsets {
    size_t codes = 0, hi = 0, meta = 0, dd = 0, wrow = 0;
};

// Row factor of the prefill GEMM (gemm_rpl.hip): 2^e with bound * 2^e in
// [2^12, 2^13), where `bound` is an upper bound on every fp16 value the
// GEMM's B-operand builder forms for the row (|scale| * qmax + |min|, or
// |scale| * (qmax + offset), over the row's sub-blocks). The GEMM multiplies
// the row's scales and mins by it before their fp16 cast and the row's
// outputs by its inverse, both exact: rows of tiny weights keep fp16's
// precision instead of going subnormal, and rows past 65504 stay finite.
// 1 for an all-zero or non-finite row.
float gemm_row_factor(double bound) {
    if (!(bound > 0.0) || !std::isfinite(bound)) return 1.0f;
    return std::ldexp(1.0f, std::min(126, std::max(-126, 12 - std::ilogb(bound))));
}
// The row-factor section: one float per row of the padded row groups, 1 for padding.
float* add_row_factors(Image& img, RplOffsets& o, int64_t rg) {
    o.wrow = img.add(size_t(rg * 64 * 4));
    float* w = reinterpret_cast<float*>(img.bytes.data() + o.wrow);
    std::fill(w, w + rg * 64, 1.0f);
    return w;
}
void build_rpl(int fmt, const uint8_t* raw, int64_t rows, int64_t cols, Image& img, RplOffsets& o) {
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256;
    int64_t cs_si = 0, cs_j = 0;
    rpl_strides(fmt, rg, nsb, cs_si, cs_j);
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
    float* wrow = add_row_factors(img, o, rg);
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* hi = base + o.hi;
    uint8_t* meta = base + o.meta;
    float* dd = reinterpret_cast<float*>(base + o.dd);
    KSpec ks;
    k_spec(fmt, ks);
    // GEMM value bounds per unit |scale| (gemm_row_factor): codes up to qmax
    // with a min (k-quants, Q4_1, Q5_1), codes minus an offset (Q6_K's 32,
    // Q4_0's 8, Q5_0's 16), Q8_0's signed bytes.
    const double qmax = fmt == FMT_Q6_K ? 63.0 + 32.0 : fmt == FMT_Q8_0 ? 128.0
                        : kq ? double((1 << ks.bits) - 1) : five ? (bmin ? 31.0 : 31.0 + 16.0) : (bmin ? 15.0 : 15.0 + 8.0);
    const int64_t sbb = kq ? k_super_bytes(ks) : 0;
    auto work = [&](int64_t g0, int64_t g1) {
        for (int64_t g = g0; g < g1; ++g)
            for (int lane = 0; lane < 64; ++lane) {
                const int64_t row = g * 64 + lane;
                if (row >= rows) continue;
                double bound = 0.0;
                for (int64_t sb = 0; sb < nsb; ++sb) {
                    const int64_t mi = (g * nsb + sb) * 64 + lane;
                    uint8_t* m = meta + mi * mb;
                    if (kq) {
                        const uint8_t* o8 = raw + (row * nsb + sb) * sbb;
                        dd[2 * mi] = f32_at(o8);
                        dd[2 * mi + 1] = f32_at(o8 + 4);
                        const double d255 = std::fabs(double(f32_at(o8))) / 255.0, dm127 = std::fabs(double(f32_at(o8 + 4))) / 127.0;
                        for (int p = 0; p < 8; ++p) {
                            const int64_t ci = ((g * nsb + sb) * cs_si + p * cs_j) * 64 + lane;
                            const uint8_t u0 = std::max<uint8_t>(o8[8 + 2 * p], 1), u1 = std::max<uint8_t>(o8[9 + 2 * p], 1);
                            for (int h = 0; h < 2; ++h)
                                bound = std::max(bound, d255 * (h ? u1 : u0) * qmax +
                                                            (fmt == FMT_Q6_K ? 0.0 : dm127 * std::abs(int(int8_t(o8[24 + 2 * p + h])))));
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
                            const int64_t ci = ((g * nsb + sb) * cs_si + p * cs_j) * 64 + lane;
                            std::memcpy(m + 4 * p, blk, 4);
                            if (bmin) std::memcpy(m + 32 + 4 * p, blk + 4, 4);
                            bound = std::max(bound, std::fabs(double(f32_at(blk))) * qmax +
                                                        (bmin ? std::fabs(double(f32_at(blk + 4))) : 0.0));
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
                wrow[row] = gemm_row_factor(bound);
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
void build_rpl_lin(int fmt, const LinCodes& lc, const uint8_t* raw, size_t raw_len, const float* scales,
                   size_t n_scales, int64_t rows, int64_t cols, Image& img, RplOffsets& o) {
    const int bits = lc.bits, sg = lc.sg;
    auto scale_at = [&](int64_t g) { return size_t(g) < n_scales && scales ? scales[g] : 1.0f; };
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256;
    int64_t cs_si = 0, cs_j = 0;
    rpl_strides(fmt, rg, nsb, cs_si, cs_j);
    const int nw = 256 / sg;  // scales per lane and super-block
    const int cb = bits == 4 ? 16 : bits >= 2 ? 8 : 4, mb = 4 * nw;
    o.codes = img.add(size_t(rg * nch * 64 * cb));
    if (bits == 3) o.hi = img.add(size_t(rg * nch * 64 * 4));
    o.meta = img.add(size_t(rg * nsb * 64 * mb));
    float* wrow = add_row_factors(img, o, rg);
    // GEMM value bound per unit |scale| (gemm_row_factor): w = scale*(q - mid)
    // with mid <= qmax (one-bit codes: 2*scale*(q - 1/2)).
    const double qmax = double((1 << bits) - 1) * (bits == 1 ? 4.0 : 2.0);
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* hi = base + o.hi;
    uint8_t* meta = base + o.meta;
    auto work = [&](int64_t g0, int64_t g1) {
        for (int64_t g = g0; g < g1; ++g)
            for (int lane = 0; lane < 64; ++lane) {
                const int64_t row = g * 64 + lane;
                if (row >= rows) continue;
                double bound = 0.0;
                for (int64_t sb = 0; sb < nsb; ++sb) {
                    float* m = reinterpret_cast<float*>(meta + ((g * nsb + sb) * 64 + lane) * mb);
                    for (int w = 0; w < nw; ++w) {
                        m[w] = scale_at((row * cols + sb * 256) / sg + w);
                        bound = std::max(bound, std::fabs(double(m[w])) * qmax);
                    }
                    for (int p = 0; p < 8; ++p) {
                        const int64_t i0 = row * cols + sb * 256 + p * 32;
                        uint8_t qv[32];
                        for (int k = 0; k < 32; ++k) {
                            const int64_t bit = (i0 + k) * bits;
                            const int64_t by = bit >> 3;
                            const uint32_t v = raw[by] | (size_t(by + 1) < raw_len ? uint32_t(raw[by + 1]) << 8 : 0u);
                            qv[k] = uint8_t((v >> (bit & 7)) & ((1u << bits) - 1));
                            if (lc.remap3 && qv[k] == 3) qv[k] = 1;  // TernaryPacked: code 3 decodes as 0
                        }
                        auto code = [&](int sw, int b) { return qv[8 * (sw >> 1) + 2 * b + (sw & 1)]; };
                        const int64_t ci = ((g * nsb + sb) * cs_si + p * cs_j) * 64 + lane;
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
                wrow[row] = gemm_row_factor(bound);
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
void build_rpl_affine(const uint8_t* raw, const float* scales, const float* mins, int64_t rows, int64_t cols, int bw,
                      Image& img, RplOffsets& o) {
    const int ng = 256 / bw;  // groups per super-block: ng scales, then ng mins, per lane
    const int64_t rg = (rows + 63) / 64, nch = cols / 32, nsb = cols / 256, gpr = cols / bw;
    int64_t cs_si = 0, cs_j = 0;
    rpl_strides(FMT_AFFINE, rg, nsb, cs_si, cs_j);
    o.codes = img.add(size_t(rg * nch * 64 * 16));
    o.meta = img.add(size_t(rg * nsb * 64 * 8 * ng));
    float* wrow = add_row_factors(img, o, rg);
    uint8_t* base = img.bytes.data();
    uint8_t* codes = base + o.codes;
    uint8_t* meta = base + o.meta;
    for (int64_t g = 0; g < rg; ++g)
        for (int lane = 0; lane < 64; ++lane) {
            const int64_t row = g * 64 + lane;
            if (row >= rows) continue;
            double bound = 0.0;
            for (int64_t sb = 0; sb < nsb; ++sb) {
                float* m = reinterpret_cast<float*>(meta + ((g * nsb + sb) * 64 + lane) * 8 * ng);
                for (int q = 0; q < ng; ++q) {
                    m[q] = scales[row * gpr + sb * ng + q];
                    m[ng + q] = mins[row * gpr + sb * ng + q];
                    bound = std::max(bound, std::fabs(double(m[q])) * 15.0 + std::fabs(double(m[ng + q])));
                }
                for (int p = 0; p < 8; ++p)
                    std::memcpy(codes + (((g * nsb + sb) * cs_si + p * cs_j) * 64 + lane) * 16, raw + (row * cols + sb * 256 + p * 32) / 2, 16);
            }
            wrow[row] = gemm_row_factor(bound);
        }
}

int upload_image(const Image& img, DevBlob& b) {
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, std::max<size_t>(img.bytes.size(), 256));
    if (e != hipSuccess) return hip_fail(e, "wv_blob_upload: hipMalloc");
    e = hipMemcpy(d, img.bytes.data(), img.bytes.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
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

bool supported_format(int fmt) { return (fmt >= FMT_NONE && fmt <= FMT_AFFINE) || narrow_bits(fmt) > 0; }

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
    switch (f) {  // core.DType names (core/dtype.go:67-140)
    case FMT_NATIVE_INT8: return "int8";
    case FMT_NATIVE_INT4: return "int4";
    case FMT_NATIVE_INT2: return "int2";
    case FMT_NATIVE_TERNARY: return "ternary";
    case FMT_NATIVE_BINARY: return "binary";
    default: return "unknown";
    }
}

// Raw bytes a blob must hold (quant.Pack sizes), or -1 if the format cannot
// be sized from (rows, cols) alone.
int64_t need_raw(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t* meta, size_t n_meta,
                 int64_t* need_scales) {
    const int64_t n = rows * cols;
    *need_scales = 0;
    if (fmt == FMT_NONE) return n * 4;  // f32 weights (quant/none.go:3-21)
    if (const int nb = narrow_bits(fmt)) return (n * nb + 7) / 8;  // packInt4/Int2/Ternary/Binary, Int8 bytes
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

int wv_pack_native(int format, const float* weights, int64_t n, uint8_t* codes, float* scale) {
    if (!weights || !codes || !scale) return fail(WV_E_ARG, "weights: nil buffer");
    if (n <= 0) return fail(WV_E_SHAPE, "weights: empty tensor");
    if (!pack_native(format, weights, n, codes, scale))
        return fail(WV_E_FORMAT, "weights: native pack for %s not provided (Int8, Int4, Int2, Ternary, Binary)", fmt_name(format));
    return WV_OK;
}

int wv_blob_upload_flags(int format, int64_t rows, int64_t cols, int32_t block_weights, const uint8_t* raw,
                         size_t raw_len, const float* scales, size_t n_scales, const float* mins, size_t n_mins,
                         const uint8_t* meta, size_t n_meta, float tensor_scale, uint32_t flags, uint64_t* handle) {
    if (!handle || !raw) return fail(WV_E_ARG, "wv_blob_upload: nil blob");
    if (flags & ~uint32_t(WV_UPLOAD_REFERENCE_LAYOUT)) return fail(WV_E_ARG, "wv_blob_upload: unknown flags 0x%x", flags);
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
    const bool raw_only = (flags & WV_UPLOAD_REFERENCE_LAYOUT) != 0;
    RplOffsets ro;
    IQSpec iqs;
    if (iq_spec(format, iqs)) {
        if (n_meta >= 2) { iqs.bits = meta[0]; iqs.sg = meta[1]; }
        b.iq_bits = iqs.bits;
        b.iq_sg = iqs.sg;
    }
    size_t o_codes = 0, o_raw = 0, o_sc = 0, o_mn = 0;
    if (narrow_bits(format) || format == FMT_NONE) {
        b.layout = format == FMT_NONE ? LAYOUT_F32 : LAYOUT_NARROW;
        if (b.layout == LAYOUT_NARROW && cols > 32768)
            return fail(WV_E_SHAPE, "wv_blob_upload: %s cols %lld > 32768", fmt_name(format), (long long)cols);
        // Whole 32-bit words plus 16 bytes, so that word and vector reads of
        // the last codes stay inside the section.
        o_codes = img.add((size_t(need) + 3) / 4 * 4 + 16);
        std::memcpy(img.bytes.data() + o_codes, raw, size_t(need));
        if (b.layout == LAYOUT_NARROW) narrow_permute_words(img.bytes.data() + o_codes, size_t(need), narrow_bits(format));
    } else if (!raw_only &&
               (format == FMT_Q2_K || format == FMT_Q3_K || format == FMT_Q4_K || format == FMT_Q5_K ||
                format == FMT_Q6_K || format == FMT_Q8_0 || format == FMT_Q4_0 || format == FMT_Q4_1 ||
                format == FMT_Q5_0 || format == FMT_Q5_1) &&
               cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl(format, raw, rows, cols, img, ro);
    } else if (LinCodes lc; !raw_only && rpl_lin_spec(format, block_weights, b.iq_bits, b.iq_sg, lc) && cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl_lin(format, lc, raw, raw_len, scales, n_scales, rows, cols, img, ro);
    } else if (!raw_only && format == FMT_AFFINE && rpl_affine_group(block_weights) && cols % 256 == 0) {
        b.layout = LAYOUT_RPL;
        build_rpl_affine(raw, scales, mins, rows, cols, block_weights, img, ro);
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
    // Reserve the bytes against the weight budget before allocating them.
    const uint64_t bytes = std::max<size_t>(img.bytes.size(), 256);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        uint64_t& res = g_dev[b.device].resident;
        if (g_budget && res + bytes > g_budget)
            return fail(WV_E_OOM, "wv_blob_upload: weight VRAM budget full (%llu resident + %llu > %llu bytes)",
                        (unsigned long long)res, (unsigned long long)bytes, (unsigned long long)g_budget);
        res += bytes;
    }
    rc = upload_image(img, b);
    if (rc) {
        std::lock_guard<std::mutex> lk(g_mu);
        g_dev[b.device].resident -= bytes;
        return rc;
    }
    uint8_t* base = static_cast<uint8_t*>(b.base);
    if (b.layout == LAYOUT_RAW) {
        b.raw = base + o_raw;
        b.scales = b.n_scales ? reinterpret_cast<const float*>(base + o_sc) : nullptr;
        b.mins = b.n_mins ? reinterpret_cast<const float*>(base + o_mn) : nullptr;
    } else if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32) {
        b.codes = base + o_codes;
    } else {
        RplArgs& r = b.rpl;
        r.codes = base + ro.codes;
        r.hi = ro.hi ? base + ro.hi : nullptr;
        r.meta = base + ro.meta;
        r.dd = ro.dd ? reinterpret_cast<const float2_t*>(base + ro.dd) : nullptr;
        r.wrow = reinterpret_cast<const float*>(base + ro.wrow);
        const float* wf = reinterpret_cast<const float*>(img.bytes.data() + ro.wrow);
        b.gemm_row_factors = std::any_of(wf, wf + rows, [](float f) { return f < 0.25f || f > 1048576.0f; });
        r.partial = nullptr;
        r.rows = int(rows);
        r.nsb = int(cols / 256);
        r.rg_count = int((rows + 63) / 64);
        r.ksplit = 1;
        rpl_strides(b.fmt, r.rg_count, r.nsb, r.cs_si, r.cs_j);
    }
    std::lock_guard<std::mutex> lk(g_mu);
    const uint64_t h = g_next++;
    g_blobs[h] = b;
    *handle = h;
    return WV_OK;
}

int wv_blob_upload(int format, int64_t rows, int64_t cols, int32_t block_weights, const uint8_t* raw, size_t raw_len,
                   const float* scales, size_t n_scales, const float* mins, size_t n_mins, const uint8_t* meta,
                   size_t n_meta, float tensor_scale, uint64_t* handle) {
    return wv_blob_upload_flags(format, rows, cols, block_weights, raw, raw_len, scales, n_scales, mins, n_mins, meta,
                                n_meta, tensor_scale, 0u, handle);
}

int wv_blob_upload_wire(int format, int64_t rows, int64_t cols, const uint8_t* wire, size_t wire_len,
                        uint64_t* handle) {
    if (!handle || !wire) return fail(WV_E_ARG, "wv_blob_upload_wire: nil wire");
    if (format == FMT_NONE || narrow_bits(format))
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
        g_dev[b.device].resident -= std::max<size_t>(b.device_bytes, 256);
    }
    (void)hipSetDevice(b.device);
    hipError_t e = hipFree(b.base);
    if (e != hipSuccess) return hip_fail(e, "wv_blob_free: hipFree");
    return WV_OK;
}

int wv_set_weight_budget(uint64_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    g_budget = bytes;
    return WV_OK;
}

int wv_weight_bytes(uint64_t* resident, uint64_t* budget) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (resident) *resident = g_current >= 0 ? g_dev[g_current].resident : 0;
    if (budget) *budget = g_budget;
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
    if (batch == 0) return WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    CallScratch sc;
    int rc = sc.get(matvec_scratch_floats(b, batch), s, "MatVec: scratch");
    if (rc) return rc;
    const int e = launch_matvec(b, d_x, d_y, batch, s, sc.f());
    if (e != hipSuccess) return hip_fail(hipError_t(e), "MatVec: kernel launch");
    return WV_OK;
}

int wv_matvec_dev_noalloc(uint64_t handle, const float* d_x, float* d_y, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVec: unknown handle %llu", (unsigned long long)handle);
    if (!d_x || !d_y) return fail(WV_E_ARG, "MatVec: nil x/y");
    if (batch < 0) return fail(WV_E_SHAPE, "MatVec: negative batch %d", batch);
    if (batch == 0) return WV_OK;
    DeviceState& dv = g_dev[b.device];
    float* sp = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        sp = dv.scratch;
    }
    if (!sp) return fail(WV_E_NODEV, "MatVec (no-alloc): device %d has no scratch (not initialised)", b.device);
    // Every partial the split kernels read was written earlier in the same
    // call, so the array needs no clearing between calls.
    const size_t need = matvec_scratch_floats(b, batch);
    if (need > kNoAllocScratchFloats)
        return fail(WV_E_SHAPE, "MatVec (no-alloc): rows=%lld cols=%lld needs %zu floats of scratch, the fixed array holds %zu",
                    (long long)b.rows, (long long)b.cols, need, kNoAllocScratchFloats);
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    // Calls on one stream are ordered by it. A call on another stream is
    // refused while the previous call's work may still be running, which is
    // the overlap that would share the array. Under graph capture nothing is
    // recorded or checked: the captured launches run when the graph does, and
    // their order is the caller's to keep.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) != hipSuccess) cap = hipStreamCaptureStatusNone;
    const bool capturing = cap != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> nl(dv.na_mu);
    if (!capturing && dv.na_pending && dv.na_stream != s) {
        const hipError_t q = hipEventQuery(dv.na_done);
        if (q == hipErrorNotReady)
            return fail(WV_E_BUSY, "MatVec (no-alloc): the previous call on device %d (another stream) is still running; "
                        "order the calls or use wv_matvec_dev", b.device);
        if (q != hipSuccess) return hip_fail(q, "MatVec (no-alloc): hipEventQuery");
    }
    const int e = launch_matvec(b, d_x, d_y, batch, s, need ? sp : nullptr);
    if (e != hipSuccess) return hip_fail(hipError_t(e), "MatVec (no-alloc): kernel launch");
    if (!capturing) {
        const hipError_t r = hipEventRecord(dv.na_done, s);
        if (r != hipSuccess) return hip_fail(r, "MatVec (no-alloc): hipEventRecord");
        dv.na_stream = s;
        dv.na_pending = true;
    }
    return WV_OK;
}

int wv_native_acc_dev(uint64_t handle, const float* d_x, int32_t* d_acc, float* d_act_scale, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "native acc: unknown handle %llu", (unsigned long long)handle);
    if (b.layout != LAYOUT_NARROW)
        return fail(WV_E_FORMAT, "native acc: blob is %s, not an Int8/Int4/Int2/Ternary/Binary store", fmt_name(b.fmt));
    if (!d_x || !d_acc) return fail(WV_E_ARG, "native acc: nil x/acc");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "native acc: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    const int e = launch_narrow_acc(b, d_x, d_acc, d_act_scale, batch, stream_or_default(stream, b.device));
    if (e != hipSuccess) return hip_fail(hipError_t(e), "native acc: kernel launch");
    return WV_OK;
}

int wv_matvec_t_dev(uint64_t handle, const float* d_gy, float* d_gx, int32_t batch, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVecT: unknown handle %llu", (unsigned long long)handle);
    if (!d_gy || !d_gx) return fail(WV_E_ARG, "MatVecT: nil gy/gx");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "MatVecT: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    CallScratch sc;
    int rc = sc.get(matvec_t_scratch_floats(b, batch), s, "MatVecT: scratch");
    if (rc) return rc;
    const int k = launch_matvec_t(b, d_gy, d_gx, batch, s, sc.f());
    if (k != hipSuccess) return hip_fail(hipError_t(k), "MatVecT: kernel launch");
    return WV_OK;
}

int wv_matmul_dev(uint64_t handle, const float* d_x, float* d_y, int32_t m, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatMul: unknown handle %llu", (unsigned long long)handle);
    if (!d_x || !d_y) return fail(WV_E_ARG, "MatMul: nil x/y");
    if (m < 0) return fail(WV_E_ARG, "MatMul: negative row count %d", m);
    if (m == 0) return WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    const bool gemm = gemm_supported(b, m);
    CallScratch sc;
    int rc = sc.get(gemm ? gemm_scratch_floats(b, m) : matvec_scratch_floats(b, m), s, "MatMul: scratch");
    if (rc) return rc;
    const int k = gemm ? launch_gemm(b, d_x, d_y, m, s, sc.f()) : launch_matvec(b, d_x, d_y, m, s, sc.f());
    if (k != hipSuccess) return hip_fail(hipError_t(k), "MatMul: kernel launch");
    return WV_OK;
}

int wv_matmul(uint64_t handle, const float* x, float* y, int32_t m) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatMul: unknown handle %llu", (unsigned long long)handle);
    if (!x || !y) return fail(WV_E_ARG, "MatMul: nil x/y");
    if (m <= 0) return m < 0 ? fail(WV_E_ARG, "MatMul: negative row count %d", m) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    Staging st(s);
    float* dx = st.in(x, size_t(m) * size_t(b.cols));
    float* dy = st.out(size_t(m) * size_t(b.rows));
    int rc = st.rc("MatMul: staging");
    if (!rc) rc = wv_matmul_dev(handle, dx, dy, m, s);
    if (!rc) rc = st.back(y, dy, size_t(m) * size_t(b.rows), "MatMul: copy y");
    return st.finish(rc, "MatMul: sync");
}

int wv_matvec(uint64_t handle, const float* x, float* y, int32_t batch) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVec: unknown handle %llu", (unsigned long long)handle);
    if (!x || !y) return fail(WV_E_ARG, "MatVec: nil x/y");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "MatVec: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    Staging st(s);
    float* dx = st.in(x, size_t(batch) * size_t(b.cols));
    float* dy = st.out(size_t(batch) * size_t(b.rows));
    int rc = st.rc("MatVec: staging");
    if (!rc) rc = wv_matvec_dev(handle, dx, dy, batch, s);
    if (!rc) rc = st.back(y, dy, size_t(batch) * size_t(b.rows), "MatVec: copy y");
    return st.finish(rc, "MatVec: sync");
}

int wv_matvec_t(uint64_t handle, const float* gy, float* gx, int32_t batch) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVecT: unknown handle %llu", (unsigned long long)handle);
    if (!gy || !gx) return fail(WV_E_ARG, "MatVecT: nil gy/gx");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "MatVecT: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    Staging st(s);
    float* dg = st.in(gy, size_t(batch) * size_t(b.rows));
    float* dx = st.in(gx, size_t(batch) * size_t(b.cols));
    int rc = st.rc("MatVecT: staging");
    if (!rc) rc = wv_matvec_t_dev(handle, dg, dx, batch, s);
    if (!rc) rc = st.back(gx, dx, size_t(batch) * size_t(b.cols), "MatVecT: copy out");
    return st.finish(rc, "MatVecT: sync");
}

int wv_quant_matvec(uint64_t handle, const float* x, size_t len_x, float* y, size_t len_y) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVec: nil blob");
    if (b.layout == LAYOUT_NARROW)
        return fail(WV_E_FORMAT, "quant: MatVec not implemented for %s (native path TBD — no QAT fallback)", fmt_name(b.fmt));
    if (int64_t(len_x) < b.cols || int64_t(len_y) < b.rows)  // checkBlobYX (quant/helpers.go:94-103)
        return fail(WV_E_SHAPE, "MatVec: size mismatch rows=%lld cols=%lld len(x)=%zu len(y)=%zu", (long long)b.rows,
                    (long long)b.cols, len_x, len_y);
    if (!x || !y) return fail(WV_E_ARG, "MatVec: nil x/y");
    return wv_matvec(handle, x, y, 1);
}

int wv_matvec_packed_blob(uint64_t handle, const float* x, size_t len_x, float* y, size_t len_y) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "dense: nil packed blob");
    if (int64_t(len_x) < b.cols || int64_t(len_y) < b.rows) return fail(WV_E_SHAPE, "dense: packed matvec shape");
    // The format switch (layers/dense/simd.go:579-613) has a case for every
    // packed format; FormatNone (and a Store's narrow DTypes, which are
    // FormatNone blobs there) falls through to the default error.
    if (b.layout == LAYOUT_F32 || b.layout == LAYOUT_NARROW)
        return fail(WV_E_FORMAT, "dense: MatVecPackedBlob unsupported none");
    if (!x || !y) return fail(WV_E_ARG, "dense: nil x/y");
    return wv_matvec(handle, x, y, 1);
}

int wv_quant_matvec_t(uint64_t handle, const float* gy, size_t len_gy, float* gx, size_t len_gx) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "MatVecT: nil blob");
    if (b.layout == LAYOUT_NARROW)
        return fail(WV_E_FORMAT, "quant: MatVecT not implemented for %s (native path TBD — no QAT fallback)", fmt_name(b.fmt));
    if (int64_t(len_gy) < b.rows || int64_t(len_gx) < b.cols)  // checkBlobGYGX (quant/helpers.go:105-114)
        return fail(WV_E_SHAPE, "MatVecT: size mismatch rows=%lld cols=%lld len(gy)=%zu len(gx)=%zu", (long long)b.rows,
                    (long long)b.cols, len_gy, len_gx);
    if (!gy || !gx) return fail(WV_E_ARG, "MatVecT: nil gy/gx");
    return wv_matvec_t(handle, gy, gx, 1);
}

int wv_dense_forward_dev(uint64_t handle, const float* d_x, float* d_pre, float* d_post, int32_t batch,
                         const double* d_bias, int32_t act, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "dense: unknown handle %llu", (unsigned long long)handle);
    if (!d_x || !d_pre) return fail(WV_E_ARG, "dense: nil layer/input");
    if (!act_valid(act)) return fail(WV_E_ARG, "dense: activation %d is not a core.ActivationType", act);
    if (!d_post && (d_bias || act != ACT_LINEAR))
        return fail(WV_E_ARG, "dense: a bias or a non-linear activation needs a post buffer");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "dense: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    CallScratch sc;
    int rc = sc.get(matvec_scratch_floats(b, batch), s, "dense: scratch");
    if (rc) return rc;
    BiasAct ba;
    ba.bias = d_bias;
    ba.act = act;
    ba.post = d_post;
    const int e = launch_matvec(b, d_x, d_pre, batch, s, sc.f(), d_post ? &ba : nullptr);
    if (e != hipSuccess) return hip_fail(hipError_t(e), "dense: kernel launch");
    return WV_OK;
}

// Host-pointer form of a dense forward entry point: stage x (and the bias),
// run `dev` on the device stream, copy pre (and post) back.
static int dense_forward_host(uint64_t handle, const float* x, float* pre, float* post, int32_t batch,
                              const double* bias, int32_t act,
                              int (*dev)(uint64_t, const float*, float*, float*, int32_t, const double*, int32_t, void*)) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "dense: unknown handle %llu", (unsigned long long)handle);
    if (!x || !pre) return fail(WV_E_ARG, "dense: nil layer/input");
    if (batch <= 0) return batch < 0 ? fail(WV_E_SHAPE, "dense: negative batch %d", batch) : WV_OK;
    (void)hipSetDevice(b.device);
    hipStream_t s = g_dev[b.device].stream;
    const size_t n = size_t(batch) * size_t(b.rows);
    Staging st(s);
    float* dx = st.in(x, size_t(batch) * size_t(b.cols));
    float* dpre = st.out(n);
    float* dpost = post ? st.out(n) : nullptr;
    const double* dbias = bias ? st.in(bias, size_t(b.rows)) : nullptr;
    int rc = st.rc("dense: staging");
    if (!rc) rc = dev(handle, dx, dpre, dpost, batch, dbias, act, s);
    if (!rc) rc = st.back(pre, dpre, n, "dense: copy pre");
    if (!rc && post) rc = st.back(post, dpost, n, "dense: copy post");
    return st.finish(rc, "dense: sync");
}

int wv_dense_forward(uint64_t handle, const float* x, float* pre, float* post, int32_t batch, const double* bias,
                     int32_t act) {
    return dense_forward_host(handle, x, pre, post, batch, bias, act, wv_dense_forward_dev);
}

int wv_dense_forward_block_dev(uint64_t handle, const float* d_x, float* d_pre, float* d_post, int32_t batch,
                               const double* d_bias, int32_t act, void* stream) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "dense: unknown handle %llu", (unsigned long long)handle);
    if (batch <= 0 || !gemm_supported(b, batch))  // the GEMV path, with its own checks
        return wv_dense_forward_dev(handle, d_x, d_pre, d_post, batch, d_bias, act, stream);
    if (!d_x || !d_pre) return fail(WV_E_ARG, "dense: nil layer/input");
    if (!act_valid(act)) return fail(WV_E_ARG, "dense: activation %d is not a core.ActivationType", act);
    if (!d_post && (d_bias || act != ACT_LINEAR))
        return fail(WV_E_ARG, "dense: a bias or a non-linear activation needs a post buffer");
    (void)hipSetDevice(b.device);
    hipStream_t s = stream_or_default(stream, b.device);
    CallScratch sc;
    int rc = sc.get(gemm_scratch_floats(b, batch), s, "dense: scratch");
    if (rc) return rc;
    int e = launch_gemm(b, d_x, d_pre, batch, s, sc.f());
    if (e == hipSuccess && d_post) e = launch_bias_act(d_pre, d_pre, d_post, d_bias, act, b.rows, batch, s);
    if (e != hipSuccess) return hip_fail(hipError_t(e), "dense: kernel launch");
    return WV_OK;
}

int wv_dense_forward_block(uint64_t handle, const float* x, float* pre, float* post, int32_t batch, const double* bias,
                           int32_t act) {
    return dense_forward_host(handle, x, pre, post, batch, bias, act, wv_dense_forward_block_dev);
}

int wv_store_matvec(uint64_t handle, const double* x, size_t len_x, double* y, size_t len_y) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "weights: nil");
    if ((len_x && !x) || (len_y && !y)) return fail(WV_E_ARG, "weights: nil x/y");
    if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32) {
        if (int64_t(len_x) < b.cols || int64_t(len_y) < b.rows) return fail(WV_E_SHAPE, "weights: matvecF64 shape");
        (void)hipSetDevice(b.device);
        hipStream_t s = g_dev[b.device].stream;
        Staging st(s);
        double* dx = st.in(x, size_t(b.cols));
        double* dy = st.out<double>(size_t(b.rows));
        int rc = st.rc("weights: staging");
        if (!rc) {
            const int e = launch_store_f64(b, dx, dy, s);
            if (e != hipSuccess) rc = hip_fail(hipError_t(e), "weights: kernel launch");
        }
        if (!rc) rc = st.back(y, dy, size_t(b.rows), "weights: copy y");
        rc = st.finish(rc, "weights: sync");
        if (!rc) std::fill(y + b.rows, y + len_y, 0.0);  // MatVec[T] returns its whole zeroed y buffer (store.go:133-145)
        return rc;
    }
    // Packed: quant.MatVec on f32 copies, then widen every entry (weights/store.go:162-180).
    std::vector<float> xf(len_x), yf(len_y, 0.0f);
    for (size_t i = 0; i < len_x; ++i) xf[i] = float(x[i]);
    const int rc = wv_quant_matvec(handle, xf.data(), len_x, yf.data(), len_y);
    if (rc) return rc;
    for (size_t i = 0; i < len_y; ++i) y[i] = double(yf[i]);
    return WV_OK;
}

int wv_store_matvec_t(uint64_t handle, const double* gy, size_t len_gy, double* gx, size_t len_gx) {
    DevBlob b;
    if (!lookup(handle, b)) return fail(WV_E_HANDLE, "weights: nil");
    if ((len_gy && !gy) || (len_gx && !gx)) return fail(WV_E_ARG, "weights: nil gy/gx");
    if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32) {
        if (int64_t(len_gy) < b.rows || int64_t(len_gx) < b.cols) return fail(WV_E_SHAPE, "weights: matvecTF64 shape");
        (void)hipSetDevice(b.device);
        hipStream_t s = g_dev[b.device].stream;
        Staging st(s);
        double* dg = st.in(gy, size_t(b.rows));
        double* dx = st.in(gx, size_t(b.cols));
        double* part = st.out<double>(std::max<size_t>(1, store_t_scratch_floats(b) / 2));
        int rc = st.rc("weights: staging");
        if (!rc) {
            const int e = launch_store_t_f64(b, dg, dx, s, part);
            if (e != hipSuccess) rc = hip_fail(hipError_t(e), "weights: kernel launch");
        }
        if (!rc) rc = st.back(gx, dx, size_t(b.cols), "weights: copy gx");
        return st.finish(rc, "weights: sync");
    }
    // Packed: quant.MatVecT on f32 copies of gy and gx, then widen gx (weights/store.go:182-206).
    std::vector<float> gyf(len_gy), gxf(len_gx);
    for (size_t i = 0; i < len_gy; ++i) gyf[i] = float(gy[i]);
    for (size_t i = 0; i < len_gx; ++i) gxf[i] = float(gx[i]);
    const int rc = wv_quant_matvec_t(handle, gyf.data(), len_gy, gxf.data(), len_gx);
    if (rc) return rc;
    for (size_t i = 0; i < len_gx; ++i) gx[i] = double(gxf[i]);
    return WV_OK;
}

int wv_sync(void* stream) {
    int rc = ensure_init();
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(stream_or_default(stream, g_current));
    if (e != hipSuccess) return hip_fail(e, "wv_sync");
    return WV_OK;
}

}  // extern "C"
