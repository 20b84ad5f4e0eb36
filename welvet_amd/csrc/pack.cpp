// pack.cpp — host-side packers of the C ABI: quant.Pack (quant/pack.go:4) and
// the DTypeTernary Store pack (weights/native.go:249-267).
//
// These produce the exact bytes welvet's Go packers produce, so a blob packed
// here and a blob packed by the Go side are interchangeable on upload. Each
// block / super-block is independent, so blocks are packed on a pool of
// std::threads. Built with -ffp-contract=off: every float expression rounds
// per operation like Go's float32 arithmetic on amd64.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

#include "wv_internal.h"

namespace wv {
namespace {

// math.Round: half away from zero (quant/helpers.go:151-153).
inline long go_round(double v) { return std::lround(v); }
inline long clampl(long v, long lo, long hi) { return v < lo ? lo : (v > hi ? hi : v); }
inline float fabs32(float v) { return v < 0 ? -v : v; }
inline void store_f32(uint8_t* p, float v) { std::memcpy(p, &v, 4); }

// Runs fn(lo, hi) over [0, n) split into contiguous ranges on worker threads.
void parallel_blocks(int64_t n, const std::function<void(int64_t, int64_t)>& fn) {
    unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    int64_t workers = std::min<int64_t>(hw, std::max<int64_t>(1, n / 4096));
    if (workers <= 1) { fn(0, n); return; }
    std::vector<std::thread> th;
    int64_t chunk = (n + workers - 1) / workers;
    for (int64_t w = 0; w < workers; ++w) {
        int64_t lo = w * chunk, hi = std::min(n, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back(fn, lo, hi);
    }
    for (auto& t : th) t.join();
}

// LSB-first bit sink over a byte range (quant/helpers.go:116-133).
struct BitSink {
    uint8_t* buf;
    int64_t pos = 0;
    void put(uint32_t v, int bits) {
        for (int i = 0; i < bits; ++i, ++pos)
            if ((v >> i) & 1u) buf[pos >> 3] |= uint8_t(1u << (pos & 7));
    }
};

struct Range {  // weights [s, e) of one block, e clipped to n
    int64_t s, e;
};
inline Range block_range(int64_t b, int64_t bs, int64_t n) { return {b * bs, std::min(n, b * bs + bs)}; }

float range_maxabs(const float* w, Range r) {
    float m = 0;
    for (int64_t i = r.s; i < r.e; ++i) m = std::max(m, fabs32(w[i]));  // helpers.go:60-69
    return m;
}
void range_minmax(const float* w, Range r, float& mn, float& mx) {  // helpers.go:71-85
    if (r.s >= r.e) { mn = mx = 0; return; }
    mn = mx = w[r.s];
    for (int64_t i = r.s + 1; i < r.e; ++i) { mn = w[i] < mn ? w[i] : mn; mx = w[i] > mx ? w[i] : mx; }
}
float range_absmean(const float* w, Range r) {  // helpers.go:49-58
    if (r.e <= r.s) return 0;
    float s = 0;
    for (int64_t i = r.s; i < r.e; ++i) s += fabs32(w[i]);
    return s / float(r.e - r.s);
}

// ---- classic 32-weight blocks ----

// Q4_0 (quant/q4_0.go:10-45, quantNibble :142-154).
void pack_q4_0(const float* w, int64_t n, uint8_t* raw) {
    parallel_blocks((n + 31) / 32, [&](int64_t lo, int64_t hi) {
        for (int64_t b = lo; b < hi; ++b) {
            Range r = block_range(b, 32, n);
            float scale = range_maxabs(w, r) / 7;
            if (scale == 0) scale = 1;
            uint8_t* o = raw + b * 20;
            store_f32(o, scale);
            auto nib = [&](int64_t i) -> int {
                if (i >= n) return 0;
                return int(clampl(go_round(double(w[i] / scale)), -8, 7));
            };
            for (int j = 0; j < 16; ++j)
                o[4 + j] = uint8_t((nib(r.s + 2 * j) & 0xF) | ((nib(r.s + 2 * j + 1) & 0xF) << 4));
        }
    });
}

// Q8_0 (quant/q8_0.go:8-44).
void pack_q8_0(const float* w, int64_t n, uint8_t* raw) {
    parallel_blocks((n + 31) / 32, [&](int64_t lo, int64_t hi) {
        for (int64_t b = lo; b < hi; ++b) {
            Range r = block_range(b, 32, n);
            float scale = range_maxabs(w, r) / 127;
            if (scale == 0) scale = 1;
            uint8_t* o = raw + b * 36;
            store_f32(o, scale);
            for (int j = 0; j < 32; ++j) {
                int64_t i = r.s + j;
                long q = i < n ? clampl(go_round(double(w[i]) / double(scale)), -127, 127) : 0;
                o[4 + j] = uint8_t(int8_t(q));
            }
        }
    });
}

// Asymmetric 32-blocks: Q4_1 (quant/q4_1.go:8-49) and Q5_1 (quant/q5_1.go:8-47).
void pack_asym32(const float* w, int64_t n, uint8_t* raw, int qmax, int bytes_per_block, bool five_bit) {
    parallel_blocks((n + 31) / 32, [&](int64_t lo, int64_t hi) {
        for (int64_t b = lo; b < hi; ++b) {
            Range r = block_range(b, 32, n);
            float mn, mx;
            range_minmax(w, r, mn, mx);
            float scale = (mx - mn) / float(qmax);
            if (scale == 0) scale = 1;
            uint8_t* o = raw + b * bytes_per_block;
            store_f32(o, scale);
            store_f32(o + 4, mn);
            uint32_t q[32];
            for (int j = 0; j < 32; ++j) {
                int64_t i = r.s + j;
                q[j] = 0;
                if (i < n) {
                    float t = (w[i] - mn) / scale;
                    q[j] = uint32_t(clampl(go_round(double(t)), 0, qmax));
                }
            }
            if (five_bit) {
                BitSink bs{o + 8};
                for (int j = 0; j < 32; ++j) bs.put(q[j], 5);
            } else {
                for (int j = 0; j < 16; ++j) o[8 + j] = uint8_t(q[2 * j] | (q[2 * j + 1] << 4));
            }
        }
    });
}

// Q5_0 (quant/q5_0.go:8-45): stored code q+16 in [0,31].
void pack_q5_0(const float* w, int64_t n, uint8_t* raw) {
    parallel_blocks((n + 31) / 32, [&](int64_t lo, int64_t hi) {
        for (int64_t b = lo; b < hi; ++b) {
            Range r = block_range(b, 32, n);
            float scale = range_maxabs(w, r) / 15;
            if (scale == 0) scale = 1;
            uint8_t* o = raw + b * 24;
            store_f32(o, scale);
            BitSink bs{o + 4};
            for (int j = 0; j < 32; ++j) {
                int64_t i = r.s + j;
                long q = i < n ? clampl(go_round(double(w[i]) / double(scale)) + 16, 0, 31) : 16;
                bs.put(uint32_t(q), 5);
            }
        }
    });
}

// ---- k-quant super-blocks (quant/kquant.go:62-176) ----
void pack_k(const KSpec& sp, const float* w, int64_t n, uint8_t* raw) {
    const int64_t sbb = k_super_bytes(sp);
    parallel_blocks((n + 255) / 256, [&](int64_t lo, int64_t hi) {
        for (int64_t si = lo; si < hi; ++si) {
            const int64_t base = si * 256;
            float gscale[16], gmin[16];
            uint32_t qs[256] = {0};
            for (int g = 0; g < 16; ++g) {
                Range r{base + g * 16, std::min(n, base + g * 16 + 16)};
                gmin[g] = 0;
                if (r.s >= n) { gscale[g] = 1; continue; }  // kquant.go:86-89
                if (sp.has_dmin) {
                    float mn, mx;
                    range_minmax(w, r, mn, mx);
                    float sc = (mx - mn) / float(sp.qmax);
                    if (sc == 0) sc = 1;
                    gmin[g] = mn;
                    gscale[g] = sc;
                    for (int j = 0; j < 16; ++j) {
                        int64_t i = r.s + j;
                        if (i < n) {
                            float t = (w[i] - mn) / sc;
                            qs[g * 16 + j] = uint32_t(clampl(go_round(double(t)), 0, sp.qmax));
                        }
                    }
                } else {
                    float sc = range_maxabs(w, r) / float(sp.mid);
                    if (sc == 0) sc = 1;
                    gscale[g] = sc;
                    for (int j = 0; j < 16; ++j) {
                        int64_t i = r.s + j;
                        long q = i < n ? clampl(go_round(double(w[i]) / double(sc)) + sp.mid, 0, sp.qmax) : sp.mid;
                        qs[g * 16 + j] = uint32_t(q);
                    }
                }
            }
            float d = 0, dmin = 0;
            for (int g = 0; g < 16; ++g) {
                d = gscale[g] > d ? gscale[g] : d;
                if (sp.has_dmin) dmin = fabs32(gmin[g]) > dmin ? fabs32(gmin[g]) : dmin;
            }
            if (d == 0) d = 1;
            if (sp.has_dmin && dmin == 0) dmin = 1;
            uint8_t* o = raw + si * sbb;
            store_f32(o, d);
            store_f32(o + 4, dmin);
            for (int g = 0; g < 16; ++g)
                o[8 + g] = uint8_t(clampl(go_round(double(gscale[g]) / double(d) * 255), 0, 255));
            int64_t qoff = 24;
            if (sp.has_dmin) {
                for (int g = 0; g < 16; ++g)
                    o[24 + g] = uint8_t(int8_t(dmin > 0 ? clampl(go_round(double(gmin[g]) / double(dmin) * 127), -127, 127) : 0));
                qoff = 40;
            }
            BitSink bs{o + qoff};
            for (int i = 0; i < 256; ++i) bs.put(qs[i], sp.bits);
        }
    });
}

// ---- IQ family (quant/iq.go:70-167) ----
// Groups are independent but share one bit stream; group s starts at bit
// s*sg*bits, which is byte aligned for every spec (sg*bits is 16..128), so
// groups can be packed in parallel.
void pack_iq(const IQSpec& sp, const float* w, int64_t n, uint8_t* raw, float* scales, uint8_t* meta) {
    const int64_t padn = (n + sp.sg - 1) / sp.sg * sp.sg, nsc = padn / sp.sg;
    const int qmax = (1 << sp.bits) - 1;
    parallel_blocks(nsc, [&](int64_t lo, int64_t hi) {
        for (int64_t s = lo; s < hi; ++s) {
            BitSink bs{raw + s * sp.sg * sp.bits / 8};
            Range r{s * sp.sg, std::min(n, s * sp.sg + sp.sg)};
            if (r.s >= n) {
                scales[s] = 1;
                continue;  // codes stay 0
            }
            float amax = range_maxabs(w, r);
            if (sp.nonlinear) {
                float scale = amax == 0 ? 1.0f : amax;
                scales[s] = scale;
                for (int j = 0; j < sp.sg; ++j) {
                    int64_t i = r.s + j;
                    int best = 0;
                    if (i < n) {
                        float target = w[i] / scale, best_err = 1e30f;
                        for (int c = 0; c < 16; ++c) {
                            float e = fabs32(kIQ4NLGrid[c] - target);
                            if (e < best_err) { best_err = e; best = c; }
                        }
                    }
                    bs.put(uint32_t(best), 4);
                }
                continue;
            }
            float scale;
            if (sp.bits == 1) {
                scale = amax;
            } else {
                float denom = float(qmax) - sp.mid;
                if (denom < 1) denom = 1;
                scale = amax / denom;
            }
            if (scale == 0) scale = 1;
            scales[s] = scale;
            for (int j = 0; j < sp.sg; ++j) {
                int64_t i = r.s + j;
                long q = 0;
                if (i < n) q = sp.bits == 1 ? (w[i] >= 0 ? 1 : 0)
                                            : clampl(go_round(double(w[i]) / double(scale) + double(sp.mid)), 0, qmax);
                bs.put(uint32_t(q), sp.bits);
            }
        }
    });
    meta[0] = uint8_t(sp.bits);
    meta[1] = uint8_t(sp.sg);
}

// ---- TernaryPacked (quant/ternary.go:11-51) / BinaryPacked (quant/binary.go:11-47) ----
void pack_ternary(const float* w, int64_t n, uint8_t* raw, float* scales) {
    parallel_blocks((n + 15) / 16, [&](int64_t lo, int64_t hi) {
        for (int64_t g = lo; g < hi; ++g) {
            Range r = block_range(g, 16, n);
            float scale = range_absmean(w, r);
            if (scale == 0) scale = 1;
            scales[g] = scale;
            uint32_t word = 0;
            for (int j = 0; j < 16; ++j) {
                int64_t i = r.s + j;
                uint32_t code = i < n ? uint32_t(clampl(go_round(double(w[i] / scale)), -1, 1) + 1) : 1u;
                word |= (code & 3u) << (2 * j);
            }
            std::memcpy(raw + g * 4, &word, 4);
        }
    });
}
void pack_binary(const float* w, int64_t n, uint8_t* raw, float* scales) {
    parallel_blocks((n + 31) / 32, [&](int64_t lo, int64_t hi) {
        for (int64_t g = lo; g < hi; ++g) {
            Range r = block_range(g, 32, n);
            float scale = range_absmean(w, r);
            if (scale == 0) scale = 1;
            scales[g] = scale;
            uint32_t word = 0;
            for (int j = 0; j < 32; ++j)
                if (r.s + j < n && w[r.s + j] >= 0) word |= 1u << j;
            std::memcpy(raw + g * 4, &word, 4);
        }
    });
}

// ---- AffinePacked (quant/affine_pack.go:15-86, BlobFromMLXAffine4 affine_g64.go:22-78) ----
// Groups of g along each row (cols % g == 0, so flat group gi starts at gi*g):
// f32 min/max, s = (max - min)/15 (0, NaN or Inf -> s = 1 and min = 0),
// code = round(f64(f32((v - min) * f32(1/s)))) clamped to [0, 15], eight codes
// per little-endian u32 LSB-first; Scales = s, Mins = min, Meta = {4}.
void pack_affine(const float* w, int64_t rows, int64_t cols, int g, uint8_t* raw, float* scales, float* mins,
                 uint8_t* meta) {
    parallel_blocks(rows * (cols / g), [&](int64_t lo, int64_t hi) {
        for (int64_t gi = lo; gi < hi; ++gi) {
            const float* v = w + gi * g;
            float mn = v[0], mx = v[0];
            for (int j = 1; j < g; ++j) {
                mn = v[j] < mn ? v[j] : mn;
                mx = v[j] > mx ? v[j] : mx;
            }
            float s = (mx - mn) / 15.0f;
            if (s == 0 || std::isnan(s) || std::isinf(s)) {
                s = 1;
                mn = 0;
            }
            scales[gi] = s;
            mins[gi] = mn;
            const float inv = 1 / s;
            for (int wi = 0; wi < g / 8; ++wi) {
                uint32_t word = 0;
                for (int j = 0; j < 8; ++j) {
                    const float t = (v[wi * 8 + j] - mn) * inv;
                    word |= uint32_t(clampl(go_round(double(t)), 0, 15)) << (4 * j);
                }
                std::memcpy(raw + (gi * g / 8 + wi) * 4, &word, 4);
            }
        }
    });
    meta[0] = 4;
}

}  // namespace

bool pack_sizes(int fmt, int64_t rows, int64_t cols, PackSizes& out) {
    out = PackSizes{};
    if (rows <= 0 || cols <= 0) return false;
    const int64_t n = rows * cols;
    KSpec ks;
    IQSpec is;
    switch (fmt) {
    case FMT_Q4_0: out.raw = (n + 31) / 32 * 20; out.block_weights = 32; return true;
    case FMT_Q8_0: out.raw = (n + 31) / 32 * 36; out.block_weights = 32; return true;
    case FMT_Q4_1: out.raw = (n + 31) / 32 * 24; out.block_weights = 32; return true;
    case FMT_Q5_0: out.raw = (n + 31) / 32 * 24; out.block_weights = 32; return true;
    case FMT_Q5_1: out.raw = (n + 31) / 32 * 28; out.block_weights = 32; return true;
    case FMT_TERNARY: out.raw = (n + 15) / 16 * 4; out.scales = (n + 15) / 16; out.block_weights = 16; return true;
    case FMT_BINARY: out.raw = (n + 31) / 32 * 4; out.scales = (n + 31) / 32; out.block_weights = 32; return true;
    case FMT_AFFINE:  // PackAffine4 with the default group of 64 (affine_pack.go:11-13)
        if (cols % 64) return false;
        out.raw = n / 2;
        out.scales = out.mins = n / 64;
        out.meta = 1;
        out.block_weights = 64;
        return true;
    default: break;
    }
    if (k_spec(fmt, ks)) { out.raw = (n + 255) / 256 * k_super_bytes(ks); out.block_weights = 256; return true; }
    if (iq_spec(fmt, is)) {
        int64_t padn = (n + is.sg - 1) / is.sg * is.sg;
        out.raw = (padn * is.bits + 7) / 8;
        out.scales = padn / is.sg;
        out.meta = 2;
        out.block_weights = 32;
        return true;
    }
    return false;
}

bool pack(int fmt, const float* w, int64_t rows, int64_t cols, uint8_t* raw, float* scales, float* mins,
          uint8_t* meta) {
    PackSizes sz;
    if (!pack_sizes(fmt, rows, cols, sz)) return false;
    const int64_t n = rows * cols;
    std::memset(raw, 0, size_t(sz.raw));
    KSpec ks;
    IQSpec is;
    switch (fmt) {
    case FMT_Q4_0: pack_q4_0(w, n, raw); return true;
    case FMT_Q8_0: pack_q8_0(w, n, raw); return true;
    case FMT_Q4_1: pack_asym32(w, n, raw, 15, 24, false); return true;
    case FMT_Q5_0: pack_q5_0(w, n, raw); return true;
    case FMT_Q5_1: pack_asym32(w, n, raw, 31, 28, true); return true;
    case FMT_TERNARY: pack_ternary(w, n, raw, scales); return true;
    case FMT_BINARY: pack_binary(w, n, raw, scales); return true;
    case FMT_AFFINE: pack_affine(w, rows, cols, 64, raw, scales, mins, meta); return true;
    default: break;
    }
    if (k_spec(fmt, ks)) { pack_k(ks, w, n, raw); return true; }
    if (iq_spec(fmt, is)) { pack_iq(is, w, n, raw, scales, meta); return true; }
    return false;
}

// weights/native.go:249-267 (absMax, weights/native.go:1160-1169).
// weights.Store packers of the narrow DTypes (weights/native.go:88-97 Int8,
// 180-194 packInt4, 218-230 packInt2, 249-269 packTernary, 271-283
// packBinary): scale = absMax (/127 Int8, /7 Int4), 1 when zero; codes
// LSB-first within bytes. `fmt` is FMT_NATIVE_*; false for other formats.
bool pack_native(int fmt, const float* w, int64_t n, uint8_t* codes, float* scale_out) {
    const int bits = narrow_bits(fmt);
    if (!bits) return false;
    float amax = 0;
    for (int64_t i = 0; i < n; ++i) amax = std::max(amax, float(std::fabs(double(w[i]))));
    float scale = fmt == FMT_NATIVE_INT8 ? amax / 127.0f : fmt == FMT_NATIVE_INT4 ? amax / 7.0f : amax;
    if (scale == 0) scale = 1;
    const int per = 8 / bits;
    // round-half-away(f64(f32(w / scale))) clamped (clampI, weights/native.go:1184-1192)
    auto qround = [&](float v, double lo, double hi) {
        const double r = std::round(double(v / scale));
        return int(r < lo ? lo : (r > hi ? hi : r));
    };
    parallel_blocks((n + per - 1) / per, [&](int64_t lo, int64_t hi) {
        for (int64_t b = lo; b < hi; ++b) {
            uint32_t v = 0;
            for (int k = 0; k < per && b * per + k < n; ++k) {
                const float x = w[b * per + k];
                uint32_t code = 0;
                switch (fmt) {
                case FMT_NATIVE_INT8: code = uint32_t(uint8_t(int8_t(qround(x, -128, 127)))); break;
                case FMT_NATIVE_INT4: code = uint32_t(qround(x, -8, 7)) & 0xFu; break;
                case FMT_NATIVE_INT2: code = uint32_t(qround(x, -2, 1) + 2) & 3u; break;
                case FMT_NATIVE_TERNARY: {
                    const float r = x / scale;
                    code = r > 0.5f ? 2u : (r < -0.5f ? 0u : 1u);
                    break;
                }
                default: code = x >= 0 ? 1u : 0u; break;  // Binary
                }
                v |= code << (bits * k);
            }
            codes[b] = uint8_t(v);
        }
    });
    *scale_out = scale;
    return true;
}

}  // namespace wv
