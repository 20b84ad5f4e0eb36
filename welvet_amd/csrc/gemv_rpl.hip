// gemv_rpl.hip — batch-1 dequant-GEMV on the row-interleaved ("one lane per
// output row") device layout, for Q4_K, Q6_K, Q8_0 and Q4_0.
//
// Layout (built at upload, same byte count as the reference blob): rows are
// taken 64 at a time (a row group = the 64 lanes of a wave); the codes of a
// 32-column chunk are stored lane-interleaved so the 64 lanes of one load read
// 1 KiB contiguous. Q4_K stores a super-block's 8 chunks of one row group
// next to each other, [rg][sb][j][lane][16 B], so the wave that owns the
// super-block streams one contiguous 8 KiB run; the other formats store the
// planes chunk-step-major, [j][rg][sb][lane][CB] (rpl_chunk, rpl_strides).
// Per-super-block metadata is [rg][sb][lane][...].
//
// Work split: wave = (row group, super-block): 64 rows x 256 columns, i.e. 8
// chunks of 16 B per lane. A block holds W waves = W consecutive super-blocks
// of one row group; gridDim.y = ceil(nsb / W) blocks split K. Each wave keeps
// D chunks in flight (ring prefetch): issuing a whole slice at once makes every
// wave wait for its first chunk until late in the launch, because vector loads
// retire in issue order; a shallow ring keeps arrival and compute interleaved.
// Each wave stages its 256 x values in its own LDS slice (one float4 per
// lane, loaded ahead of the weights) and reads them back as wave-wide
// broadcasts. Partial row sums of the W waves meet in LDS; when K is split
// across blocks, each block writes its partial to a per-blob scratch row and
// a second launch (k_rpl_ksum) adds the partials in split order, so the
// result does not depend on arrival order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "wave_ops.h"
#include "wv_internal.h"

namespace wv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Streaming (non-temporal) loads: weights are read once per launch.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_stream(const uint2* p) {
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint32_t ld_stream(const uint32_t* p) { return __builtin_nontemporal_load(p); }

__device__ __forceinline__ float ub0(uint32_t v) { return float(v & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t v) { return float((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t v) { return float((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t v) { return float(v >> 24); }

// sum_k q_k x[k] over the 16 unsigned 4-bit codes of two words (code k of
// word w = nibble k). The nibbles are spread to bytes first; the asm barrier
// keeps the compiler from folding the mask into each byte extraction, so
// every byte converts with a single v_cvt_f32_ubyteN.
__device__ __forceinline__ float dot16_u4(uint32_t w0, uint32_t w1, const float* x) {
    uint32_t l0 = w0 & 0x0F0F0F0Fu, h0 = (w0 >> 4) & 0x0F0F0F0Fu;
    uint32_t l1 = w1 & 0x0F0F0F0Fu, h1 = (w1 >> 4) & 0x0F0F0F0Fu;
    asm("" : "+v"(l0), "+v"(h0), "+v"(l1), "+v"(h1));
    float a = ub0(l0) * x[0];
    a = fmaf(ub0(h0), x[1], a);
    a = fmaf(ub1(l0), x[2], a);
    a = fmaf(ub1(h0), x[3], a);
    a = fmaf(ub2(l0), x[4], a);
    a = fmaf(ub2(h0), x[5], a);
    a = fmaf(ub3(l0), x[6], a);
    a = fmaf(ub3(h0), x[7], a);
    a = fmaf(ub0(l1), x[8], a);
    a = fmaf(ub0(h1), x[9], a);
    a = fmaf(ub1(l1), x[10], a);
    a = fmaf(ub1(h1), x[11], a);
    a = fmaf(ub2(l1), x[12], a);
    a = fmaf(ub2(h1), x[13], a);
    a = fmaf(ub3(l1), x[14], a);
    a = fmaf(ub3(h1), x[15], a);
    return a;
}
// sum_k q_k x[k] over 4 unsigned byte codes.
__device__ __forceinline__ float dot4_u8(uint32_t w, const float* x, float a) {
    a = fmaf(ub0(w), x[0], a);
    a = fmaf(ub1(w), x[1], a);
    a = fmaf(ub2(w), x[2], a);
    a = fmaf(ub3(w), x[3], a);
    return a;
}

// Per-format pieces. Ch = one chunk's codes for one lane; Sb = one
// super-block's metadata for one lane; dot() = this lane's row partial for
// chunk j (0..7) of the super-block, given x[32] and the two 16-column sums.
struct RplQ4K {  // w = dmin*m/127 + (d*u/255)*q  (quant/kquant.go:178-188)
    static constexpr bool kIntX = false;
    static constexpr bool kWords2 = false;  // a second metadata word per chunk (block min)
    struct Ch { uint4 c; };
    struct Sb { uint4 g0, g1; float d255, dm127; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        return {ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane)};
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 2;
        const float2 dd = reinterpret_cast<const float2*>(a.dd)[si * 64 + lane];
        return {ld_stream(m), ld_stream(m + 1), dd.x * (1.0f / 255.0f), dd.y * (1.0f / 127.0f)};
    }
    // Chunk j's metadata word, and an Sb whose chunk-0 word is w (lets a
    // kernel pick a word per lane and call dot with j = 0).
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) {
        const uint32_t gw[8] = {sb.g0.x, sb.g0.y, sb.g0.z, sb.g0.w, sb.g1.x, sb.g1.y, sb.g1.z, sb.g1.w};
        return gw[j];
    }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.g0.x = w;
        return sb;
    }
    static __device__ __forceinline__ float dot(const Ch& ch, const Sb& sb, int j, const float* x, float s0, float s1) {
        const uint32_t gw[8] = {sb.g0.x, sb.g0.y, sb.g0.z, sb.g0.w, sb.g1.x, sb.g1.y, sb.g1.z, sb.g1.w};
        const uint32_t g = gw[j];  // (u'0, u'1, m0, m1) bytes
        const float a0 = dot16_u4(ch.c.x, ch.c.y, x), a1 = dot16_u4(ch.c.z, ch.c.w, x + 16);
        const float m0 = float(int8_t(g >> 16)), m1 = float(int32_t(g) >> 24);
        return fmaf(sb.d255, fmaf(ub1(g), a1, ub0(g) * a0), sb.dm127 * fmaf(m1, s1, m0 * s0));
    }
};

// Q4_K with x held as 24-bit fixed point (X = round(x * 2^s), s per
// 32-column chunk, |X| < 2^22) split into three byte planes X = X0 + 2^8 X1 +
// 2^16 X2 (X0, X1 unsigned, X2 signed). The 4-bit codes multiply the planes
// with packed-dot v_dot4 instructions; sum_j q_j X_j is exact in int32
// (|.| < 16*15*2^22 < 2^31) and is converted to f32 once per 16-column group.
// The fixed-point step adds at most 2^-23 of the chunk's max |x| per element.
struct RplQ4KI : RplQ4K {
    static constexpr bool kIntX = true;
    // xi: 24 dwords [plane][lo w0..3 | hi w0..3], xm = (2^-s/255, sum0, sum1, -128*(sum0+sum1))
    static __device__ __forceinline__ float dot_i(const Ch& ch, const Sb& sb, int j, const uint32_t* xi, float4 xm) {
        const uint32_t gw[8] = {sb.g0.x, sb.g0.y, sb.g0.z, sb.g0.w, sb.g1.x, sb.g1.y, sb.g1.z, sb.g1.w};
        const uint32_t g = gw[j];
        const uint32_t wd[4] = {ch.c.x, ch.c.y, ch.c.z, ch.c.w};
        int A[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int gi = w >> 1;
            const uint32_t lo = wd[w] & 0x0F0F0F0Fu, hi = (wd[w] >> 4) & 0x0F0F0F0Fu;
            A[gi][0] = int(__builtin_amdgcn_udot4(lo, xi[w], uint32_t(A[gi][0]), false));
            A[gi][0] = int(__builtin_amdgcn_udot4(hi, xi[4 + w], uint32_t(A[gi][0]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(lo, xi[8 + w], uint32_t(A[gi][1]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(hi, xi[12 + w], uint32_t(A[gi][1]), false));
            A[gi][2] = __builtin_amdgcn_sdot4(int(lo), int(xi[16 + w]), A[gi][2], false);
            A[gi][2] = __builtin_amdgcn_sdot4(int(hi), int(xi[20 + w]), A[gi][2], false);
        }
        const int T0 = A[0][0] + (A[0][1] << 8) + (A[0][2] << 16);
        const int T1 = A[1][0] + (A[1][1] << 8) + (A[1][2] << 16);
        // (float)(int8)m = ub(m ^ 0x80) - 128; the -128 terms are folded into xm.w.
        // The group sums stay floats: a NaN or infinite x (which the fixed-point
        // planes would turn into a finite value) makes this term, and so the
        // row, non-finite, as the reference's float arithmetic does.
        const uint32_t gx = g ^ 0x80800000u;
        const float mn = fmaf(ub3(gx), xm.z, fmaf(ub2(gx), xm.y, xm.w));
        const float sc = sb.d255 * 255.0f * xm.x;  // d * 2^-s / 255
        return fmaf(sc, fmaf(ub1(g), float(T1), ub0(g) * float(T0)), sb.dm127 * mn);
    }
};

// Q2_K, Q3_K and Q5_K with the int-dot x planes of RplQ4KI. A chunk's codes
// are rebuilt as the 8 spread words of Q4_K (spread word s = 2*word + half
// holds, in byte b, the code of column 8*(s/2) + 2b + s%2), from:
//   B = 5: the low nibbles as in Q4_K, plus a 32-bit plane whose byte b holds
//          at bit s the fifth bit of that code: ((h >> s) & 0x01010101) << 4;
//   B = 2, 3: a 64-bit plane of the low two bits, dword s/4 holding at bits
//          2(s%4)..2(s%4)+1 of byte b the code of spread word s, plus for
//          B = 3 the third bits as B = 5's fifth bits, shifted by 2.
// Codes reach 2^B - 1 <= 31: a 16-column group sum stays below
// 16*31*2^22 < 2^31, exact in int32.
template <int B>
struct RplKxI : RplQ4KI {
    struct Ch { uint4 c; uint32_t h; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        Ch r;
        if constexpr (B == 5) {
            r.c = ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane);
        } else {
            const uint2 v = ld_stream(reinterpret_cast<const uint2*>(a.codes) + ci * 64 + lane);
            r.c = make_uint4(v.x, v.y, 0u, 0u);
        }
        r.h = B == 2 ? 0u : ld_stream(reinterpret_cast<const uint32_t*>(a.hi) + ci * 64 + lane);
        return r;
    }
    // spread word s of the chunk (s a compile-time constant after unrolling)
    static __device__ __forceinline__ uint32_t spread(const Ch& ch, int s) {
        const uint32_t wd[4] = {ch.c.x, ch.c.y, ch.c.z, ch.c.w};
        if constexpr (B == 5) {
            const uint32_t nib = (s & 1) ? (wd[s >> 1] >> 4) & 0x0F0F0F0Fu : wd[s >> 1] & 0x0F0F0F0Fu;
            return nib | (((ch.h >> s) & 0x01010101u) << 4);
        } else {
            const uint32_t lo2 = (wd[s >> 2] >> (2 * (s & 3))) & 0x03030303u;
            if constexpr (B == 2) return lo2;
            else return lo2 | (((ch.h >> s) & 0x01010101u) << 2);
        }
    }
    static __device__ __forceinline__ float dot_i(const Ch& ch, const Sb& sb, int j, const uint32_t* xi, float4 xm) {
        const uint32_t gw[8] = {sb.g0.x, sb.g0.y, sb.g0.z, sb.g0.w, sb.g1.x, sb.g1.y, sb.g1.z, sb.g1.w};
        const uint32_t g = gw[j];
        int A[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int gi = w >> 1;
            const uint32_t lo = spread(ch, 2 * w), hi = spread(ch, 2 * w + 1);
            A[gi][0] = int(__builtin_amdgcn_udot4(lo, xi[w], uint32_t(A[gi][0]), false));
            A[gi][0] = int(__builtin_amdgcn_udot4(hi, xi[4 + w], uint32_t(A[gi][0]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(lo, xi[8 + w], uint32_t(A[gi][1]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(hi, xi[12 + w], uint32_t(A[gi][1]), false));
            A[gi][2] = __builtin_amdgcn_sdot4(int(lo), int(xi[16 + w]), A[gi][2], false);
            A[gi][2] = __builtin_amdgcn_sdot4(int(hi), int(xi[20 + w]), A[gi][2], false);
        }
        const int T0 = A[0][0] + (A[0][1] << 8) + (A[0][2] << 16);
        const int T1 = A[1][0] + (A[1][1] << 8) + (A[1][2] << 16);
        const uint32_t gx = g ^ 0x80800000u;
        const float mn = fmaf(ub3(gx), xm.z, fmaf(ub2(gx), xm.y, xm.w));
        const float sc = sb.d255 * 255.0f * xm.x;
        return fmaf(sc, fmaf(ub1(g), float(T1), ub0(g) * float(T0)), sb.dm127 * mn);
    }
};

// The 32-weight block formats with the int-dot x planes: Q4_0 (XR = 0x8...8:
// the signed nibble q becomes q + 8, OFF = 8), Q5_0 (stored q + 16, OFF =
// 16), Q4_1 and Q5_1 (MIN: w = min + scale*q). Per chunk (one block) the
// metadata holds the f32 scale and, with MIN, the f32 min: words j and 8 + j
// of the lane's 16-word super-block record. Codes are spread as in RplKxI
// (B = 5 adds the fifth-bit plane); the two 16-column group sums stay exact
// in int32 and are added as floats.
template <int B, bool MIN, int OFF, uint32_t XR, int GSH = 0>
struct RplB32I {
    // GSH: chunk j's scale (and min) is group j >> GSH of the super-block
    // (AffinePacked with 32-, 64-, 128-, 256-column groups: GSH = 0..3); NG
    // groups, the mins follow the scales.
    static constexpr int NG = 8 >> GSH, NW = MIN ? 2 * NG : NG;
    static constexpr bool kIntX = true;
    static constexpr bool kWords2 = MIN;
    struct Ch { uint4 c; uint32_t h; };
    struct Sb { uint4 s0, s1, m0, m1; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        Ch r;
        r.c = ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane);
        r.h = B == 5 ? ld_stream(reinterpret_cast<const uint32_t*>(a.hi) + ci * 64 + lane) : 0u;
        return r;
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        Sb r;
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (NW == 2) {  // one scale and one min per super-block
            const uint2 v = ld_stream(reinterpret_cast<const uint2*>(a.meta) + si * 64 + lane);
            r.s0 = make_uint4(v.x, v.y, 0u, 0u);
            r.s1 = r.m0 = r.m1 = z;
            return r;
        }
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * (NW / 4);
        r.s0 = ld_stream(m);
        r.s1 = NW >= 8 ? ld_stream(m + 1) : z;
        r.m0 = NW >= 12 ? ld_stream(m + 2) : z;
        r.m1 = NW >= 16 ? ld_stream(m + 3) : z;
        return r;
    }
    static __device__ __forceinline__ uint32_t sw(const Sb& sb, int k) {
        const uint32_t w[16] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w,
                                sb.m0.x, sb.m0.y, sb.m0.z, sb.m0.w, sb.m1.x, sb.m1.y, sb.m1.z, sb.m1.w};
        return w[k];
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) { return sw(sb, j >> GSH); }
    static __device__ __forceinline__ uint32_t word2(const Sb& sb, int j) { return sw(sb, NG + (j >> GSH)); }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.s0.x = w;
        return sb;
    }
    static __device__ __forceinline__ Sb with_word2(Sb sb, uint32_t w) {  // the slot word2(sb, 0) reads: word NG
        if constexpr (NG == 8) sb.m0.x = w;
        else if constexpr (NG == 4) sb.s1.x = w;
        else if constexpr (NG == 2) sb.s0.z = w;
        else sb.s0.y = w;
        return sb;
    }
    static __device__ __forceinline__ uint32_t spread(const Ch& ch, int s) {
        const uint32_t wd[4] = {ch.c.x ^ XR, ch.c.y ^ XR, ch.c.z ^ XR, ch.c.w ^ XR};
        const uint32_t nib = (s & 1) ? (wd[s >> 1] >> 4) & 0x0F0F0F0Fu : wd[s >> 1] & 0x0F0F0F0Fu;
        if constexpr (B == 5) return nib | (((ch.h >> s) & 0x01010101u) << 4);
        else return nib;
    }
    static __device__ __forceinline__ float dot_i(const Ch& ch, const Sb& sb, int j, const uint32_t* xi, float4 xm) {
        int A[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int gi = w >> 1;
            const uint32_t lo = spread(ch, 2 * w), hi = spread(ch, 2 * w + 1);
            A[gi][0] = int(__builtin_amdgcn_udot4(lo, xi[w], uint32_t(A[gi][0]), false));
            A[gi][0] = int(__builtin_amdgcn_udot4(hi, xi[4 + w], uint32_t(A[gi][0]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(lo, xi[8 + w], uint32_t(A[gi][1]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(hi, xi[12 + w], uint32_t(A[gi][1]), false));
            A[gi][2] = __builtin_amdgcn_sdot4(int(lo), int(xi[16 + w]), A[gi][2], false);
            A[gi][2] = __builtin_amdgcn_sdot4(int(hi), int(xi[20 + w]), A[gi][2], false);
        }
        const int T0 = A[0][0] + (A[0][1] << 8) + (A[0][2] << 16);
        const int T1 = A[1][0] + (A[1][1] << 8) + (A[1][2] << 16);
        const float scale = __uint_as_float(word(sb, j));
        const float S = xm.y + xm.z;  // sum of the chunk's 32 x
        const float bias = MIN ? __uint_as_float(word2(sb, j)) : -float(OFF) * scale;
        return fmaf(scale * (xm.x * 255.0f), float(T0) + float(T1), bias * S);
    }
};
using RplQ4I = RplB32I<4, false, 8, 0x88888888u>;
using RplQ41I = RplB32I<4, true, 0, 0u>;
using RplQ50I = RplB32I<5, false, 16, 0u>;
using RplQ51I = RplB32I<5, true, 0, 0u>;
template <int GSH>
using RplAffI = RplB32I<4, true, 0, 0u, GSH>;  // AffinePacked, 32 << GSH-column groups: w = scale*code + min

// The linear IQ formats at their default code width and scale group
// (quant/iq.go:49-68, 169-180): w = scale*(q - mid), and for one-bit codes
// w = +-scale = (2*scale)*(q - 1/2). Planes as RplKxI (B = 2, 3) or Q4_K's
// nibbles (B = 4); one-bit codes sit in a 32-bit plane arranged as the
// fifth bits of Q5_K. Scales come from the blob's Scales array: one f32 per
// chunk (scale group 32), two (group 16, words 2j and 2j + 1), or one per
// 2^GSH chunks (BinaryPacked g128: GSH = 2, two words per super-block).
template <int B, bool SG16, int MID2, int GSH = 0>
struct RplIQI {
    static constexpr int kBits = B;
    static constexpr bool kIntX = true;
    static constexpr bool kWords2 = SG16;
    static constexpr int kGsh = GSH;
    static constexpr int NW = SG16 ? 16 : (8 >> GSH);  // metadata words per lane and super-block
    static constexpr float kMid = 0.5f * MID2;
    static constexpr float kScaleMul = B == 1 ? 2.0f : 1.0f;  // +-scale = (2*scale)*(q - 1/2)
    struct Ch { uint4 c; uint32_t h; };
    struct Sb { uint4 s0, s1, m0, m1; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        Ch r{};
        if constexpr (B == 4) {
            r.c = ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane);
        } else if constexpr (B >= 2) {
            const uint2 v = ld_stream(reinterpret_cast<const uint2*>(a.codes) + ci * 64 + lane);
            r.c = make_uint4(v.x, v.y, 0u, 0u);
        } else {
            r.c = make_uint4(ld_stream(reinterpret_cast<const uint32_t*>(a.codes) + ci * 64 + lane), 0u, 0u, 0u);
        }
        r.h = B == 3 ? ld_stream(reinterpret_cast<const uint32_t*>(a.hi) + ci * 64 + lane) : 0u;
        return r;
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        Sb r;
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (NW == 2) {
            const uint2 v = ld_stream(reinterpret_cast<const uint2*>(a.meta) + si * 64 + lane);
            r.s0 = make_uint4(v.x, v.y, 0u, 0u);
            r.s1 = r.m0 = r.m1 = z;
            return r;
        }
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * (NW / 4);
        r.s0 = ld_stream(m);
        r.s1 = ld_stream(m + 1);
        if constexpr (SG16) {
            r.m0 = ld_stream(m + 2);
            r.m1 = ld_stream(m + 3);
        } else {
            r.m0 = r.m1 = z;
        }
        return r;
    }
    static __device__ __forceinline__ uint32_t sw(const Sb& sb, int k) {
        const uint32_t w[16] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w,
                                sb.m0.x, sb.m0.y, sb.m0.z, sb.m0.w, sb.m1.x, sb.m1.y, sb.m1.z, sb.m1.w};
        return w[k];
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) { return sw(sb, SG16 ? 2 * j : (j >> GSH)); }
    static __device__ __forceinline__ uint32_t word2(const Sb& sb, int j) { return sw(sb, 2 * j + 1); }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.s0.x = w;
        return sb;
    }
    static __device__ __forceinline__ Sb with_word2(Sb sb, uint32_t w) {
        sb.s0.y = w;
        return sb;
    }
    static __device__ __forceinline__ uint32_t spread(const Ch& ch, int s) {
        const uint32_t wd[4] = {ch.c.x, ch.c.y, ch.c.z, ch.c.w};
        if constexpr (B == 4) {
            return (s & 1) ? (wd[s >> 1] >> 4) & 0x0F0F0F0Fu : wd[s >> 1] & 0x0F0F0F0Fu;
        } else if constexpr (B == 1) {
            return (ch.c.x >> s) & 0x01010101u;
        } else {
            const uint32_t lo2 = (wd[s >> 2] >> (2 * (s & 3))) & 0x03030303u;
            if constexpr (B == 2) return lo2;
            else return lo2 | (((ch.h >> s) & 0x01010101u) << 2);
        }
    }
    // the chunk's group scales (doubled for one-bit codes)
    static __device__ __forceinline__ float2 scales(const Sb& sb, int j) {
        const float s0 = __uint_as_float(word(sb, j)) * kScaleMul;
        const float s1 = SG16 ? __uint_as_float(word2(sb, j)) * kScaleMul : s0;
        return make_float2(s0, s1);
    }
    static __device__ __forceinline__ float dot_i(const Ch& ch, const Sb& sb, int j, const uint32_t* xi, float4 xm) {
        int A[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int gi = w >> 1;
            const uint32_t lo = spread(ch, 2 * w), hi = spread(ch, 2 * w + 1);
            A[gi][0] = int(__builtin_amdgcn_udot4(lo, xi[w], uint32_t(A[gi][0]), false));
            A[gi][0] = int(__builtin_amdgcn_udot4(hi, xi[4 + w], uint32_t(A[gi][0]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(lo, xi[8 + w], uint32_t(A[gi][1]), false));
            A[gi][1] = int(__builtin_amdgcn_udot4(hi, xi[12 + w], uint32_t(A[gi][1]), false));
            A[gi][2] = __builtin_amdgcn_sdot4(int(lo), int(xi[16 + w]), A[gi][2], false);
            A[gi][2] = __builtin_amdgcn_sdot4(int(hi), int(xi[20 + w]), A[gi][2], false);
        }
        const int T0 = A[0][0] + (A[0][1] << 8) + (A[0][2] << 16);
        const int T1 = A[1][0] + (A[1][1] << 8) + (A[1][2] << 16);
        const float2 sc = scales(sb, j);
        const float sx = xm.x * 255.0f;
        return fmaf(sx * sc.x, float(T0), fmaf(sx * sc.y, float(T1), -kMid * fmaf(sc.x, xm.y, sc.y * xm.z)));
    }
};
using RplIQ1S = RplIQI<1, false, 1>;
using RplBin128 = RplIQI<1, false, 1, 2>;  // BinaryPacked g128: +-scale per 128 weights
using RplIQ2XXS = RplIQI<2, false, 3>;
using RplIQ2XS = RplIQI<2, true, 3>;
using RplIQ3XXS = RplIQI<3, false, 7>;
using RplIQ3S = RplIQI<3, true, 7>;
using RplIQ4XS = RplIQI<4, true, 15>;
// TernaryPacked (quant/ternary.go:53-62): codes 0/1/2 -> -s/0/+s per 16 weights,
// i.e. s*(q - 1); the layout stores code 3 (also 0) as 1.
using RplTernI = RplIQI<2, true, 2>;

struct RplQ6K {  // q = lo4 | hi2 << 4, w = (d*u/255)*(q - 32)
    static constexpr bool kIntX = false;
    static constexpr bool kWords2 = false;  // a second metadata word per chunk (block min)
    struct Ch { uint4 c; uint2 h; };
    struct Sb { uint4 g; float d255; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        return {ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane),
                ld_stream(reinterpret_cast<const uint2*>(a.hi) + ci * 64 + lane)};
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        return {ld_stream(reinterpret_cast<const uint4*>(a.meta) + si * 64 + lane), reinterpret_cast<const float*>(a.dd)[(si * 64 + lane) * 2] * (1.0f / 255.0f)};
    }
    // 8 codes of code word w; the high-bit plane holds, in byte b of dword t,
    // at bits 2f..2f+1, the top bits of the code in byte b of spread word
    // s = 4t + f (s = 2*word + nibble half).
    static __device__ __forceinline__ float dot8(uint32_t w, uint32_t h, int f0, const float* x) {
        uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * f0)) & 0x03030303u) << 4);
        uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * f0 + 2)) & 0x03030303u) << 4);
        asm("" : "+v"(lo), "+v"(hi));
        float a = ub0(lo) * x[0];
        a = fmaf(ub0(hi), x[1], a);
        a = fmaf(ub1(lo), x[2], a);
        a = fmaf(ub1(hi), x[3], a);
        a = fmaf(ub2(lo), x[4], a);
        a = fmaf(ub2(hi), x[5], a);
        a = fmaf(ub3(lo), x[6], a);
        a = fmaf(ub3(hi), x[7], a);
        return a;
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) {
        const uint32_t gw[4] = {sb.g.x, sb.g.y, sb.g.z, sb.g.w};
        return gw[j >> 1] >> (16 * (j & 1));
    }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.g.x = w;
        return sb;
    }
    static __device__ __forceinline__ float dot(const Ch& ch, const Sb& sb, int j, const float* x, float s0, float s1) {
        const uint32_t gw[4] = {sb.g.x, sb.g.y, sb.g.z, sb.g.w};
        const uint32_t g = gw[j >> 1] >> (16 * (j & 1));  // (u'0, u'1) bytes
        const float a0 = dot8(ch.c.x, ch.h.x, 0, x) + dot8(ch.c.y, ch.h.x, 2, x + 8);
        const float a1 = dot8(ch.c.z, ch.h.y, 0, x + 16) + dot8(ch.c.w, ch.h.y, 2, x + 24);
        return sb.d255 * fmaf(ub1(g), fmaf(-32.0f, s1, a1), ub0(g) * fmaf(-32.0f, s0, a0));
    }
};

struct RplQ8 {  // w = scale * q, q int8; q + 128 converts as an unsigned byte
    static constexpr bool kIntX = false;
    static constexpr bool kWords2 = false;  // a second metadata word per chunk (block min)
    struct Ch { uint4 c0, c1; };
    struct Sb { uint4 s0, s1; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        const uint4* p = reinterpret_cast<const uint4*>(a.codes) + (ci * 64 + lane) * 2;
        return {ld_stream(p), ld_stream(p + 1)};
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 2;
        return {ld_stream(m), ld_stream(m + 1)};
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) {
        const uint32_t sw[8] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w};
        return sw[j];
    }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.s0.x = w;
        return sb;
    }
    static __device__ __forceinline__ float dot(const Ch& ch, const Sb& sb, int j, const float* x, float s0, float s1) {
        const uint32_t sw[8] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w};
        const uint32_t B = 0x80808080u;
        uint32_t w[8] = {ch.c0.x ^ B, ch.c0.y ^ B, ch.c0.z ^ B, ch.c0.w ^ B, ch.c1.x ^ B, ch.c1.y ^ B, ch.c1.z ^ B, ch.c1.w ^ B};
        float a = -128.0f * (s0 + s1);
#pragma unroll
        for (int k = 0; k < 8; ++k) a = dot4_u8(w[k], x + 4 * k, a);
        return __uint_as_float(sw[j]) * a;
    }
};

struct RplQ4 {  // w = scale * q, q signed nibble; q ^ 8 = q + 8
    static constexpr bool kIntX = false;
    static constexpr bool kWords2 = false;  // a second metadata word per chunk (block min)
    struct Ch { uint4 c; };
    struct Sb { uint4 s0, s1; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        return {ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane)};
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 2;
        return {ld_stream(m), ld_stream(m + 1)};
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) {
        const uint32_t sw[8] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w};
        return sw[j];
    }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.s0.x = w;
        return sb;
    }
    static __device__ __forceinline__ float dot(const Ch& ch, const Sb& sb, int j, const float* x, float s0, float s1) {
        const uint32_t sw[8] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w};
        const uint32_t B = 0x88888888u;
        const float a = dot16_u4(ch.c.x ^ B, ch.c.y ^ B, x) + dot16_u4(ch.c.z ^ B, ch.c.w ^ B, x + 16);
        return __uint_as_float(sw[j]) * fmaf(-8.0f, s0 + s1, a);
    }
};

// IQ4_NL's grid (quant/iq.go:23-40) in LDS, one 16-float copy per wave of
// the block (rows of tab), written by the wave's lanes 0..15 and read only by
// that wave: a lookup is a broadcast ds_read_b32 from 16 consecutive words.
__device__ __forceinline__ float* iq4nl_tab() {
    __shared__ float tab[16 * 16];
    return tab;
}
// Byte offset of this wave's copy, after writing it. A wave's LDS accesses
// complete in issue order, so its later lookups see the copy.
__device__ __forceinline__ int iq4nl_fill_tab() {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane < 16) iq4nl_tab()[wave * 16 + lane] = kIQ4NLGrid[lane];
    return wave * 64;
}
// grid[nibble n of w], the wave's table at byte offset tb
__device__ __forceinline__ float iq4nl_at(uint32_t w, int n, int tb) {
    const uint32_t q4 = (n == 0 ? w << 2 : w >> (4 * n - 2)) & 0x3Cu;
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(iq4nl_tab()) + (q4 | uint32_t(tb)));
}

// IQ4_NL (quant/iq.go:169-180, nonlinear): w = scale * grid[q], one scale per
// 32-column chunk; the f32 x of the chunk meets the looked-up grid values.
// The super-block record carries the offset of the wave's grid table.
struct RplIQ4NL {
    static constexpr bool kIntX = false;
    static constexpr bool kWords2 = false;
    struct Ch { uint4 c; };
    struct Sb { uint4 s0, s1; int tb; };
    static __device__ __forceinline__ Ch load_ch(const RplArgs& a, int64_t ci, int lane) {
        return {ld_stream(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane)};
    }
    static __device__ __forceinline__ Sb load_sb(const RplArgs& a, int64_t si, int lane) {
        const uint4* m = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 2;
        return {ld_stream(m), ld_stream(m + 1), iq4nl_fill_tab()};
    }
    static __device__ __forceinline__ uint32_t word(const Sb& sb, int j) {
        const uint32_t sw[8] = {sb.s0.x, sb.s0.y, sb.s0.z, sb.s0.w, sb.s1.x, sb.s1.y, sb.s1.z, sb.s1.w};
        return sw[j];
    }
    static __device__ __forceinline__ Sb with_word(Sb sb, uint32_t w) {
        sb.s0.x = w;
        return sb;
    }
    static __device__ __forceinline__ float dot(const Ch& ch, const Sb& sb, int j, const float* x, float, float) {
        const uint32_t wd[4] = {ch.c.x, ch.c.y, ch.c.z, ch.c.w};
        float a0 = 0.f, a1 = 0.f;  // two chains: even and odd weights
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int n = 0; n < 8; n += 2) {
                a0 = fmaf(iq4nl_at(wd[i], n, sb.tb), x[8 * i + n], a0);
                a1 = fmaf(iq4nl_at(wd[i], n + 1, sb.tb), x[8 * i + n + 1], a1);
            }
        return __uint_as_float(word(sb, j)) * (a0 + a1);
    }
};

// Writes one output of the forward kernel under the launch's epilogue mode
// and returns the stored value.
__device__ __forceinline__ float store_y(const RplArgs& a, float* y, int64_t idx, float s) {
    if (a.mode == RPL_ADD) {
        s += y[idx];
    } else if (a.mode == RPL_SILU_MUL) {
        const float g = a.aux[idx];
        s *= g / (1.0f + expf(-g));
    }
    y[idx] = s;
    return s;
}

// Epilogue of one wave of output rows (all 64 lanes call it; lanes with
// `valid` own row `row`): store, and for a fused-RMSNorm producer the sums of
// the stored y^2 over each 16 consecutive rows ([batch][rg_count*4]).
__device__ __forceinline__ void finish_rows(const RplArgs& a, float* y, int b, int row, bool valid, int lane, float s) {
    if (a.mode == RPL_SWIGLU) {
        const float u = quad_xor1(s);
        if (valid && !(lane & 1) && row < a.rows) y[int64_t(b) * (a.rows / 2) + row / 2] = s / (1.0f + expf(-s)) * u;
        return;
    }
    float v = 0.f;
    if (valid && row < a.rows) v = store_y(a, y, int64_t(b) * a.rows + row, s);
    if (a.ss_out) {
        const float q = row_sum16(v * v);
        if (valid && (lane & 15) == 0) a.ss_out[int64_t(b) * a.rg_count * 4 + row / 16] = q;
    }
}

// L-way pick of a per-chunk metadata word: chunk base + lg (lg < L). The
// candidates pass through empty asm statements so that the compiler keeps the
// selects as v_cndmask: seen as elements of one vector, a per-lane index would
// become a dynamically indexed extract, which goes through scratch memory.
template <int L>
__device__ __forceinline__ uint32_t pick(const uint32_t* c, int lg) {
    if constexpr (L == 1) {
        return c[0];
    } else if constexpr (L == 2) {
        uint32_t c0 = c[0], c1 = c[1];
        asm("" : "+v"(c0), "+v"(c1));
        return (lg & 1) ? c1 : c0;
    } else {
        uint32_t c0 = c[0], c1 = c[1], c2 = c[2], c3 = c[3];
        asm("" : "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3));
        const uint32_t lo = (lg & 1) ? c1 : c0, hi = (lg & 1) ? c3 : c2;
        return (lg & 2) ? hi : lo;
    }
}

// The row-interleaved forward kernel.
//   Block (hx, ks, b): row group rg = hx / L, row subgroup h = hx % L (R = 64/L
//   rows), K slice ks, batch row b. W waves; wave w owns S consecutive
//   super-blocks starting at (ks*W + w)*S.
//   Lane = (lg, r) = (lane / R, lane % R): row rg*64 + h*R + r; lane group lg
//   takes chunks lg, lg+L, ... of each super-block, so one load instruction
//   reads L runs of R*16 bytes.
//   Per lane: T = S*8/L chunk steps, D of them in flight (ring).
// L > 1 splits a 64-row group over L blocks and S > 1 lets a wave cover more
// columns, so that shapes with few rows fill the GPU without a K split.
template <class P, int L, int S, int D>
__global__ void __launch_bounds__(1024) k_gemv_rpl(RplArgs a, const float* __restrict__ x, float* __restrict__ y) {
    constexpr int R = 64 / L;
    constexpr int CPL = 8 / L;    // chunks per super-block per lane
    constexpr int T = S * CPL;    // chunk steps per lane
    constexpr int DD = D < T ? D : T;
    extern __shared__ float4 sm4[];
    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int lg = lane / R, r = lane % R;
    const int hx = blockIdx.x, ks = blockIdx.y, b = blockIdx.z;
    const int rg = hx / L, h = hx % L;
    const int sl = h * R + r;  // this lane's row slot inside the row group
    const int sb0 = (ks * W + wave) * S;
    bool act[S];
    int64_t si[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        act[s] = sb0 + s < a.nsb;
        si[s] = int64_t(rg) * a.nsb + (act[s] ? sb0 + s : a.nsb - 1);
    }

    // x for the S super-blocks (one float4 per lane each), issued before the
    // weights so that waiting for x does not wait for weight data (vector
    // loads retire in issue order); then the metadata and the first chunks.
    float4 xv4[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
        xv4[s] = reinterpret_cast<const float4*>(x + int64_t(b) * a.nsb * 256 + (si[s] - int64_t(rg) * a.nsb) * 256)[lane];
    float4 gv4[S];
    // The producer's sum-of-squares partials: the first kSsU per lane are
    // loaded together here (clamped, masked to 0) and added after the weight
    // loads are issued, in the same order as one pass i = lane, lane+64, ...
    // S = 4 (wide K, never behind a norm in the decoder) sums them in one
    // loop here: eight more live registers would spill there.
    constexpr int kSsU = S >= 4 ? 0 : 8;
    float ssv[kSsU > 0 ? kSsU : 1];
    double ssp = 0.0;
    const float* ssb = a.nrm_ss + int64_t(b) * a.nrm_n;
    if (a.nrm_gamma) {
#pragma unroll
        for (int s = 0; s < S; ++s)
            gv4[s] = reinterpret_cast<const float4*>(a.nrm_gamma + (si[s] - int64_t(rg) * a.nsb) * 256)[lane];
        if constexpr (kSsU == 0) {
            for (int i = lane; i < a.nrm_n; i += 64) ssp += ssb[i];
        } else {
#pragma unroll
            for (int k = 0; k < kSsU; ++k) {
                const int i = lane + 64 * k;
                const float v = ssb[min(i, a.nrm_n - 1)];
                ssv[k] = i < a.nrm_n ? v : 0.f;
            }
        }
    }
    typename P::Sb sbm[S];
#pragma unroll
    for (int s = 0; s < S; ++s) sbm[s] = P::load_sb(a, si[s], sl);
    auto chunk_index = [&](int t) {  // plane index of step t's chunk for this lane
        const int s = t / CPL, j = lg + L * (t % CPL);
        return rpl_chunk(a, si[s], j);
    };
    typename P::Ch ch[T];
#pragma unroll
    for (int t = 0; t < DD; ++t) ch[t] = P::load_ch(a, chunk_index(t), sl);
    if (a.nrm_gamma) {
        // RMSNorm of x folded in (layers/rmsnorm/cpu.go:70-85): f64 total of
        // the producer's partial sums, y = f32((x * inv) * gamma).
        if constexpr (kSsU > 0) {
#pragma unroll
            for (int k = 0; k < kSsU; ++k) ssp += ssv[k];
            for (int i = lane + 64 * kSsU; i < a.nrm_n; i += 64) ssp += ssb[i];
        }
        ssp = wave_total_f64(ssp);
        const double inv = 1.0 / sqrt(ssp / double(a.nsb * 256) + a.nrm_eps);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            xv4[s].x = float(double(xv4[s].x) * inv * double(gv4[s].x));
            xv4[s].y = float(double(xv4[s].y) * inv * double(gv4[s].y));
            xv4[s].z = float(double(xv4[s].z) * inv * double(gv4[s].z));
            xv4[s].w = float(double(xv4[s].w) * inv * double(gv4[s].w));
        }
    }

    // Stage x in this wave's LDS slice (only this wave reads it, so a
    // wave-level LDS wait replaces a block barrier), one kSlice per super-block:
    //   f32 policies: [256 x][16 sums of 16 columns]
    //   int policies: per chunk 24 dwords of X byte planes + 4 floats meta
    constexpr int kSlice = 256 + 16;
    float* xw = reinterpret_cast<float*>(sm4) + wave * (S * kSlice);
    float* part = reinterpret_cast<float*>(sm4) + W * (S * kSlice);  // [W*64]
#pragma unroll
    for (int s = 0; s < S; ++s) {
        float* xs = xw + s * kSlice;
        const float4 xv = xv4[s];
        float gsum = (xv.x + xv.y) + (xv.z + xv.w);
        gsum += quad_xor1(gsum);
        gsum += quad_xor2(gsum);  // lanes 4g..4g+3: sum of columns 16g..16g+15
        if constexpr (!P::kIntX) {
            reinterpret_cast<float4*>(xs)[lane] = xv;
            if ((lane & 3) == 0) xs[256 + (lane >> 2)] = gsum;
        } else {
            // lane = 8c + q holds columns 4q..4q+3 of chunk c
            const int c = lane >> 3, q = lane & 7;
            float m = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
            m = fmaxf(m, quad_xor1(m));
            m = fmaxf(m, quad_xor2(m));
            m = fmaxf(m, half_mirror(m));  // max over lanes 8c..8c+7
            int e = 0;
            frexpf(m, &e);
            const int sh = m > 0.f ? 22 - e : 0;  // |x| * 2^sh < 2^22
            const int X0 = int(rintf(ldexpf(xv.x, sh))), X1 = int(rintf(ldexpf(xv.y, sh)));
            const int X2 = int(rintf(ldexpf(xv.z, sh))), X3 = int(rintf(ldexpf(xv.w, sh)));
            // code word w = q/2 covers columns 8w..8w+7; its lo spread word holds
            // columns 8w+{0,2,4,6}, its hi spread word 8w+{1,3,5,7}: this lane
            // supplies the byte pair at half (q & 1) of each.
            uint16_t* h16 = reinterpret_cast<uint16_t*>(xs + c * 28);
            const int w = q >> 1, half = q & 1;
#pragma unroll
            for (int pl = 0; pl < 3; ++pl) {
                // byte pl of X0 (X1) and of X2 (X3) in one v_perm_b32 each
                const uint32_t sel = uint32_t(pl) | (uint32_t(4 + pl) << 8) | 0x0C0C0000u;
                const uint32_t blo = __builtin_amdgcn_perm(uint32_t(X2), uint32_t(X0), sel);
                const uint32_t bhi = __builtin_amdgcn_perm(uint32_t(X3), uint32_t(X1), sel);
                h16[(pl * 8 + w) * 2 + half] = uint16_t(blo);
                h16[(pl * 8 + 4 + w) * 2 + half] = uint16_t(bhi);
            }
            // for q == 0: this quad's column sum and the other quad's (lanes 8c+4..8c+7)
            const float s0 = gsum, s1 = half_mirror(gsum);
            if (q == 0) {
                float* xm = xs + c * 28 + 24;
                xm[0] = ldexpf(1.0f, -sh) * (1.0f / 255.0f);
                xm[1] = s0;
                xm[2] = s1;
                xm[3] = -128.0f * (s0 + s1);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
        if (t + DD < T) ch[t + DD] = P::load_ch(a, chunk_index(t + DD), sl);
        __builtin_amdgcn_sched_barrier(0);
        const int s = t / CPL, jb = L * (t % CPL);  // chunk = jb + lg
        if (act[s]) {
            // this step's metadata word for chunk jb + lg, moved to slot 0
            typename P::Sb mv = sbm[s];
            int jsel = jb;
            if constexpr (L > 1) {
                uint32_t cand[L];
#pragma unroll
                for (int i = 0; i < L; ++i) cand[i] = P::word(sbm[s], jb + i);
                mv = P::with_word(sbm[s], pick<L>(cand, lg));
                if constexpr (P::kWords2) {
                    uint32_t cand2[L];
#pragma unroll
                    for (int i = 0; i < L; ++i) cand2[i] = P::word2(sbm[s], jb + i);
                    mv = P::with_word2(mv, pick<L>(cand2, lg));
                }
                jsel = 0;
            }
            const float* xs = xw + s * kSlice;
            const int j = jb + lg;
            if constexpr (P::kIntX) {
                const uint4* xq = reinterpret_cast<const uint4*>(xs + j * 28);
                uint32_t xi[24];
#pragma unroll
                for (int k = 0; k < 6; ++k) {
                    const uint4 tq = xq[k];
                    xi[4 * k] = tq.x;
                    xi[4 * k + 1] = tq.y;
                    xi[4 * k + 2] = tq.z;
                    xi[4 * k + 3] = tq.w;
                }
                acc += P::dot_i(ch[t], mv, jsel, xi, reinterpret_cast<const float4*>(xq)[6]);
            } else {
                const float4* xq = reinterpret_cast<const float4*>(xs + j * 32);
                float xv[32];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 tq = xq[k];
                    xv[4 * k] = tq.x;
                    xv[4 * k + 1] = tq.y;
                    xv[4 * k + 2] = tq.z;
                    xv[4 * k + 3] = tq.w;
                }
                const float2 s2 = reinterpret_cast<const float2*>(xs + 256)[j];
                acc += P::dot(ch[t], mv, jsel, xv, s2.x, s2.y);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // the L lane groups of a row hold partial sums of different chunks; a lane
    // swap with both operands equal is the xor-16 / xor-32 butterfly step
    if constexpr (R <= 16) acc = reduce_scatter16(acc, acc);
    if constexpr (R <= 32) acc = reduce_scatter32(acc, acc);
    part[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += part[w * 64 + lane];
    const int row = rg * 64 + sl;
    const bool valid = lane < R;
    if (a.ksplit == 1) {
        finish_rows(a, y, b, row, valid, lane, sum);
        return;
    }
    // K split across gridDim.y blocks: store the partial; k_rpl_ksum adds the
    // splits and applies the epilogue in a second launch.
    const int64_t rows_pad = int64_t(a.rg_count) * 64;
    if (valid) a.partial[(int64_t(b) * a.ksplit + ks) * rows_pad + row] = sum;
}

// k_gemv_q4k's x records: 32 dwords per chunk (24 of digit planes, 4 zero,
// then 2^-s and the two group sums), 8 to a wave's slice. A 40-dword stride,
// which puts the 32 dwords of one staging store in 32 distinct LDS banks
// (records 0, 2, 4 and 6 share banks at 32), ran the same.
constexpr int kQ4kRec = 32, kQ4kSlice = 8 * kQ4kRec + 16;

// Q4_K forward for the one-lane-per-row plan (L = 1, S = 1; the headline
// 4096->14336). Same layout and work split as k_gemv_rpl<RplQ4KI, 1, 1, 4>,
// the same 24-bit fixed-point x per 32-column chunk, and the same integer
// group dots, taken on the i8 matrix cores instead of v_dot4:
//   * x is staged as three signed digit planes (X = d0 + 256 d1 + 65536 d2),
//     the A operand of v_mfma_i32_32x32x32_i8; the codes, lane-swapped and
//     widened to bytes, are the B operand, so one MFMA gives 32 rows x 6
//     (plane, group) dots of a chunk and each step takes two chunks in four
//     MFMAs (about 62 VALU per two chunks against 108 with v_dot4);
//   * the chunk's codes are one contiguous 8 KiB run per super-block (Q4_K's
//     super-block-major order), addressed from one base with constant
//     offsets, and the wave is either active or not for its whole life (no
//     per-step activity test);
//   * the group scales meet T0, T1 as floats, P = u0*T0 + u1*T1, and the
//     chunk's fixed-point scale 2^-s multiplies P into a super-block
//     accumulator; d/255 is applied once per super-block;
//   * the mins accumulate as sum_g (m_g + 128)*S_g over the super-block (S_g
//     the 16-column sums of x), and the -128*sum(x) correction is taken once
//     from the wave's total of x.
// The integer dots are exact, so the rows equal the v_dot4 kernel's up to the
// association of the float sums.
__global__ void __launch_bounds__(1024) k_gemv_q4k(RplArgs a, const float* __restrict__ x, float* __restrict__ y) {
    extern __shared__ float4 sm4[];
    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int rg = blockIdx.x, ks = blockIdx.y, b = blockIdx.z;
    const int sb = ks * W + wave;
    const bool act = sb < a.nsb;
    const int sbc = act ? sb : a.nsb - 1;  // an idle wave reads a valid super-block and contributes 0
    const int64_t si = int64_t(rg) * a.nsb + sbc;

    // x first (vector loads retire in issue order), then the metadata and D chunks.
    constexpr int D = 4;
    const float4 xv0 = reinterpret_cast<const float4*>(x + (int64_t(b) * a.nsb + sbc) * 256)[lane];
    float4 gv = make_float4(1.f, 1.f, 1.f, 1.f);
    float ssv[8];
    const float* ssb = a.nrm_ss + int64_t(b) * a.nrm_n;
    if (a.nrm_gamma) {
        gv = reinterpret_cast<const float4*>(a.nrm_gamma + int64_t(sbc) * 256)[lane];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = lane + 64 * k;
            const float v = ssb[min(i, a.nrm_n - 1)];
            ssv[k] = i < a.nrm_n ? v : 0.f;
        }
    }
    const uint4* mp = reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 2;
    const uint4 g0 = ld_stream(mp), g1 = ld_stream(mp + 1);
    const float2 dd = reinterpret_cast<const float2*>(a.dd)[si * 64 + lane];
    const uint4* cp = reinterpret_cast<const uint4*>(a.codes) + si * 512 + lane;  // chunk t at cp + 64 t
    uint4 ch[8];
#pragma unroll
    for (int t = 0; t < D; ++t) ch[t] = ld_stream(cp + t * 64);

    float4 xv = xv0;
    if (a.nrm_gamma) {
        // RMSNorm of x folded in (layers/rmsnorm/cpu.go:70-85), as in k_gemv_rpl.
        double ssp = 0.0;
#pragma unroll
        for (int k = 0; k < 8; ++k) ssp += ssv[k];
        for (int i = lane + 512; i < a.nrm_n; i += 64) ssp += ssb[i];
        ssp = wave_total_f64(ssp);
        const double inv = 1.0 / sqrt(ssp / double(a.nsb * 256) + a.nrm_eps);
        xv.x = float(double(xv0.x) * inv * double(gv.x));
        xv.y = float(double(xv0.y) * inv * double(gv.y));
        xv.z = float(double(xv0.z) * inv * double(gv.z));
        xv.w = float(double(xv0.w) * inv * double(gv.w));
    }

    // Stage x in this wave's LDS slice, one kRec-dword record per chunk c: the
    // X digit planes as MFMA A-operand rows [plane][group][lo w0, w1 | hi w0, w1]
    // (16 bytes per plane and 16-column group), 4 zero dwords, then
    // (2^-s, s0, s1). The digits are signed: X = d0 + 256 d1 + 65536 d2 with
    // every d in [-128, 127], from the bytes of X + 0x808080 less 128 each.
    constexpr int kRec = kQ4kRec, kSlice = kQ4kSlice;
    float* xs = reinterpret_cast<float*>(sm4) + wave * kSlice;
    float* part = reinterpret_cast<float*>(sm4) + W * kSlice;
    const float lsum = (xv.x + xv.y) + (xv.z + xv.w);
    float gsum = lsum;
    gsum += quad_xor1(gsum);
    gsum += quad_xor2(gsum);  // lanes 4g..4g+3: sum of columns 16g..16g+15
    const float xtot = wave_total(lsum);
    {
        const int c = lane >> 3, q = lane & 7;  // lane = 8c + q holds columns 4q..4q+3 of chunk c
        float m = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
        m = fmaxf(m, quad_xor1(m));
        m = fmaxf(m, quad_xor2(m));
        m = fmaxf(m, half_mirror(m));
        int e = 0;
        frexpf(m, &e);
        const int sh = m > 0.f ? 22 - e : 0;  // |x| * 2^sh < 2^22
        constexpr int kBias = 0x808080;
        const int X0 = int(rintf(ldexpf(xv.x, sh))) + kBias, X1 = int(rintf(ldexpf(xv.y, sh))) + kBias;
        const int X2 = int(rintf(ldexpf(xv.z, sh))) + kBias, X3 = int(rintf(ldexpf(xv.w, sh))) + kBias;
        uint16_t* h16 = reinterpret_cast<uint16_t*>(xs + c * kRec);
        const int g = q >> 2, ew = (q >> 1) & 1, half = q & 1;  // code word 2g + ew of the chunk
#pragma unroll
        for (int pl = 0; pl < 3; ++pl) {
            const uint32_t sel = uint32_t(pl) | (uint32_t(4 + pl) << 8) | 0x0C0C0000u;
            const uint32_t blo = __builtin_amdgcn_perm(uint32_t(X2), uint32_t(X0), sel) ^ 0x8080u;
            const uint32_t bhi = __builtin_amdgcn_perm(uint32_t(X3), uint32_t(X1), sel) ^ 0x8080u;
            h16[((pl * 2 + g) * 4 + ew) * 2 + half] = uint16_t(blo);
            h16[((pl * 2 + g) * 4 + 2 + ew) * 2 + half] = uint16_t(bhi);
        }
        const float s1 = half_mirror(gsum);
        if (q == 0) {
            float* xm = xs + c * kRec + 28;
            xm[0] = ldexpf(1.0f, -sh);
            xm[1] = gsum;
            xm[2] = s1;
        }
        if (q == 1) *reinterpret_cast<uint4*>(xs + c * kRec + 24) = make_uint4(0u, 0u, 0u, 0u);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // Two chunks per step on v_mfma_i32_32x32x32_i8, D = X-planes x codes^T.
    // B: after a lane swap, lanes 0-31 hold rows 0-31 (or 32-63) with their
    // first 16-column group, lanes 32-63 the same rows' second group; the
    // nibbles widen to bytes. A: lane (i, h) = (l & 31, l >> 5) carries the
    // 16 digit bytes of plane p, group h of one chunk when row i of D is a
    // slot n = 6e + 3g + p with g = h, else zeros. Rows 0-3, 8-11, 16-19 take
    // the slots of rows 0-31 of the weights, rows 4-7, 12-15, 20-23 those of
    // rows 32-63, so after both MFMAs accumulator r of lane l is slot r of row l.
    const int ir = lane & 31;
    const int n = (ir >> 3) * 4 + (ir & 3);
    const int en = n / 6, gn = (n % 6) / 3, pn = n % 3, setn = (ir >> 2) & 1;
    const bool dlane = ir < 24 && gn == (lane >> 5);
    int ao[2][2];  // [weight rows 0-31 | 32-63][chunk of the pair]: dword offset in the record
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 2; ++e) ao[st][e] = (dlane && setn == st && en == e) ? (pn * 2 + gn) * 4 : 24;

    const uint32_t gw[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};  // (u'0, u'1, m0, m1) per chunk
    float pacc = 0.f, macc = 0.f;
#pragma unroll
    for (int t0 = 0; t0 < 8; t0 += 2) {
        if (t0 + D < 8) {
            ch[t0 + D] = ld_stream(cp + (t0 + D) * 64);
            ch[t0 + D + 1] = ld_stream(cp + (t0 + D + 1) * 64);
        }
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        i32x16 acc = {};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = t0 + e;
            const float* xr = xs + t * kRec;
            const i32x4 A0 = *reinterpret_cast<const i32x4*>(xr + ao[0][e]);
            const i32x4 A1 = *reinterpret_cast<const i32x4*>(xr + ao[1][e]);
            const auto ka = __builtin_amdgcn_permlane32_swap(ch[t].x, ch[t].z, false, false);
            const auto kb = __builtin_amdgcn_permlane32_swap(ch[t].y, ch[t].w, false, false);
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                const uint32_t wa = ka[T], wb = kb[T];
                const i32x4 Bt = {int(wa & 0x0F0F0F0Fu), int(wb & 0x0F0F0F0Fu), int((wa >> 4) & 0x0F0F0F0Fu),
                                  int((wb >> 4) & 0x0F0F0F0Fu)};
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(T == 0 ? A0 : A1, Bt, acc, 0, 0, 0);
            }
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = t0 + e;
            const int T0 = acc[6 * e] + acc[6 * e + 1] * 256 + acc[6 * e + 2] * 65536;
            const int T1 = acc[6 * e + 3] + acc[6 * e + 4] * 256 + acc[6 * e + 5] * 65536;
            const float4 xm = *reinterpret_cast<const float4*>(xs + t * kRec + 28);
            const uint32_t g = gw[t];
            const float P = fmaf(ub1(g), float(T1), ub0(g) * float(T0));
            pacc = fmaf(P, xm.x, pacc);
            // A NaN or infinite x reaches the row through these float group sums
            // (the fixed-point planes would turn it into a finite value).
            const uint32_t gx = g ^ 0x80800000u;  // bytes 2, 3: m + 128 as unsigned
            macc = fmaf(ub2(gx), xm.y, macc);
            macc = fmaf(ub3(gx), xm.z, macc);
        }
        asm volatile("" : "+v"(pacc), "+v"(macc));
        __builtin_amdgcn_sched_barrier(0);
    }
    // w = dmin*m/127 + (d*u/255)*q  (quant/kquant.go:178-188)
    float acc = fmaf(dd.x * (1.0f / 255.0f), pacc, (dd.y * (1.0f / 127.0f)) * fmaf(-128.0f, xtot, macc));
    if (!act) acc = 0.f;
    part[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    float sum = 0.f;
    for (int w = 0; w < W; ++w) sum += part[w * 64 + lane];
    const int row = rg * 64 + lane;
    if (a.ksplit == 1) {
        finish_rows(a, y, b, row, true, lane, sum);
        return;
    }
    const int64_t rows_pad = int64_t(a.rg_count) * 64;
    a.partial[(int64_t(b) * a.ksplit + ks) * rows_pad + row] = sum;
}

// Tail of a K-split forward launch: one wave per (64-row group, batch row)
// adds the ksplit partials in split order and applies the launch's epilogue.
// A last-arriving-block tail in the forward kernel instead costs more: its
// ticket and partials must bypass the caches, about 1.5 us per round trip on
// MI355X.
__global__ void __launch_bounds__(64) k_rpl_ksum(RplArgs a, float* __restrict__ y) {
    const int rg = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int64_t rows_pad = int64_t(a.rg_count) * 64;
    const int row = rg * 64 + lane;
    const float* p = a.partial + int64_t(b) * a.ksplit * rows_pad + row;
    // Each group of 8 loads (clamped to the last split, the extra ones masked
    // out of the sum) is issued before any add: one round trip for up to 8.
    float s = 0.f;
    for (int k = 0; k < a.ksplit; k += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p[int64_t(min(k + j, a.ksplit - 1)) * rows_pad];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (k + j < a.ksplit) s += v[j];
    }
    finish_rows(a, y, b, row, true, lane, s);
}

// Blocks a K-split plan aims for (measured on MI355X: fewer leave CUs idle).
constexpr int kRplMinBlocks = 200;

// Launch plan of the forward kernel: lanes per row L, super-blocks per wave
// S, waves per block W and K split (measured on MI355X):
//   * up to 16 super-blocks (K <= 4096): one wave per super-block, and L
//     doubles (to 4) until the grid (row groups x L) has >= 180 blocks; a lane
//     keeps >= 4 chunk steps, so L = 4 takes two super-blocks per wave.
//     4096x4096 runs in 5.1 us with L=4 S=2 against 7.2 us with L=1.
//   * wider, when 4 x (row groups) blocks of W = ceil(nsb / 4) waves fill the
//     GPU (>= 180) in one resident pass (<= 256 x floor(16 / W)): L = 4, S = 4
//     and no K split. 14336->4096 runs in 10.5 us against 11.0 us split 4
//     ways, 8192->4096 in 6.9 against 8.1; 14336->8192 (too many blocks)
//     takes 19.4 against 17.3.
//   * otherwise L = S = 1 and K split over blocks of W = 16..4 waves; W
//     prefers grids of >= min_blocks() blocks, then the fewest idle waves,
//     then the largest W, and the split is capped by the scratch the blob
//     carries.
struct RplPlan {
    int L, S, W, ksplit;
};
// max_s: the most super-blocks per wave whose metadata fits the registers
// (2 for the policies with a second metadata word: 4 spill at 128 VGPRs).
RplPlan rpl_plan(const DevBlob& bl, int max_s = 4) {
    const RplArgs& a = bl.rpl;
    RplPlan p{1, 1, 1, 1};
    const int max_split = std::max(1, (a.nsb + 3) / 4);  // K-split partials per row at most
    if (a.nsb <= 16) {
        while (p.L < 4 && int64_t(a.rg_count) * p.L < 180) p.L *= 2;
        if (p.L == 4 && a.nsb >= 2) p.S = 2;
    } else if (const int w4 = (a.nsb + 3) / 4;
               max_s >= 4 && w4 <= 16 && int64_t(a.rg_count) * 4 >= 180 && int64_t(a.rg_count) * 4 <= 256 * (16 / w4)) {
        // No K split: L = 4, S = 4, one block per 16-row subgroup covering
        // all of K, when those blocks fill the GPU in one resident pass.
        p.L = 4;
        p.S = 4;
        p.W = w4;
    } else {
        const int target = kRplMinBlocks;
        int best = -1;
        for (int w = 16; w >= 4; --w) {
            const int k = (a.nsb + w - 1) / w;
            if (k > max_split) continue;
            const bool fills = int64_t(a.rg_count) * k >= target;
            const int idle = k * w - a.nsb;
            const int score = (fills ? 1 << 20 : 0) + (1 << 10) * (64 - std::min(idle, 63)) + w;
            if (score > best) {
                best = score;
                p.W = w;
            }
        }
    }
    const int waves = (a.nsb + p.S - 1) / p.S;
    if (a.nsb <= 16) p.W = std::min(16, waves);
    p.W = std::min(p.W, waves);
    p.ksplit = (waves + p.W - 1) / p.W;
    return p;
}

// Policies with a second metadata word are planned with S <= 2 (rpl_plan's
// max_s; launch_rpl_t checks it), so their S = 4 kernels are not built.
template <class P, int L, int S>
void launch_rpl_ls(const RplArgs& a, const RplPlan& p, dim3 grid, size_t lds, hipStream_t s, const float* x, float* y) {
    if constexpr (!(P::kWords2 && S > 2))
        hipLaunchKernelGGL((k_gemv_rpl<P, L, S, 4>), grid, dim3(unsigned(64 * p.W)), lds, s, a, x, y);
}

template <class P>
int launch_rpl_t(const DevBlob& bl, const float* x, float* y, int batch, hipStream_t s, const RplExtra& ex) {
    RplArgs a = bl.rpl;
    const int mode = ex.mode;
    const float* aux = ex.aux;
    a.mode = mode;
    a.aux = aux;
    a.nrm_gamma = ex.nrm_gamma;
    a.nrm_ss = ex.nrm_ss;
    a.nrm_n = ex.nrm_n;
    a.nrm_eps = ex.nrm_eps;
    a.ss_out = ex.ss_out;
    a.partial = ex.partial;
    const RplPlan p = rpl_plan(bl, P::kWords2 ? 2 : 4);
    if (P::kWords2 && p.S > 2) return int(hipErrorInvalidValue);  // not reachable: the plan caps S
    if (p.ksplit > 1 && !a.partial) return int(hipErrorInvalidValue);  // the caller owes the split scratch
    a.ksplit = p.ksplit;
    const size_t lds = size_t(p.W) * (p.S * (256 + 16) + 64) * sizeof(float);  // x slices + partial row sums
    // A K-split launch carries kRplFwdBatch batch rows (the scratch holds their
    // partials; chunks run in stream order and reuse it); otherwise one launch.
    const int chunk = p.ksplit > 1 ? kRplFwdBatch : std::min(batch, 65535);
    for (int b0 = 0; b0 < batch; b0 += chunk) {
        const int nb = std::min(chunk, batch - b0);
        dim3 grid(unsigned(a.rg_count * p.L), unsigned(p.ksplit), unsigned(nb));
        RplArgs ab = a;
        if (aux) ab.aux = aux + int64_t(b0) * a.rows;
        if (ab.nrm_ss) ab.nrm_ss += int64_t(b0) * a.nrm_n;
        if (ab.ss_out) ab.ss_out += int64_t(b0) * a.rg_count * 4;
        const int64_t ystride = mode == RPL_SWIGLU ? a.rows / 2 : a.rows;
        const float* xb = x + int64_t(b0) * a.nsb * 256;
        float* yb = y + int64_t(b0) * ystride;
        if constexpr (std::is_same<P, RplQ4KI>::value) {
            // k_gemv_q4k takes 77 VGPRs, so one 16-wave block per CU: it runs
            // the grids that fit the GPU in one pass (the 4096->14336
            // headline, 224 blocks). Larger grids (the decoder's gate||up,
            // 448 blocks, and LM head, 500) keep the 64-VGPR policy kernel,
            // two blocks per CU.
            constexpr int64_t kCUs = 256;  // MI355X
            if (p.L == 1 && p.S == 1 && a.cs_si == 8 && a.cs_j == 1 && int64_t(grid.x) * grid.y * grid.z <= kCUs) {
                const size_t lq = size_t(p.W) * (kQ4kSlice + 64) * sizeof(float);
                hipLaunchKernelGGL(k_gemv_q4k, grid, dim3(unsigned(64 * p.W)), lq, s, ab, xb, yb);
                if (p.ksplit > 1)
                    hipLaunchKernelGGL(k_rpl_ksum, dim3(unsigned(a.rg_count), unsigned(nb)), dim3(64), 0, s, ab, yb);
                continue;
            }
        }
        switch (p.L * 8 + p.S) {
        case 9: launch_rpl_ls<P, 1, 1>(ab, p, grid, lds, s, xb, yb); break;
        case 10: launch_rpl_ls<P, 1, 2>(ab, p, grid, lds, s, xb, yb); break;
        case 12: launch_rpl_ls<P, 1, 4>(ab, p, grid, lds, s, xb, yb); break;
        case 17: launch_rpl_ls<P, 2, 1>(ab, p, grid, lds, s, xb, yb); break;
        case 18: launch_rpl_ls<P, 2, 2>(ab, p, grid, lds, s, xb, yb); break;
        case 20: launch_rpl_ls<P, 2, 4>(ab, p, grid, lds, s, xb, yb); break;
        case 33: launch_rpl_ls<P, 4, 1>(ab, p, grid, lds, s, xb, yb); break;
        case 34: launch_rpl_ls<P, 4, 2>(ab, p, grid, lds, s, xb, yb); break;
        default: launch_rpl_ls<P, 4, 4>(ab, p, grid, lds, s, xb, yb); break;
        }
        if (p.ksplit > 1) hipLaunchKernelGGL(k_rpl_ksum, dim3(unsigned(a.rg_count), unsigned(nb)), dim3(64), 0, s, ab, yb);
    }
    return int(hipGetLastError());
}

// ---------------------------------------------------------------------------
// gx += W^T gy on the row-interleaved layout (quant.MatVecT).
//
// Lane = row, as in the forward layout, so the sum over rows runs across
// lanes. A wave owns one chunk pair (64 columns) of one super-block and walks
// GP consecutive row groups, accumulating per-lane column partials in
// registers (acc[c] += coef_group(row) * ucode(row, c), plus one offset term
// per 16-column group: the k-quant min or the code bias). Only then does it
// reduce across lanes, with a reduce-scatter that leaves column l in lane l.
// A block is one 64-column group and one slice of W * GP row groups: its W
// waves add their columns in LDS in wave order, so when the column groups
// alone fill the GPU (one slice) the block adds its total to gx and no second
// pass runs. With several slices each block stores a partial [b][slice][cols]
// that a fixed-order pass adds to gx.
// ---------------------------------------------------------------------------

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// acc[0..7] += coef * (codes of an 8-column run): byte b of `lo` holds the
// code of column 2b, byte b of `hi` that of column 2b + 1. Codes below 16
// (kMix) become fp16 two at a time with v_cvt_scalef32_pk_f16_fp8 (a byte
// q < 16 read as fp8 e4m3 is q * 2^-9 exactly, and the scale 512 makes it
// q), and an fmaf of an fp16 code widened to f32 is one v_fma_mix_f32: the
// same single-rounding result as fmaf(float(q), coef, acc), in 12 VALU
// operations per 8 codes instead of 16. Wider codes go through
// v_cvt_f32_ubyte.
template <bool kMix>
__device__ __forceinline__ void tacc8(uint32_t lo, uint32_t hi, float coef, float* acc) {
    asm("" : "+v"(lo), "+v"(hi));
    if constexpr (kMix) {
        const half2v l01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, false);
        const half2v l23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 512.0f, true);
        const half2v h01 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, false);
        const half2v h23 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 512.0f, true);
        acc[0] = fmaf(float(l01.x), coef, acc[0]);
        acc[1] = fmaf(float(h01.x), coef, acc[1]);
        acc[2] = fmaf(float(l01.y), coef, acc[2]);
        acc[3] = fmaf(float(h01.y), coef, acc[3]);
        acc[4] = fmaf(float(l23.x), coef, acc[4]);
        acc[5] = fmaf(float(h23.x), coef, acc[5]);
        acc[6] = fmaf(float(l23.y), coef, acc[6]);
        acc[7] = fmaf(float(h23.y), coef, acc[7]);
    } else {
        acc[0] = fmaf(ub0(lo), coef, acc[0]);
        acc[1] = fmaf(ub0(hi), coef, acc[1]);
        acc[2] = fmaf(ub1(lo), coef, acc[2]);
        acc[3] = fmaf(ub1(hi), coef, acc[3]);
        acc[4] = fmaf(ub2(lo), coef, acc[4]);
        acc[5] = fmaf(ub2(hi), coef, acc[5]);
        acc[6] = fmaf(ub3(lo), coef, acc[6]);
        acc[7] = fmaf(ub3(hi), coef, acc[7]);
    }
}
// acc[2b], acc[2b+1] += coef * (nibbles 2b, 2b+1 of v), b = 0..3
__device__ __forceinline__ void tacc_nib(uint32_t v, float coef, float* acc) {
    tacc8<true>(v & 0x0F0F0F0Fu, (v >> 4) & 0x0F0F0F0Fu, coef, acc);
}
// acc[k] += coef * byte k of v
__device__ __forceinline__ void tacc_u8(uint32_t v, float coef, float* acc) {
    asm("" : "+v"(v));
    acc[0] = fmaf(ub0(v), coef, acc[0]);
    acc[1] = fmaf(ub1(v), coef, acc[1]);
    acc[2] = fmaf(ub2(v), coef, acc[2]);
    acc[3] = fmaf(ub3(v), coef, acc[3]);
}

// Per-format metadata of one chunk pair (jp) and the accumulate step for
// chunk jj of the pair. off[0..1] collect the per-group offsets.
struct TQ4K : RplQ4K {
    struct TM { uint2 g; float2 dd; };  // (u'0,u'1,m0,m1) bytes of chunks 2jp, 2jp+1
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        const uint2* m = reinterpret_cast<const uint2*>(a.meta) + (si * 64 + lane) * 4 + jp;
        const float2 dd = reinterpret_cast<const float2*>(a.dd)[si * 64 + lane];
        return {ld_stream(m), dd};
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const uint32_t g = jj ? t.g.y : t.g.x;
        const float gd = gy * (t.dd.x * (1.0f / 255.0f));
        const float c0 = gd * ub0(g), c1 = gd * ub1(g);
        const float gm = gy * (t.dd.y * (1.0f / 127.0f));
        off[0] = fmaf(gm, float(int8_t(g >> 16)), off[0]);
        off[1] = fmaf(gm, float(int32_t(g) >> 24), off[1]);
        tacc_nib(ch.c.x, c0, acc);
        tacc_nib(ch.c.y, c0, acc + 8);
        tacc_nib(ch.c.z, c1, acc + 16);
        tacc_nib(ch.c.w, c1, acc + 24);
    }
};

template <int B>
struct TKx : RplKxI<B> {
    using Ch = typename RplKxI<B>::Ch;
    using TM = TQ4K::TM;
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        return TQ4K::load_tm(a, si, lane, jp);
    }
    // the 8 codes of code word w (spread words 2w, 2w + 1), column order
    static __device__ __forceinline__ void tacc_w(const Ch& ch, int w, float coef, float* acc) {
        tacc8<(B <= 4)>(RplKxI<B>::spread(ch, 2 * w), RplKxI<B>::spread(ch, 2 * w + 1), coef, acc);
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const uint32_t g = jj ? t.g.y : t.g.x;
        const float gd = gy * (t.dd.x * (1.0f / 255.0f));
        const float c0 = gd * ub0(g), c1 = gd * ub1(g);
        const float gm = gy * (t.dd.y * (1.0f / 127.0f));
        off[0] = fmaf(gm, float(int8_t(g >> 16)), off[0]);
        off[1] = fmaf(gm, float(int32_t(g) >> 24), off[1]);
        tacc_w(ch, 0, c0, acc);
        tacc_w(ch, 1, c0, acc + 8);
        tacc_w(ch, 2, c1, acc + 16);
        tacc_w(ch, 3, c1, acc + 24);
    }
};

template <int B, bool MIN, int OFF, uint32_t XR, int GSH = 0>
struct TB32 : RplB32I<B, MIN, OFF, XR, GSH> {
    using P = RplB32I<B, MIN, OFF, XR, GSH>;
    using Ch = typename P::Ch;
    struct TM { uint2 s, m; };  // scales (and mins) of chunks 2jp, 2jp+1
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        const uint32_t* m = reinterpret_cast<const uint32_t*>(a.meta) + (si * 64 + lane) * P::NW;
        if constexpr (GSH == 0) {
            const uint2* m2 = reinterpret_cast<const uint2*>(m);
            return {ld_stream(m2 + jp), MIN ? ld_stream(m2 + 4 + jp) : make_uint2(0u, 0u)};
        } else {  // both chunks in group (2 jp) >> GSH
            const int g = (2 * jp) >> GSH;
            const uint32_t sc = m[g], mn = MIN ? m[P::NG + g] : 0u;
            return {make_uint2(sc, sc), make_uint2(mn, mn)};
        }
    }
    static __device__ __forceinline__ void tacc_w(const Ch& ch, int w, float coef, float* acc) {
        tacc8<(B <= 4)>(P::spread(ch, 2 * w), P::spread(ch, 2 * w + 1), coef, acc);
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const float c = gy * __uint_as_float(jj ? t.s.y : t.s.x);
        const float b = MIN ? gy * __uint_as_float(jj ? t.m.y : t.m.x) : -float(OFF) * c;
        off[0] += b;
        off[1] += b;
        tacc_w(ch, 0, c, acc);
        tacc_w(ch, 1, c, acc + 8);
        tacc_w(ch, 2, c, acc + 16);
        tacc_w(ch, 3, c, acc + 24);
    }
};

template <class PQ>
struct TIQ : PQ {
    using Ch = typename PQ::Ch;
    struct TM { uint4 s; };  // scales of chunks 2jp, 2jp+1 (group 32: .xy; group 16: .xyzw)
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        if constexpr (PQ::kWords2) {
            return {ld_stream(reinterpret_cast<const uint4*>(a.meta) + (si * 64 + lane) * 4 + jp)};
        } else if constexpr (PQ::kGsh > 0) {  // both chunks share group (2 jp) >> GSH
            const uint32_t v = ld_stream(reinterpret_cast<const uint32_t*>(a.meta) + (si * 64 + lane) * PQ::NW +
                                         ((2 * jp) >> PQ::kGsh));
            return {make_uint4(v, v, 0u, 0u)};
        } else {
            const uint2 v = ld_stream(reinterpret_cast<const uint2*>(a.meta) + (si * 64 + lane) * 4 + jp);
            return {make_uint4(v.x, v.y, 0u, 0u)};
        }
    }
    static __device__ __forceinline__ void tacc_w(const Ch& ch, int w, float coef, float* acc) {
        static_assert(PQ::kBits <= 4, "fp8 code conversion");
        tacc8<true>(PQ::spread(ch, 2 * w), PQ::spread(ch, 2 * w + 1), coef, acc);
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const float k = PQ::kMid;
        const uint32_t w[4] = {t.s.x, t.s.y, t.s.z, t.s.w};
        const float s0 = __uint_as_float(PQ::kWords2 ? w[2 * jj] : w[jj]) * PQ::kScaleMul;
        const float s1 = PQ::kWords2 ? __uint_as_float(w[2 * jj + 1]) * PQ::kScaleMul : s0;
        const float c0 = gy * s0, c1 = gy * s1;
        off[0] = fmaf(-k, c0, off[0]);
        off[1] = fmaf(-k, c1, off[1]);
        tacc_w(ch, 0, c0, acc);
        tacc_w(ch, 1, c0, acc + 8);
        tacc_w(ch, 2, c1, acc + 16);
        tacc_w(ch, 3, c1, acc + 24);
    }
};

struct TQ6K : RplQ6K {
    struct TM { uint32_t g; float d; };  // (u'0,u'1) of chunk 2jp | (u'0,u'1) of 2jp+1 << 16
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        const uint32_t* m = reinterpret_cast<const uint32_t*>(a.meta) + (si * 64 + lane) * 4 + jp;
        return {*m, reinterpret_cast<const float*>(a.dd)[(si * 64 + lane) * 2]};
    }
    // q = lo4 | hi2 << 4 spread to bytes as in RplQ6K::dot8
    static __device__ __forceinline__ void tacc6(uint32_t w, uint32_t h, int f0, float coef, float* acc) {
        uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * f0)) & 0x03030303u) << 4);
        uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * f0 + 2)) & 0x03030303u) << 4);
        asm("" : "+v"(lo), "+v"(hi));
        acc[0] = fmaf(ub0(lo), coef, acc[0]);
        acc[1] = fmaf(ub0(hi), coef, acc[1]);
        acc[2] = fmaf(ub1(lo), coef, acc[2]);
        acc[3] = fmaf(ub1(hi), coef, acc[3]);
        acc[4] = fmaf(ub2(lo), coef, acc[4]);
        acc[5] = fmaf(ub2(hi), coef, acc[5]);
        acc[6] = fmaf(ub3(lo), coef, acc[6]);
        acc[7] = fmaf(ub3(hi), coef, acc[7]);
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const uint32_t g = t.g >> (16 * jj);
        const float gd = gy * (t.d * (1.0f / 255.0f));
        const float c0 = gd * ub0(g), c1 = gd * ub1(g);
        off[0] = fmaf(-32.0f, c0, off[0]);
        off[1] = fmaf(-32.0f, c1, off[1]);
        tacc6(ch.c.x, ch.h.x, 0, c0, acc);
        tacc6(ch.c.y, ch.h.x, 2, c0, acc + 8);
        tacc6(ch.c.z, ch.h.y, 0, c1, acc + 16);
        tacc6(ch.c.w, ch.h.y, 2, c1, acc + 24);
    }
};

struct TQ8 : RplQ8 {
    struct TM { uint2 s; };  // f32 scales of chunks 2jp, 2jp+1
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        return {ld_stream(reinterpret_cast<const uint2*>(a.meta) + (si * 64 + lane) * 4 + jp)};
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const float c = gy * __uint_as_float(jj ? t.s.y : t.s.x);
        off[0] = fmaf(-128.0f, c, off[0]);
        off[1] = fmaf(-128.0f, c, off[1]);
        const uint32_t B = 0x80808080u;
        tacc_u8(ch.c0.x ^ B, c, acc);
        tacc_u8(ch.c0.y ^ B, c, acc + 4);
        tacc_u8(ch.c0.z ^ B, c, acc + 8);
        tacc_u8(ch.c0.w ^ B, c, acc + 12);
        tacc_u8(ch.c1.x ^ B, c, acc + 16);
        tacc_u8(ch.c1.y ^ B, c, acc + 20);
        tacc_u8(ch.c1.z ^ B, c, acc + 24);
        tacc_u8(ch.c1.w ^ B, c, acc + 28);
    }
};

struct TQ4 : RplQ4 {
    struct TM { uint2 s; };
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        return {ld_stream(reinterpret_cast<const uint2*>(a.meta) + (si * 64 + lane) * 4 + jp)};
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float* off) {
        const float c = gy * __uint_as_float(jj ? t.s.y : t.s.x);
        off[0] = fmaf(-8.0f, c, off[0]);
        off[1] = fmaf(-8.0f, c, off[1]);
        const uint32_t B = 0x88888888u;
        tacc_nib(ch.c.x ^ B, c, acc);
        tacc_nib(ch.c.y ^ B, c, acc + 8);
        tacc_nib(ch.c.z ^ B, c, acc + 16);
        tacc_nib(ch.c.w ^ B, c, acc + 24);
    }
};

// MatVecT looks the grid up across the wave instead: lane l holds grid[l & 15],
// and ds_bpermute from byte address a returns the value of lane (a >> 2) & 63,
// so a code word shifted to put nibble n at bits 2..5 reads grid[nibble n]
// whatever the bits above hold (every lane of the wave is active here). Per
// column of the transposed product this measured 29-31 us against 21-23 us
// with the LDS table at 4096x14336 (one box).
__device__ __forceinline__ float iq4nl_perm(uint32_t w, int n, int grid) {
    const uint32_t addr = n == 0 ? w << 2 : w >> (4 * n - 2);
    return __int_as_float(__builtin_amdgcn_ds_bpermute(int(addr), grid));
}
struct TIQ4NL : RplIQ4NL {
    struct TM { uint2 s; int grid; };  // scales of chunks 2jp, 2jp+1; this lane's grid value
    static __device__ __forceinline__ TM load_tm(const RplArgs& a, int64_t si, int lane, int jp) {
        return {ld_stream(reinterpret_cast<const uint2*>(a.meta) + (si * 64 + lane) * 4 + jp),
                __float_as_int(kIQ4NLGrid[lane & 15])};
    }
    template <int jj>
    static __device__ __forceinline__ void tacc(const Ch& ch, const TM& t, float gy, float* acc, float*) {
        const float c = gy * __uint_as_float(jj ? t.s.y : t.s.x);
        const uint32_t wd[4] = {ch.c.x, ch.c.y, ch.c.z, ch.c.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int n = 0; n < 8; ++n) acc[8 * i + n] = fmaf(iq4nl_perm(wd[i], n, t.grid), c, acc[8 * i + n]);
    }
};

// Column group of block x in XCD-aware order. Consecutive block ids go to
// the 8 XCDs in turn, so x = 32q + 8jp + k gives super-block sb = 8q + k,
// chunk pair jp: the four chunk pairs of a super-block (ids 8 apart) run on
// one XCD and read its metadata lines (each lane's chunk-pair words are
// interleaved per super-block) through one L2. Grids round the super-blocks
// up to a multiple of 8; the blocks past nsb return at once.
__device__ __forceinline__ void rpl_t_cg(int x, int& sb, int& jp) {
    jp = (x >> 3) & 3;
    sb = (x >> 5) * 8 + (x & 7);
}

template <class P, int GP>
__global__ void __launch_bounds__(1024) k_gemvt_rpl(RplArgs a, const float* __restrict__ gy, float* __restrict__ gx,
                                                   float* __restrict__ part) {
    __shared__ float red[16 * 64];
    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    int sb, jp;
    rpl_t_cg(blockIdx.x, sb, jp);
    if (sb >= a.nsb) return;  // uniform over the block
    const int slice = blockIdx.y, b = blockIdx.z;
    const int nslices = gridDim.y;
    const int g0 = (slice * W + wave) * GP;
    const int64_t cols = int64_t(a.nsb) * 256;
    const float* gyb = gy + int64_t(b) * a.rows;

    float acc[64], off[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 64; ++k) acc[k] = 0.f;

    // GP row groups, fully unrolled with a 2-deep register ring so that every
    // index is static and no load sits under a branch (either would make the
    // next use wait for all outstanding loads). Row groups past the end are
    // clamped to the last one and contribute gy = 0.
    struct Set {
        typename P::Ch c0, c1;
        typename P::TM tm;
        float gy;
    };
    auto load = [&](int i, Set& st) {
        const int g = min(g0 + i, a.rg_count - 1);
        const int64_t si = int64_t(g) * a.nsb + sb;
        st.c0 = P::load_ch(a, rpl_chunk(a, si, 2 * jp), lane);
        st.c1 = P::load_ch(a, rpl_chunk(a, si, 2 * jp + 1), lane);
        st.tm = P::load_tm(a, si, lane, jp);
        st.gy = gyb[min(g * 64 + lane, a.rows - 1)];
    };
    constexpr int R = GP < 2 ? GP : 2;
    Set ring[R];
#pragma unroll
    for (int i = 0; i < R; ++i) load(i, ring[i]);
#pragma unroll
    for (int i = 0; i < GP; ++i) {
        Set& st = ring[i % R];
        __builtin_amdgcn_sched_barrier(0);
        const int row = (g0 + i) * 64 + lane;
        const float gv = row < a.rows ? st.gy : 0.f;
        P::template tacc<0>(st.c0, st.tm, gv, acc, off);
        P::template tacc<1>(st.c1, st.tm, gv, acc + 32, off + 2);
        __builtin_amdgcn_sched_barrier(0);
        if (i + R < GP) load(i + R, ring[i % R]);
    }

    // Reduce-scatter over the 64 lanes: at each level a lane keeps half of
    // its 2m values and adds its partner's copy of that half; lane l ends
    // with column l of this wave's 64. Every level runs on the VALU: lane
    // swaps for m = 32 and 16, DPP for m = 8 (l ^ 8), 4 (partner l ^ 7, which
    // also differs in bit 2), 2 and 1.
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = reduce_scatter32(acc[i], acc[i + 32]);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = reduce_scatter16(acc[i], acc[i + 16]);
    {
        const bool hi = (lane & 8) != 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float keep = hi ? acc[i + 8] : acc[i], send = hi ? acc[i] : acc[i + 8];
            acc[i] = keep + row_xor8(send);
        }
    }
    {
        const bool hi = (lane & 4) != 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float keep = hi ? acc[i + 4] : acc[i], send = hi ? acc[i] : acc[i + 4];
            acc[i] = keep + half_mirror(send);
        }
    }
    {
        const bool hi = (lane & 2) != 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float keep = hi ? acc[i + 2] : acc[i], send = hi ? acc[i] : acc[i + 2];
            acc[i] = keep + quad_xor2(send);
        }
    }
    {
        const bool hi = (lane & 1) != 0;
        const float keep = hi ? acc[1] : acc[0], send = hi ? acc[0] : acc[1];
        acc[0] = keep + quad_xor1(send);
    }
    // Group offsets: column l is in local group l >> 4 = 2*bit5 + bit4; after
    // the two swap levels every lane of a 16-lane row adds up its row.
    off[0] = reduce_scatter32(off[0], off[2]);
    off[1] = reduce_scatter32(off[1], off[3]);
    const float o = row_sum16(reduce_scatter16(off[0], off[1]));

    // the block's waves, added in wave order
    red[wave * 64 + lane] = acc[0] + o;
    __syncthreads();
    if (wave != 0) return;
    float total = 0.f;
    for (int w = 0; w < W; ++w) total += red[w * 64 + lane];
    const int64_t col = int64_t(sb) * 256 + jp * 64 + lane;
    float* gxb = gx + int64_t(b) * cols;
    if (nslices == 1) {
        gxb[col] += total;
        return;
    }
    // Several slices: store this slice's partial; a separate launch adds the
    // slices in slice order (a last-arriving-block tail costs more here than
    // the extra launch: its ticket round trips bypass the caches).
    part[(int64_t(b) * nslices + slice) * cols + col] = total;
}

// Row-group slices for `batch` rows. One slice (no second pass) when the
// column groups alone give at least kRplTMinBlocks blocks; otherwise enough
// slices for about kRplTBlocks blocks. Each block runs W <= 16 waves of GP
// (1, 2, 4 or 8) row groups, GP the smallest that keeps W <= 16 (at least 2
// when the slice has more than one row group), so a slice is W * GP row
// groups.
constexpr int kRplTMinBlocks = 180;
constexpr int kRplTBlocks = 256;

struct RplTPlan {
    int slices, W, GP;
};
RplTPlan rpl_t_plan(const RplArgs& a, int batch) {
    const int64_t per_slice = int64_t(a.nsb) * 4 * std::max(1, batch);
    int64_t slices = 1;
    if (per_slice < kRplTMinBlocks) slices = (kRplTBlocks + per_slice - 1) / per_slice;
    slices = std::min<int64_t>(slices, a.rg_count);
    int64_t rps = (a.rg_count + slices - 1) / slices;
    if (rps > 16 * 8) rps = 16 * 8;
    int gp = rps > 1 ? 2 : 1;
    while (gp < 8 && (rps + gp - 1) / gp > 8) gp *= 2;
    RplTPlan p;
    p.GP = gp;
    p.W = int((rps + gp - 1) / gp);
    p.slices = int((a.rg_count + int64_t(p.W) * gp - 1) / (int64_t(p.W) * gp));
    return p;
}

template <class P>
int launch_rpl_tr(const DevBlob& bl, const float* gy, float* gx, int batch, hipStream_t s, float* part) {
    const RplArgs& a = bl.rpl;
    const int64_t cols = int64_t(a.nsb) * 256;
    for (int b0 = 0; b0 < batch; b0 += kRplTMaxBatch) {
        const int nb = std::min(kRplTMaxBatch, batch - b0);
        const RplTPlan p = rpl_t_plan(a, nb);
        auto kern = p.GP == 1 ? k_gemvt_rpl<P, 1> : p.GP == 2 ? k_gemvt_rpl<P, 2> : p.GP == 4 ? k_gemvt_rpl<P, 4> : k_gemvt_rpl<P, 8>;
        if (p.slices > 1 && !part) return int(hipErrorInvalidValue);  // the caller owes the slice scratch
        dim3 grid(unsigned((a.nsb + 7) / 8 * 32), unsigned(p.slices), unsigned(nb));
        hipLaunchKernelGGL(kern, grid, dim3(unsigned(64 * p.W)), 0, s, a, gy + int64_t(b0) * a.rows, gx + int64_t(b0) * cols,
                           part);
        if (p.slices > 1) launch_gemvt_reduce(part, gx + int64_t(b0) * cols, cols, p.slices, nb, s);
    }
    return int(hipGetLastError());
}

}  // namespace

// The forward policy of a row-interleaved blob has a second metadata word per
// chunk (block min or second scale group), which caps its plan at S = 2.
bool rpl_words2(const DevBlob& b) {
    switch (b.fmt) {
    case FMT_Q4_1: return RplQ41I::kWords2;
    case FMT_Q5_1: return RplQ51I::kWords2;
    case FMT_AFFINE: return RplAffI<1>::kWords2;  // every Affine group width: scale and min
    case FMT_TERNARY: return RplTernI::kWords2;
    case FMT_IQ2_XS: return RplIQ2XS::kWords2;
    case FMT_IQ3_S: return RplIQ3S::kWords2;
    case FMT_IQ4_XS: return RplIQ4XS::kWords2;
    default: return false;
    }
}

int launch_rpl_ex(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, const RplExtra& ex) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (b.fmt) {
    case FMT_Q4_K:
        return launch_rpl_t<RplQ4KI>(b, d_x, d_y, batch, s, ex);
    case FMT_Q2_K: return launch_rpl_t<RplKxI<2>>(b, d_x, d_y, batch, s, ex);
    case FMT_Q3_K: return launch_rpl_t<RplKxI<3>>(b, d_x, d_y, batch, s, ex);
    case FMT_Q5_K: return launch_rpl_t<RplKxI<5>>(b, d_x, d_y, batch, s, ex);
    case FMT_Q6_K: return launch_rpl_t<RplQ6K>(b, d_x, d_y, batch, s, ex);
    case FMT_Q8_0: return launch_rpl_t<RplQ8>(b, d_x, d_y, batch, s, ex);
    case FMT_Q4_0: return launch_rpl_t<RplQ4I>(b, d_x, d_y, batch, s, ex);
    case FMT_Q4_1: return launch_rpl_t<RplQ41I>(b, d_x, d_y, batch, s, ex);
    case FMT_Q5_0: return launch_rpl_t<RplQ50I>(b, d_x, d_y, batch, s, ex);
    case FMT_Q5_1: return launch_rpl_t<RplQ51I>(b, d_x, d_y, batch, s, ex);
    case FMT_AFFINE:
        switch (b.block_weights) {
        case 32: return launch_rpl_t<RplAffI<0>>(b, d_x, d_y, batch, s, ex);
        case 64: return launch_rpl_t<RplAffI<1>>(b, d_x, d_y, batch, s, ex);
        case 128: return launch_rpl_t<RplAffI<2>>(b, d_x, d_y, batch, s, ex);
        case 256: return launch_rpl_t<RplAffI<3>>(b, d_x, d_y, batch, s, ex);
        default: return int(hipErrorInvalidValue);
        }
    case FMT_TERNARY: return launch_rpl_t<RplTernI>(b, d_x, d_y, batch, s, ex);
    case FMT_BINARY:  // +-scale per 32 as IQ1_S, or per 128
        return b.block_weights == 128 ? launch_rpl_t<RplBin128>(b, d_x, d_y, batch, s, ex)
                                      : launch_rpl_t<RplIQ1S>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ1_S: return launch_rpl_t<RplIQ1S>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ2_XXS: return launch_rpl_t<RplIQ2XXS>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ2_XS: return launch_rpl_t<RplIQ2XS>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ3_XXS: return launch_rpl_t<RplIQ3XXS>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ3_S: return launch_rpl_t<RplIQ3S>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ4_XS: return launch_rpl_t<RplIQ4XS>(b, d_x, d_y, batch, s, ex);
    case FMT_IQ4_NL: return launch_rpl_t<RplIQ4NL>(b, d_x, d_y, batch, s, ex);
    default: return int(hipErrorInvalidValue);
    }
}

int launch_rpl(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, int mode, const float* aux,
               float* d_scratch) {
    RplExtra ex;
    ex.mode = mode;
    ex.aux = aux;
    ex.partial = d_scratch;
    return launch_rpl_ex(b, d_x, d_y, batch, stream, ex);
}

namespace {

// Bytes per (row group, super-block, lane) item of each image section.
struct RplItems {
    int cb, hb, mb, db;  // code chunk (x8 planes), high-bit chunk (x8), metadata, (d, dmin)
};
bool rpl_items(const DevBlob& b, RplItems& it) {
    LinCodes lc;
    if (rpl_lin_spec(b.fmt, b.block_weights, b.iq_bits, b.iq_sg, lc)) {
        const int cb = lc.bits == 4 ? 16 : lc.bits >= 2 ? 8 : 4;
        it = {cb, lc.bits == 3 ? 4 : 0, 4 * (256 / lc.sg), 0};
        return true;
    }
    if (b.fmt == FMT_AFFINE && rpl_affine_group(b.block_weights)) {
        it = {16, 0, 8 * (256 / b.block_weights), 0};
        return true;
    }
    switch (b.fmt) {
    case FMT_Q4_K: it = {16, 0, 32, 8}; return true;
    case FMT_Q2_K: it = {8, 0, 32, 8}; return true;
    case FMT_Q3_K: it = {8, 4, 32, 8}; return true;
    case FMT_Q5_K: it = {16, 4, 32, 8}; return true;
    case FMT_Q6_K: it = {16, 8, 16, 8}; return true;
    case FMT_Q8_0: it = {32, 0, 32, 0}; return true;
    case FMT_Q4_0: it = {16, 0, 32, 0}; return true;
    case FMT_Q4_1: it = {16, 0, 64, 0}; return true;
    case FMT_Q5_0: it = {16, 4, 32, 0}; return true;
    case FMT_Q5_1: it = {16, 4, 64, 0}; return true;
    default: return false;
    }
}

// Rows 2i / 2i+1 of dst <- row i of a / b, items of isz bytes (a multiple of
// 4), G < 2*rg_in the destination row group: with sb_major (Q4_K code
// planes, rpl_strides) dst[G][sb][p][L] = (L even ? a : b)[G/2][sb][p][32*(G%2)
// + L/2], otherwise the same in [p][G][sb][L] order; metadata has planes = 1.
__global__ void __launch_bounds__(256) k_rpl_pairs(uint8_t* __restrict__ dst, const uint8_t* __restrict__ a,
                                                   const uint8_t* __restrict__ b, int isz, int64_t rg_in, int64_t nsb,
                                                   int64_t planes, int sb_major) {
    const int64_t n = planes * 2 * rg_in * nsb * 64;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const int L = int(i & 63);
    int64_t r = i >> 6, p, sb, G;
    if (sb_major) {
        p = r % planes;
        r /= planes;
        sb = r % nsb;
        G = r / nsb;
    } else {
        sb = r % nsb;
        r /= nsb;
        G = r % (2 * rg_in);
        p = r / (2 * rg_in);
    }
    const uint8_t* src = (L & 1) ? b : a;
    const int64_t si = sb_major ? (((G / 2) * nsb + sb) * planes + p) * 64 + 32 * (G & 1) + (L >> 1)
                                : ((p * rg_in + G / 2) * nsb + sb) * 64 + 32 * (G & 1) + (L >> 1);
    const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src + si * isz);
    uint32_t* d4 = reinterpret_cast<uint32_t*>(dst + i * isz);
    for (int k = 0; k < isz / 4; ++k) d4[k] = s4[k];
}

struct FusedLayout {
    size_t codes, hi, meta, dd, wrow, total;
};
FusedLayout fused_layout(const RplItems& it, int64_t rg, int64_t nsb, bool with_wrow = false) {
    FusedLayout f{};
    auto add = [&](size_t n) {
        const size_t off = (f.total + 255) & ~size_t(255);
        f.total = off + n;
        return off;
    };
    const size_t per = size_t(rg) * size_t(nsb) * 64;
    f.codes = add(per * 8 * it.cb);
    f.hi = it.hb ? add(per * 8 * it.hb) : 0;
    f.meta = add(per * it.mb);
    f.dd = it.db ? add(per * it.db) : 0;
    f.wrow = with_wrow ? add(size_t(rg) * 64 * sizeof(float)) : 0;
    return f;
}

void finish_fused(const DevBlob& proto, int64_t rows, int64_t rg, const FusedLayout& f, uint8_t* base, DevBlob& out) {
    out = DevBlob{};
    out.fmt = proto.fmt;
    out.iq_bits = proto.iq_bits;
    out.iq_sg = proto.iq_sg;
    out.block_weights = proto.block_weights;
    out.rows = rows;
    out.cols = proto.cols;
    out.layout = LAYOUT_RPL;
    out.device = proto.device;
    out.base = base;
    out.device_bytes = f.total;
    RplArgs& r = out.rpl;
    r.codes = base + f.codes;
    r.hi = f.hi ? base + f.hi : nullptr;
    r.meta = base + f.meta;
    r.dd = f.dd ? reinterpret_cast<const float2_t*>(base + f.dd) : nullptr;
    r.wrow = f.wrow ? reinterpret_cast<const float*>(base + f.wrow) : nullptr;
    r.partial = nullptr;
    r.rows = int(rows);
    r.nsb = proto.rpl.nsb;
    r.rg_count = int(rg);
    r.ksplit = 1;
    rpl_strides(proto.fmt, rg, r.nsb, r.cs_si, r.cs_j);
}

}  // namespace

int rpl_fuse_rows(const DevBlob* parts, int n, DevBlob& out, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RplItems it{};
    if (n <= 0 || !rpl_items(parts[0], it)) return int(hipErrorInvalidValue);
    int64_t rg = 0, rows = 0;
    for (int i = 0; i < n; ++i) {
        const DevBlob& b = parts[i];
        if (b.layout != LAYOUT_RPL || b.fmt != parts[0].fmt || b.cols != parts[0].cols || b.rows % 64 ||
            b.iq_bits != parts[0].iq_bits || b.iq_sg != parts[0].iq_sg || b.block_weights != parts[0].block_weights)
            return int(hipErrorInvalidValue);
        rg += b.rpl.rg_count;
        rows += b.rows;
    }
    const int64_t nsb = parts[0].rpl.nsb;
    // the stack keeps the parts' prefill-GEMM row factors when every part has them
    bool with_wrow = true, row_factors = false;
    for (int i = 0; i < n; ++i) {
        with_wrow = with_wrow && parts[i].rpl.wrow;
        row_factors = row_factors || parts[i].gemm_row_factors;
    }
    const FusedLayout f = fused_layout(it, rg, nsb, with_wrow);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, f.total);
    if (e != hipSuccess) return int(e);
    uint8_t* b8 = static_cast<uint8_t*>(base);
    int64_t g0 = 0;
    for (int i = 0; i < n && e == hipSuccess; ++i) {
        const RplArgs& r = parts[i].rpl;
        const size_t per = size_t(r.rg_count) * nsb * 64, off = size_t(g0) * nsb * 64;
        const size_t per_all = size_t(rg) * nsb * 64;
        if (rpl_sb_major(parts[0].fmt)) {  // row-group-major planes: one contiguous run per part
            e = hipMemcpyAsync(b8 + f.codes + off * 8 * it.cb, r.codes, per * 8 * it.cb, hipMemcpyDeviceToDevice, s);
            if (it.hb && e == hipSuccess)
                e = hipMemcpyAsync(b8 + f.hi + off * 8 * it.hb, r.hi, per * 8 * it.hb, hipMemcpyDeviceToDevice, s);
        } else {  // chunk-step-major planes: one run per chunk step
            for (int p = 0; p < 8 && e == hipSuccess; ++p) {
                e = hipMemcpyAsync(b8 + f.codes + (p * per_all + off) * it.cb, r.codes + p * per * it.cb, per * it.cb,
                                   hipMemcpyDeviceToDevice, s);
                if (it.hb && e == hipSuccess)
                    e = hipMemcpyAsync(b8 + f.hi + (p * per_all + off) * it.hb, r.hi + p * per * it.hb, per * it.hb,
                                       hipMemcpyDeviceToDevice, s);
            }
        }
        if (e == hipSuccess) e = hipMemcpyAsync(b8 + f.meta + off * it.mb, r.meta, per * it.mb, hipMemcpyDeviceToDevice, s);
        if (it.db && e == hipSuccess)
            e = hipMemcpyAsync(b8 + f.dd + off * it.db, r.dd, per * it.db, hipMemcpyDeviceToDevice, s);
        if (with_wrow && e == hipSuccess)
            e = hipMemcpyAsync(b8 + f.wrow + size_t(g0) * 64 * sizeof(float), r.wrow,
                               size_t(r.rg_count) * 64 * sizeof(float), hipMemcpyDeviceToDevice, s);
        g0 += r.rg_count;
    }
    if (e == hipSuccess) {
        finish_fused(parts[0], rows, rg, f, b8, out);
        out.gemm_row_factors = row_factors;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        (void)hipFree(base);  // cleanup after the error being returned
        out = DevBlob{};
    }
    return int(e);
}

int rpl_fuse_pairs(const DevBlob& a, const DevBlob& b, DevBlob& out, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    RplItems it{};
    if (!rpl_items(a, it) || a.layout != LAYOUT_RPL || b.layout != LAYOUT_RPL || a.fmt != b.fmt ||
        a.iq_bits != b.iq_bits || a.iq_sg != b.iq_sg || a.block_weights != b.block_weights ||
        a.rows != b.rows || a.cols != b.cols || a.rows % 32)
        return int(hipErrorInvalidValue);
    const int64_t rg_in = a.rpl.rg_count, rg = 2 * rg_in, nsb = a.rpl.nsb;
    const FusedLayout f = fused_layout(it, rg, nsb);
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, f.total);
    if (e != hipSuccess) return int(e);
    uint8_t* b8 = static_cast<uint8_t*>(base);
    const int sbm = rpl_sb_major(a.fmt) ? 1 : 0;
    auto run = [&](size_t off, const uint8_t* pa, const uint8_t* pb, int isz, int64_t planes) {
        const int64_t n = planes * rg * nsb * 64;
        hipLaunchKernelGGL(k_rpl_pairs, dim3(unsigned((n + 255) / 256)), dim3(256), 0, s, b8 + off, pa, pb, isz, rg_in,
                           nsb, planes, sbm);
    };
    run(f.codes, a.rpl.codes, b.rpl.codes, it.cb, 8);
    if (it.hb) run(f.hi, a.rpl.hi, b.rpl.hi, it.hb, 8);
    run(f.meta, a.rpl.meta, b.rpl.meta, it.mb, 1);
    if (it.db)
        run(f.dd, reinterpret_cast<const uint8_t*>(a.rpl.dd), reinterpret_cast<const uint8_t*>(b.rpl.dd), it.db, 1);
    e = hipGetLastError();
    if (e == hipSuccess) finish_fused(a, 2 * a.rows, rg, f, b8, out);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        (void)hipFree(base);  // cleanup after the error being returned
        out = DevBlob{};
    }
    return int(e);
}

size_t rpl_t_scratch_floats(const RplArgs& a, int batch) {
    // batch rows go kRplTMaxBatch per launch (the last launch may take fewer)
    size_t most = 0;
    const int full = std::min(batch, kRplTMaxBatch), rest = batch % kRplTMaxBatch;
    for (int nb : {full, rest}) {
        if (nb <= 0) continue;
        const RplTPlan p = rpl_t_plan(a, nb);
        if (p.slices > 1) most = std::max(most, size_t(p.slices) * size_t(nb) * size_t(a.nsb) * 256);
    }
    return most;
}

size_t rpl_scratch_floats(const DevBlob& b, int batch) {
    if (b.layout != LAYOUT_RPL || batch <= 0) return 0;
    const RplPlan p = rpl_plan(b, rpl_words2(b) ? 2 : 4);  // the plan launch_rpl_t makes for this blob
    if (p.ksplit <= 1) return 0;
    return size_t(std::min(batch, kRplFwdBatch)) * size_t(p.ksplit) * size_t(b.rpl.rg_count) * 64;
}

int launch_rpl_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (b.fmt) {
    case FMT_Q4_K: return launch_rpl_tr<TQ4K>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q2_K: return launch_rpl_tr<TKx<2>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q3_K: return launch_rpl_tr<TKx<3>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q5_K: return launch_rpl_tr<TKx<5>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q6_K: return launch_rpl_tr<TQ6K>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q8_0: return launch_rpl_tr<TQ8>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q4_0: return launch_rpl_tr<TQ4>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q4_1: return launch_rpl_tr<TB32<4, true, 0, 0u>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q5_0: return launch_rpl_tr<TB32<5, false, 16, 0u>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_Q5_1: return launch_rpl_tr<TB32<5, true, 0, 0u>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_AFFINE:
        switch (b.block_weights) {
        case 32: return launch_rpl_tr<TB32<4, true, 0, 0u, 0>>(b, d_gy, d_gx, batch, s, d_scratch);
        case 64: return launch_rpl_tr<TB32<4, true, 0, 0u, 1>>(b, d_gy, d_gx, batch, s, d_scratch);
        case 128: return launch_rpl_tr<TB32<4, true, 0, 0u, 2>>(b, d_gy, d_gx, batch, s, d_scratch);
        case 256: return launch_rpl_tr<TB32<4, true, 0, 0u, 3>>(b, d_gy, d_gx, batch, s, d_scratch);
        default: return int(hipErrorInvalidValue);
        }
    case FMT_TERNARY: return launch_rpl_tr<TIQ<RplTernI>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_BINARY:
        return b.block_weights == 128 ? launch_rpl_tr<TIQ<RplBin128>>(b, d_gy, d_gx, batch, s, d_scratch)
                                      : launch_rpl_tr<TIQ<RplIQ1S>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ1_S: return launch_rpl_tr<TIQ<RplIQ1S>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ2_XXS: return launch_rpl_tr<TIQ<RplIQ2XXS>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ2_XS: return launch_rpl_tr<TIQ<RplIQ2XS>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ3_XXS: return launch_rpl_tr<TIQ<RplIQ3XXS>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ3_S: return launch_rpl_tr<TIQ<RplIQ3S>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ4_XS: return launch_rpl_tr<TIQ<RplIQ4XS>>(b, d_gy, d_gx, batch, s, d_scratch);
    case FMT_IQ4_NL: return launch_rpl_tr<TIQ4NL>(b, d_gy, d_gx, batch, s, d_scratch);
    default: return int(hipErrorInvalidValue);
    }
}

}  // namespace wv
