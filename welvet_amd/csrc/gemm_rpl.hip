// gemm_rpl.hip — batched prefill on the row-interleaved layouts:
// Y[M][rows] = X[M][cols] * W^T with fp16 MFMA (v_mfma_f32_32x32x16_f16) and
// f32 accumulation. It replaces welvet's M independent GEMVs for a token block
// (forwardSIMDBlockFused, layers/dense/simd_block.go:17-39), within the 2e-3
// tolerance of an fp16 contraction.
//
// X is first converted once to fp16 (k_x_f16r), so the GEMM streams half the
// bytes for the operand every row tile re-reads and spends no VALU on it. Each
// token row is scaled by a power of two that puts its max|x| in [2^14, 2^15)
// before the cast, and the epilogue multiplies the row back: the scaling is
// exact, so rows that fit fp16 get the same fp16 values as an unscaled cast,
// while outlier rows (|x| > 65504) stay finite and rows of tiny activations
// keep their precision instead of going subnormal. Weight rows get the same
// treatment from a power-of-two factor stored per row at upload
// (RplArgs::wrow) that puts the row's largest fp16 B-operand value in
// [2^12, 2^13): the B-operand builders multiply the row's scales and mins by
// it before their fp16 cast and the epilogue divides it back out, so rows of
// tiny weights keep fp16's precision and rows past 65504 stay finite.
//
// W goes from the row-interleaved planes straight into MFMA B operands: a
// lane holds 32 columns of its row per chunk, and a lane swap puts them into
// the 32x32x16 operand layout (per-format B-operand builders). Within every
// 8-column block both operands are in k order [0,2,4,6,1,3,5,7], the order in
// which the code spread produces pairs; a dot product over the block does not
// depend on the order. Two kernels:
//   * k_gemm_rg, up to 128 tokens: a block per 64-row group, its waves
//     splitting K and reading X fragments straight from global memory, every
//     weight dequantized once;
//   * k_gemm_q4k_pw, more tokens: 256-row x 128-token tiles with X staged
//     through LDS.
// K is split over gridDim.z when the tile grid alone would leave CUs idle;
// the splits' partials meet in a fixed-order sum.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "wave_ops.h"
#include "wv_internal.h"

namespace wv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BK = 64;        // columns per K-step
constexpr int LDK = BK + 8;   // LDS row stride in halves (144 B: conflict-free 16 B row reads)

__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const half2v h = {_Float16(a), _Float16(b)};
    return __builtin_bit_cast(uint32_t, h);
}

// 8 weights from two spread words (byte b of `se` / `so` = the code of
// column 2b / 2b + 1 of an 8-column run) -> 4 half2 w = fma(q, sc, mn) in
// fp16, in k order [0,2,4,6,1,3,5,7].
// Codes of up to 4 bits convert with v_cvt_scalef32_pk_f16_fp8: a byte q <
// 16 read as fp8 e4m3 is q * 2^-9 exactly (exponent fields 0 and 1 share the
// step 2^-9), and the instruction applies the exponent of its f32 scale, so
// scale 512 gives q as fp16 for two bytes in one instruction. Wider codes
// (up to 5 bits) take the exponent-byte form: 0x64 | q is 1024 + q in fp16.
template <int FB>
__device__ __forceinline__ uint4 dequant8s(uint32_t se, uint32_t so, half2v sc, half2v mn) {
    half2v q[4];
    if constexpr (FB <= 4) {
        q[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(se, 512.0f, false);
        q[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(se, 512.0f, true);
        q[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(so, 512.0f, false);
        q[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(so, 512.0f, true);
    } else {
        const half2v k1024 = {_Float16(1024.0f), _Float16(1024.0f)};
        const uint32_t e = 0x64646464u;
        q[0] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(e, se, 0x04010400u)) - k1024;
        q[1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(e, se, 0x04030402u)) - k1024;
        q[2] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(e, so, 0x04010400u)) - k1024;
        q[3] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(e, so, 0x04030402u)) - k1024;
    }
    uint32_t p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_bit_cast(uint32_t, q[i] * sc + mn);
    return make_uint4(p[0], p[1], p[2], p[3]);
}

// Code planes of one 32-column chunk of a k-quant row (lane = row) and, after
// the lane swaps, the spread words of the MFMA B operands: for 32-row tile T
// and k16 step kk, lanes 0-31 take columns 16kk + 0..7 of rows 32T + lane and
// lanes 32-63 columns 16kk + 8..15 of the same rows. FB = code bits (2, 3, 4,
// 5); the planes are those of the forward kernels (Q4_K nibbles; Q5_K fifth
// bits; Q2_K / Q3_K two-bit plane and third bits).
template <int FB>
struct GemmCodes {
    struct C { uint4 c; uint32_t h; };
    static __device__ __forceinline__ C load(const RplArgs& a, int64_t ci, int lane) {
        C r;
        if constexpr (FB >= 4) {
            r.c = ld_nt(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane);
        } else {
            const uint2 v = reinterpret_cast<const uint2*>(a.codes)[ci * 64 + lane];
            r.c = make_uint4(v.x, v.y, 0u, 0u);
        }
        r.h = (FB == 5 || FB == 3) ? reinterpret_cast<const uint32_t*>(a.hi)[ci * 64 + lane] : 0u;
        return r;
    }
    // se/so[T][kk]: even / odd columns of the lane's 8-column run
    static __device__ __forceinline__ void spread(const C& c, int lane, uint32_t (&se)[2][2], uint32_t (&so)[2][2]) {
        const int up = lane >> 5;
        if constexpr (FB >= 4) {
            const auto k0 = __builtin_amdgcn_permlane32_swap(c.c.x, c.c.y, false, false);  // columns 0-15
            const auto k1 = __builtin_amdgcn_permlane32_swap(c.c.z, c.c.w, false, false);  // columns 16-31
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                se[T][0] = k0[T] & 0x0F0F0F0Fu;
                so[T][0] = (k0[T] >> 4) & 0x0F0F0F0Fu;
                se[T][1] = k1[T] & 0x0F0F0F0Fu;
                so[T][1] = (k1[T] >> 4) & 0x0F0F0F0Fu;
            }
        } else {  // dword kk holds spread words 4kk..4kk+3; this lane's are 4kk + 2up (+1)
            const auto p0 = __builtin_amdgcn_permlane32_swap(c.c.x, c.c.x, false, false);
            const auto p1 = __builtin_amdgcn_permlane32_swap(c.c.y, c.c.y, false, false);
            const int sh = 4 * up;
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                se[T][0] = (p0[T] >> sh) & 0x03030303u;
                so[T][0] = (p0[T] >> (sh + 2)) & 0x03030303u;
                se[T][1] = (p1[T] >> sh) & 0x03030303u;
                so[T][1] = (p1[T] >> (sh + 2)) & 0x03030303u;
            }
        }
        if constexpr (FB == 5 || FB == 3) {  // top bit of spread word s at bit s of each byte
            constexpr int top = FB == 5 ? 4 : 2;
            const auto hh = __builtin_amdgcn_permlane32_swap(c.h, c.h, false, false);
#pragma unroll
            for (int T = 0; T < 2; ++T)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int sb = 4 * kk + 2 * up;
                    se[T][kk] |= ((hh[T] >> sb) & 0x01010101u) << top;
                    so[T][kk] |= ((hh[T] >> (sb + 1)) & 0x01010101u) << top;
                }
        }
    }
};

// Per-format B-operand builders of the GEMM kernels. Ch holds one 32-column
// chunk of the lane's row (codes, the chunk's metadata, the super-block's
// scales); bops() returns the fp16 B operands bf[T][kk] of 32-row tile T and
// k16 step kk, in X's k order [0,2,4,6,1,3,5,7], with the tile row's scales
// and mins multiplied by its power-of-two row factor wk[T] (RplArgs::wrow)
// before their fp16 cast.
template <int FB>
struct GemmKQ {  // Q2_K, Q3_K, Q4_K, Q5_K: w = (d/255)*u*q + (dmin/127)*m
    struct Ch { typename GemmCodes<FB>::C c; uint32_t mw; float2 dd; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        return {GemmCodes<FB>::load(a, ci, lane), reinterpret_cast<const uint32_t*>(a.meta)[(si * 64 + lane) * 8 + j],
                reinterpret_cast<const float2*>(a.dd)[si * 64 + lane]};
    }
    // The lane forms the fp16 scales and mins of its own row (row `lane` of
    // the group: tile lane / 32) and the lane swap hands each lane both tiles'
    // pairs, the same values the other lane computed.
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        float w0 = wk[0], w1 = wk[1];
        asm("" : "+v"(w0), "+v"(w1));  // a select of values, not an indexed load of the array
        const float wo = (lane & 32) ? w1 : w0;  // the own row's factor
        const float d255 = c.dd.x * (wo * (1.0f / 255.0f)), dm127 = c.dd.y * (wo * (1.0f / 127.0f));
        const uint32_t gm = c.mw;
        const half2v scp = {_Float16(d255 * float(gm & 0xFFu)), _Float16(d255 * float((gm >> 8) & 0xFFu))};
        const half2v mnp = {_Float16(dm127 * float(int8_t(gm >> 16))), _Float16(dm127 * float(int32_t(gm) >> 24))};
        const auto sc2 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, scp),
                                                          __builtin_bit_cast(uint32_t, scp), false, false);
        const auto mn2 = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mnp),
                                                          __builtin_bit_cast(uint32_t, mnp), false, false);
        uint32_t se[2][2], so[2][2];
        GemmCodes<FB>::spread(c.c, lane, se, so);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const half2v sp = __builtin_bit_cast(half2v, uint32_t(sc2[T])), np = __builtin_bit_cast(half2v, uint32_t(mn2[T]));
            const half2v s0 = {sp.x, sp.x}, s1 = {sp.y, sp.y}, n0 = {np.x, np.x}, n1 = {np.y, np.y};
            bf[T][0] = __builtin_bit_cast(half8, dequant8s<FB>(se[T][0], so[T][0], s0, n0));
            bf[T][1] = __builtin_bit_cast(half8, dequant8s<FB>(se[T][1], so[T][1], s1, n1));
        }
    }
};

struct GemmQ6 {  // Q6_K: q = lo4 | hi2 << 4, w = (d/255)*u*(q - 32)
    struct Ch { uint4 c; uint2 h; uint32_t mw; float d; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        const uint32_t m = reinterpret_cast<const uint32_t*>(a.meta)[(si * 64 + lane) * 4 + (j >> 1)];
        return {ld_nt(reinterpret_cast<const uint4*>(a.codes) + ci * 64 + lane),
                reinterpret_cast<const uint2*>(a.hi)[ci * 64 + lane], m >> (16 * (j & 1)),
                reinterpret_cast<const float*>(a.dd)[(si * 64 + lane) * 2]};
    }
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        typename GemmCodes<4>::C nib{c.c, 0u};
        uint32_t se[2][2], so[2][2];
        GemmCodes<4>::spread(nib, lane, se, so);
        // high-bit dword kk holds spread words 4kk..4kk+3 at bits 2f; this lane's are 4kk + 2up (+1)
        const int sh = 4 * (lane >> 5);
        const auto h0 = __builtin_amdgcn_permlane32_swap(c.h.x, c.h.x, false, false);
        const auto h1 = __builtin_amdgcn_permlane32_swap(c.h.y, c.h.y, false, false);
        const auto dt = __builtin_amdgcn_permlane32_swap(__float_as_uint(c.d), __float_as_uint(c.d), false, false);
        const auto mt = __builtin_amdgcn_permlane32_swap(c.mw, c.mw, false, false);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            se[T][0] |= ((h0[T] >> sh) & 0x03030303u) << 4;
            so[T][0] |= ((h0[T] >> (sh + 2)) & 0x03030303u) << 4;
            se[T][1] |= ((h1[T] >> sh) & 0x03030303u) << 4;
            so[T][1] |= ((h1[T] >> (sh + 2)) & 0x03030303u) << 4;
            const float d255 = __uint_as_float(dt[T]) * (wk[T] * (1.0f / 255.0f));
            const _Float16 sc0 = _Float16(d255 * float(mt[T] & 0xFFu)), sc1 = _Float16(d255 * float((mt[T] >> 8) & 0xFFu));
            const _Float16 mn0 = _Float16(-32.0f) * sc0, mn1 = _Float16(-32.0f) * sc1;
            const half2v s0 = {sc0, sc0}, s1 = {sc1, sc1}, n0 = {mn0, mn0}, n1 = {mn1, mn1};
            bf[T][0] = __builtin_bit_cast(half8, dequant8s<6>(se[T][0], so[T][0], s0, n0));
            bf[T][1] = __builtin_bit_cast(half8, dequant8s<6>(se[T][1], so[T][1], s1, n1));
        }
    }
};

struct GemmQ8 {  // Q8_0: w = scale*q, q int8, 32 bytes per chunk (consecutive columns)
    struct Ch { uint4 c0, c1; uint32_t sc; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        const uint4* p = reinterpret_cast<const uint4*>(a.codes) + (ci * 64 + lane) * 2;
        return {ld_nt(p), ld_nt(p + 1), reinterpret_cast<const uint32_t*>(a.meta)[(si * 64 + lane) * 8 + j]};
    }
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        (void)lane;
        const uint32_t dw[8] = {c.c0.x, c.c0.y, c.c0.z, c.c0.w, c.c1.x, c.c1.y, c.c1.z, c.c1.w};
        const auto st = __builtin_amdgcn_permlane32_swap(c.sc, c.sc, false, false);
        const half2v k1152 = {_Float16(1152.0f), _Float16(1152.0f)};
        const uint32_t e = 0x64646464u;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            // lanes 0-31: columns 16kk + 0..7 (dwords 4kk, 4kk+1); lanes 32-63: + 8..15
            const auto A = __builtin_amdgcn_permlane32_swap(dw[4 * kk], dw[4 * kk + 2], false, false);
            const auto B = __builtin_amdgcn_permlane32_swap(dw[4 * kk + 1], dw[4 * kk + 3], false, false);
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                const uint32_t lo = A[T] ^ 0x80808080u, hi = B[T] ^ 0x80808080u;  // q + 128 as unsigned bytes
                const uint32_t hb[4] = {__builtin_amdgcn_perm(e, lo, 0x04020400u), __builtin_amdgcn_perm(e, hi, 0x04020400u),
                                        __builtin_amdgcn_perm(e, lo, 0x04030401u), __builtin_amdgcn_perm(e, hi, 0x04030401u)};
                const _Float16 sh = _Float16(__uint_as_float(st[T]) * wk[T]);
                const half2v s2 = {sh, sh};
                uint32_t p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) p[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2v, hb[i]) - k1152) * s2);
                bf[T][kk] = __builtin_bit_cast(half8, make_uint4(p[0], p[1], p[2], p[3]));
            }
        }
    }
};

// The 32-weight block formats (Q4_0 with its nibble xor 8, Q4_1, Q5_0, Q5_1)
// and AffinePacked g64 (GSH = 1: chunks 2g, 2g+1 share group g): one scale
// (and min) per chunk from the lane's 8 (16) metadata words per super-block;
// w = scale*q + min, or scale*(q - OFF).
template <int FB, bool MIN, int OFF, uint32_t XR, int GSH = 0>
struct GemmB32 {
    static constexpr int NG = 8 >> GSH, NW = MIN ? 2 * NG : NG;
    struct Ch { typename GemmCodes<FB>::C c; uint32_t sc, mn; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        Ch r;
        r.c = GemmCodes<FB>::load(a, ci, lane);
        r.c.c.x ^= XR;
        r.c.c.y ^= XR;
        r.c.c.z ^= XR;
        r.c.c.w ^= XR;
        const uint32_t* m = reinterpret_cast<const uint32_t*>(a.meta) + (si * 64 + lane) * NW;
        r.sc = m[j >> GSH];
        r.mn = MIN ? m[NG + (j >> GSH)] : 0u;
        return r;
    }
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        uint32_t se[2][2], so[2][2];
        GemmCodes<FB>::spread(c.c, lane, se, so);
        const auto st = __builtin_amdgcn_permlane32_swap(c.sc, c.sc, false, false);
        const auto mt = __builtin_amdgcn_permlane32_swap(c.mn, c.mn, false, false);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const float scf = __uint_as_float(st[T]) * wk[T];
            const _Float16 sc = _Float16(scf), mn = _Float16(MIN ? __uint_as_float(mt[T]) * wk[T] : -float(OFF) * scf);
            const half2v s2 = {sc, sc}, n2 = {mn, mn};
            bf[T][0] = __builtin_bit_cast(half8, dequant8s<FB>(se[T][0], so[T][0], s2, n2));
            bf[T][1] = __builtin_bit_cast(half8, dequant8s<FB>(se[T][1], so[T][1], s2, n2));
        }
    }
};

// Codes of one bit (BinaryPacked g32, IQ1_S): one word per chunk whose byte b
// holds at bit s the code of column 8(s/2) + 2b + s%2.
struct GemmCodes1 {
    struct C { uint32_t c; };
    static __device__ __forceinline__ C load(const RplArgs& a, int64_t ci, int lane) {
        return {reinterpret_cast<const uint32_t*>(a.codes)[ci * 64 + lane]};
    }
    static __device__ __forceinline__ void spread(const C& c, int lane, uint32_t (&se)[2][2], uint32_t (&so)[2][2]) {
        const auto hh = __builtin_amdgcn_permlane32_swap(c.c, c.c, false, false);
        const int up = lane >> 5;
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int sb = 4 * kk + 2 * up;
                se[T][kk] = (hh[T] >> sb) & 0x01010101u;
                so[T][kk] = (hh[T] >> (sb + 1)) & 0x01010101u;
            }
    }
};

// The linear-code formats (the linear IQ formats, TernaryPacked, BinaryPacked
// g32 and g128): w = scale*(q - MID2/2), one scale per 32 columns, two (SG16,
// one per k16 step) or one per 2^GSH chunks; one-bit codes read +-scale =
// (2*scale)*(q - 1/2).
template <int FB, bool SG16, int MID2, int GSH = 0>
struct GemmLin {
    using Codes = std::conditional_t<FB == 1, GemmCodes1, GemmCodes<FB>>;
    static constexpr int NW = SG16 ? 16 : (8 >> GSH);  // metadata words per lane and super-block
    struct Ch { typename Codes::C c; uint32_t s0, s1; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        const uint32_t* m = reinterpret_cast<const uint32_t*>(a.meta) + (si * 64 + lane) * NW;
        const uint32_t s0 = m[SG16 ? 2 * j : (j >> GSH)];
        return {Codes::load(a, ci, lane), s0, SG16 ? m[2 * j + 1] : s0};
    }
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        uint32_t se[2][2], so[2][2];
        Codes::spread(c.c, lane, se, so);
        const auto t0 = __builtin_amdgcn_permlane32_swap(c.s0, c.s0, false, false);
        const auto t1 = __builtin_amdgcn_permlane32_swap(c.s1, c.s1, false, false);
        constexpr float mul = FB == 1 ? 2.0f : 1.0f, mid = 0.5f * MID2;
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const float scf = __uint_as_float(kk ? t1[T] : t0[T]) * (mul * wk[T]);
                const _Float16 sc = _Float16(scf), mn = _Float16(-mid * scf);
                const half2v s2 = {sc, sc}, n2 = {mn, mn};
                bf[T][kk] = __builtin_bit_cast(half8, dequant8s<FB>(se[T][kk], so[T][kk], s2, n2));
            }
    }
};

// IQ4_NL (quant/iq.go:169-180): w = scale * grid[q], the 16-value float grid
// (kIQ4NLGrid) as fp16, one scale per 32-column chunk. The codes are Q4_K's
// nibble planes; the grid is looked up four codes at a time with
// v_perm_b32 from byte tables of the fp16 values' low and high bytes (codes
// 0-7 from the first two dwords of a table, 8-15 from the last two, picked
// per byte by the code's bit 3), and the low and high bytes are interleaved
// into half2 pairs in k order [0,2,4,6,1,3,5,7].
struct GemmNL {
    static constexpr uint16_t h16(int q) { return __builtin_bit_cast(uint16_t, _Float16(kIQ4NLGrid[q])); }
    static constexpr uint32_t tab(int n, int sh) {  // bytes 4n..4n+3 of the low (sh 0) or high (sh 8) table
        return uint32_t((h16(4 * n) >> sh) & 0xFF) | uint32_t((h16(4 * n + 1) >> sh) & 0xFF) << 8 |
               uint32_t((h16(4 * n + 2) >> sh) & 0xFF) << 16 | uint32_t((h16(4 * n + 3) >> sh) & 0xFF) << 24;
    }
    struct Ch { GemmCodes<4>::C c; uint32_t s0; };
    static __device__ __forceinline__ Ch load(const RplArgs& a, int64_t ci, int64_t si, int j, int lane) {
        return {GemmCodes<4>::load(a, ci, lane), reinterpret_cast<const uint32_t*>(a.meta)[(si * 64 + lane) * 8 + j]};
    }
    // fp16 grid values of the 4 codes in the bytes of c: half2 of bytes 0, 1 and of bytes 2, 3
    static __device__ __forceinline__ void look4(uint32_t c, half2v& q01, half2v& q23) {
        constexpr uint32_t L0 = tab(0, 0), L1 = tab(1, 0), L2 = tab(2, 0), L3 = tab(3, 0);
        constexpr uint32_t H0 = tab(0, 8), H1 = tab(1, 8), H2 = tab(2, 8), H3 = tab(3, 8);
        const uint32_t sel = c & 0x07070707u;
        const uint32_t hi8 = ((c >> 3) & 0x01010101u) * 0xFFu;  // 0xFF in the bytes of codes 8-15
        const uint32_t lo = (__builtin_amdgcn_perm(L3, L2, sel) & hi8) | (__builtin_amdgcn_perm(L1, L0, sel) & ~hi8);
        const uint32_t hi = (__builtin_amdgcn_perm(H3, H2, sel) & hi8) | (__builtin_amdgcn_perm(H1, H0, sel) & ~hi8);
        q01 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi, lo, 0x05010400u));
        q23 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi, lo, 0x07030602u));
    }
    static __device__ __forceinline__ void bops(const Ch& c, int lane, const float (&wk)[2], half8 (&bf)[2][2]) {
        uint32_t se[2][2], so[2][2];
        GemmCodes<4>::spread(c.c, lane, se, so);
        const auto st = __builtin_amdgcn_permlane32_swap(c.s0, c.s0, false, false);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const _Float16 sc = _Float16(__uint_as_float(st[T]) * wk[T]);
            const half2v s2 = {sc, sc};
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                half2v q[4];
                look4(se[T][kk], q[0], q[1]);
                look4(so[T][kk], q[2], q[3]);
                uint32_t p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) p[i] = __builtin_bit_cast(uint32_t, q[i] * s2);
                bf[T][kk] = __builtin_bit_cast(half8, make_uint4(p[0], p[1], p[2], p[3]));
            }
        }
    }
};

// Row factors (RplArgs::wrow) of row group g in the B-operand layout: wk[T]
// belongs to row 32T + lane % 32, the lane's row in 32-row tile T. Two plain
// loads rather than one and a lane swap: nothing waits for them before the
// first B operands (a swap right after the load would stall the wave for a
// memory round trip before its first code loads go out).
__device__ __forceinline__ void row_factors(const RplArgs& a, int g, int lane, float (&wk)[2]) {
    wk[0] = a.wrow[int64_t(g) * 64 + (lane & 31)];
    wk[1] = a.wrow[int64_t(g) * 64 + 32 + (lane & 31)];
}

struct GemmArgs {
    RplArgs w;
    // fp16 8-column blocks of X in permuted k order, row m scaled by
    // 1 / xscale[m]: [M][K/8] row-major, or for k_gemm_rg in MFMA A-fragment
    // order [K/16][ceil(M/32)][64] (lane l of fragment (q, tile): token
    // 32*tile + l%32, block 2q + l/32; tokens past M are zero)
    const uint4* xh;
    const float* xscale;   // [M] power-of-two factor of each row's fp16 copy
    float* y;         // [M][rows] (splits == 1) or partials [split][M][rows]
    int M, K;
    int sb_per_split;
};

// 8 columns of X times `up`, as fp16 pairs in k order [0,2,4,6,1,3,5,7].
__device__ __forceinline__ uint4 pack_x8(float4 lo, float4 hi, float up) {
    lo = make_float4(lo.x * up, lo.y * up, lo.z * up, lo.w * up);
    hi = make_float4(hi.x * up, hi.y * up, hi.z * up, hi.w * up);
    return make_uint4(pack_h2(lo.x, lo.z), pack_h2(hi.x, hi.z), pack_h2(lo.y, lo.w), pack_h2(hi.y, hi.w));
}
__device__ __forceinline__ float absmax8(float4 lo, float4 hi) {
    return fmaxf(fmaxf(fmaxf(fabsf(lo.x), fabsf(lo.y)), fmaxf(fabsf(lo.z), fabsf(lo.w))),
                 fmaxf(fmaxf(fabsf(hi.x), fabsf(hi.y)), fmaxf(fabsf(hi.z), fabsf(hi.w))));
}
// The row's factor from its max|x| (the block-wide reduction), 2^-shift.
__device__ __forceinline__ float row_shift_up(float mx, float* red, float* xscale_m, int t) {
    mx = wave_maximum(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int sh = 0;  // x is multiplied by 2^sh
    if (mx > 0.f && mx <= 3.4028235e38f) sh = min(126, max(-126, 14 - ilogbf(mx)));
    if (t == 0) *xscale_m = ldexpf(1.0f, -sh);
    return ldexpf(1.0f, sh);
}
// silu(g) * u of one element, the expression of the SwiGLU kernels
// (layers/swiglu/cpu.go:41-53).
__device__ __forceinline__ float silu_mul1(float g, float u) { return g / (1.0f + expf(-g)) * u; }
__device__ __forceinline__ float4 silu_mul4(float4 g, float4 u) {
    return make_float4(silu_mul1(g.x, u.x), silu_mul1(g.y, u.y), silu_mul1(g.z, u.z), silu_mul1(g.w, u.w));
}

// X f32 [M][K] -> fp16 blocks of 8 in the B operands' k order
// [0,2,4,6,1,3,5,7] (pack_x8), one block per token row:
// the row's max|x| picks xscale = 2^e with max|x| / xscale in [2^14, 2^15)
// (1 for an all-zero or non-finite row), and the blocks hold x / xscale.
// A row of up to 256 * NR blocks of 8 is read once, into registers, with every
// load issued before the first use (slots past the row re-read its last block).
// FRAG writes the A-fragment order of GemmArgs::xh (block i of row m at
// ((i/2)*mt + m/32)*64 + m%32 + 32*(i%2)); its grid covers the padded rows,
// which get zeros. SW: x is the gate and u the up projection, and the row
// converted is silu(x) * u (the SwiGLU product feeding the down projection).
template <int NR, bool FRAG, bool SW>
__global__ void __launch_bounds__(256) k_x_f16r(const float4* __restrict__ x, const float4* __restrict__ u,
                                                 uint4* __restrict__ xh, float* __restrict__ xscale, int kb8, int M) {
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x;
    const int mt = (M + 31) / 32;
    auto put = [&](int i, uint4 v) {
        if constexpr (FRAG)
            xh[(int64_t(i >> 1) * mt + (m >> 5)) * 64 + (m & 31) + 32 * (i & 1)] = v;
        else
            xh[int64_t(m) * kb8 + i] = v;
    };
    if (FRAG && m >= M) {
        for (int i = t; i < kb8; i += 256) put(i, make_uint4(0u, 0u, 0u, 0u));
        return;
    }
    const float4* xr = x + int64_t(m) * kb8 * 2;
    const float4* ur = SW ? u + int64_t(m) * kb8 * 2 : nullptr;
    auto ld = [&](int k) { return SW ? silu_mul4(xr[k], ur[k]) : xr[k]; };
    float mx = 0.f;
    if constexpr (NR > 0) {
        float4 lo[NR], hi[NR];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
            const int i = min(t + 256 * j, kb8 - 1);
            lo[j] = xr[2 * i];
            hi[j] = xr[2 * i + 1];
        }
        if constexpr (SW) {
            float4 ul[NR], uh[NR];
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                const int i = min(t + 256 * j, kb8 - 1);
                ul[j] = ur[2 * i];
                uh[j] = ur[2 * i + 1];
            }
#pragma unroll
            for (int j = 0; j < NR; ++j) {
                lo[j] = silu_mul4(lo[j], ul[j]);
                hi[j] = silu_mul4(hi[j], uh[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < NR; ++j) mx = fmaxf(mx, absmax8(lo[j], hi[j]));
        const float up = row_shift_up(mx, red, xscale + m, t);
#pragma unroll
        for (int j = 0; j < NR; ++j)
            if (t + 256 * j < kb8) put(t + 256 * j, pack_x8(lo[j], hi[j], up));
    } else {  // longer rows: two passes, the second mostly from L2
        for (int i = t; i < kb8; i += 256) mx = fmaxf(mx, absmax8(ld(2 * i), ld(2 * i + 1)));
        const float up = row_shift_up(mx, red, xscale + m, t);
        for (int i = t; i < kb8; i += 256) put(i, pack_x8(ld(2 * i), ld(2 * i + 1), up));
    }
}
// The key-split prompt attention's merge straight into the O projection's
// fp16 operand: per row and head, sum_z 2^(m_z - M) o_z / sum_z 2^(m_z - M) l_z
// over the ks ranges of part ([ks][M][heads][hd + 4]: the unnormalized
// output, then the running max in log2 units and the running sum; ranges
// with m_z = -inf count 0), in the order and arithmetic of the decoder's
// k_attn_prefill_merge, then the row factor and blocks as k_x_f16r<NR, FRAG,
// false> makes them from the merged rows. Every range's values of a slot are
// loaded before the first add.
template <int NR, bool FRAG>
__global__ void __launch_bounds__(256) k_merge_x_f16r(const float* __restrict__ part, int ks, int n_heads, int hd,
                                                       uint4* __restrict__ xh, float* __restrict__ xscale, int kb8,
                                                       int M) {
    constexpr int KS = 8;
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x;
    const int mt = (M + 31) / 32;
    auto put = [&](int i, uint4 v) {
        if constexpr (FRAG)
            xh[(int64_t(i >> 1) * mt + (m >> 5)) * 64 + (m & 31) + 32 * (i & 1)] = v;
        else
            xh[int64_t(m) * kb8 + i] = v;
    };
    if (FRAG && m >= M) {
        for (int i = t; i < kb8; i += 256) put(i, make_uint4(0u, 0u, 0u, 0u));
        return;
    }
    const int ps = hd + 4;
    float4 lo[NR], hi[NR];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < NR; ++j) {
        const int i = min(t + 256 * j, kb8 - 1), col = 8 * i, head = col / hd, dim = col % hd;
        float mv[KS], lv[KS];
        float4 ol[KS], oh[KS];
#pragma unroll
        for (int z = 0; z < KS; ++z) {
            if (z < ks) {
                const float* pz = part + ((int64_t(z) * M + m) * n_heads + head) * ps;
                mv[z] = pz[hd];
                lv[z] = pz[hd + 1];
                ol[z] = *reinterpret_cast<const float4*>(pz + dim);
                oh[z] = *reinterpret_cast<const float4*>(pz + dim + 4);
            }
        }
        float Mz = mv[0];
#pragma unroll
        for (int z = 1; z < KS; ++z)
            if (z < ks) Mz = fmaxf(Mz, mv[z]);
        float4 nl = make_float4(0.f, 0.f, 0.f, 0.f), nh = nl;
        float den = 0.f;
#pragma unroll
        for (int z = 0; z < KS; ++z) {
            if (z < ks && mv[z] != -INFINITY) {
                const float w = exp2f(mv[z] - Mz);
                nl = make_float4(fmaf(w, ol[z].x, nl.x), fmaf(w, ol[z].y, nl.y), fmaf(w, ol[z].z, nl.z),
                                 fmaf(w, ol[z].w, nl.w));
                nh = make_float4(fmaf(w, oh[z].x, nh.x), fmaf(w, oh[z].y, nh.y), fmaf(w, oh[z].z, nh.z),
                                 fmaf(w, oh[z].w, nh.w));
                den = fmaf(w, lv[z], den);
            }
        }
        lo[j] = make_float4(nl.x / den, nl.y / den, nl.z / den, nl.w / den);
        hi[j] = make_float4(nh.x / den, nh.y / den, nh.z / den, nh.w / den);
        mx = fmaxf(mx, absmax8(lo[j], hi[j]));
    }
    const float up = row_shift_up(mx, red, xscale + m, t);
#pragma unroll
    for (int j = 0; j < NR; ++j)
        if (t + 256 * j < kb8) put(t + 256 * j, pack_x8(lo[j], hi[j], up));
}
template <bool FRAG, bool SW>
void launch_x_f16r_t(const float* x, const float* u, uint4* xh, float* xscale, int M, int kb8, hipStream_t s) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* u4 = reinterpret_cast<const float4*>(u);
    const dim3 g = dim3(unsigned(FRAG ? (M + 31) / 32 * 32 : M)), b = dim3(256);
    if (kb8 <= 256) hipLaunchKernelGGL((k_x_f16r<1, FRAG, SW>), g, b, 0, s, x4, u4, xh, xscale, kb8, M);
    else if (kb8 <= 512) hipLaunchKernelGGL((k_x_f16r<2, FRAG, SW>), g, b, 0, s, x4, u4, xh, xscale, kb8, M);
    else if (kb8 <= 1024) hipLaunchKernelGGL((k_x_f16r<4, FRAG, SW>), g, b, 0, s, x4, u4, xh, xscale, kb8, M);
    else if (kb8 <= 2048) hipLaunchKernelGGL((k_x_f16r<8, FRAG, SW>), g, b, 0, s, x4, u4, xh, xscale, kb8, M);
    else hipLaunchKernelGGL((k_x_f16r<0, FRAG, SW>), g, b, 0, s, x4, u4, xh, xscale, kb8, M);
}
template <bool FRAG>
void launch_x_f16r(const float* x, uint4* xh, float* xscale, int M, int kb8, hipStream_t s) {
    launch_x_f16r_t<FRAG, false>(x, nullptr, xh, xscale, M, kb8, s);
}

// The prompt forward's RMSNorm of a token block straight into the prefill
// GEMM's fp16 operand, one block per row: with `a`, h += a first (per element,
// the updated row written back: the residual add); then the norm with f64
// sums, y = float(x * inv * gamma) in f64 (layers/rmsnorm/cpu.go:70-85, as the
// decoder's k_rmsnorm); then the row's factor and fp16 blocks exactly as
// k_x_f16r<NR, false, false> makes them from y (max|y| in [2^14, 2^15), k
// order [0,2,4,6,1,3,5,7]); with `y`, the f32 rows as well (a and y may be
// the same rows: a block reads its row of a before its first barrier and
// writes y after it). An 8-column block is float4s 2b, 2b + 1, held by lanes
// 2b, 2b + 1; the even lane packs it. FRAG writes the blocks in the
// A-fragment order of GemmArgs::xh, as k_x_f16r<NR, true, false> does: the
// grid covers the M rows padded to 32, and the padding rows get zeros.
// `a` may be the unsummed K split of the GEMM that made it (a_splits
// slices a_stride floats apart, at most 4): the slices are added in split
// order, as k_split_sum adds them, every load issued before the first add.
template <bool FRAG>
__global__ void __launch_bounds__(1024) k_norm_x_f16r(float* __restrict__ h, const float* a, int a_splits,
                                                      int64_t a_stride, const float* __restrict__ gamma, float* y,
                                                      uint4* __restrict__ xh, float* __restrict__ xscale, int dim,
                                                      double eps, int M) {
    __shared__ double part[16];
    __shared__ float redm[16];
    const int m = blockIdx.x, t = threadIdx.x;
    constexpr int R = 4;
    const int n4 = dim / 4, kb8 = dim / 8;
    const int mt = (M + 31) / 32;
    auto put = [&](int b, uint4 v) {
        if constexpr (FRAG)
            xh[(int64_t(b >> 1) * mt + (m >> 5)) * 64 + (m & 31) + 32 * (b & 1)] = v;
        else
            xh[int64_t(m) * kb8 + b] = v;
    };
    if (FRAG && m >= M) {
        for (int b = t; b < kb8; b += 1024) put(b, make_uint4(0u, 0u, 0u, 0u));
        return;
    }
    h += int64_t(m) * dim;
    float4 xv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = t + 1024 * r;
        xv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < n4) {
            xv[r] = reinterpret_cast<const float4*>(h)[i];
            if (a) {
                const float4* ap = reinterpret_cast<const float4*>(a + int64_t(m) * dim) + i;
                float4 sv[4];
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    if (k < a_splits) sv[k] = ap[(int64_t(k) * a_stride) >> 2];
                float4 av = sv[0];
#pragma unroll
                for (int k = 1; k < 4; ++k)
                    if (k < a_splits) av = make_float4(av.x + sv[k].x, av.y + sv[k].y, av.z + sv[k].z, av.w + sv[k].w);
                xv[r] = make_float4(xv[r].x + av.x, xv[r].y + av.y, xv[r].z + av.z, xv[r].w + av.w);
            }
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r)
        ss += double(xv[r].x) * xv[r].x + double(xv[r].y) * xv[r].y + double(xv[r].z) * xv[r].z +
              double(xv[r].w) * xv[r].w;
    ss = wave_total_f64(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < 16; ++w) tot += part[w];
    const double inv = 1.0 / sqrt(tot / double(dim) + eps);
    float4 yv[R];
    float mx = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = t + 1024 * r;
        yv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < n4) {
            if (a) reinterpret_cast<float4*>(h)[i] = xv[r];
            const float4 g = gamma ? reinterpret_cast<const float4*>(gamma)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
            yv[r].x = float(double(xv[r].x) * inv * double(g.x));
            yv[r].y = float(double(xv[r].y) * inv * double(g.y));
            yv[r].z = float(double(xv[r].z) * inv * double(g.z));
            yv[r].w = float(double(xv[r].w) * inv * double(g.w));
            if (y) reinterpret_cast<float4*>(y + int64_t(m) * dim)[i] = yv[r];
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(yv[r].x), fabsf(yv[r].y)), fmaxf(fabsf(yv[r].z), fabsf(yv[r].w))));
        }
    }
    mx = wave_maximum(mx);
    if ((t & 63) == 0) redm[t >> 6] = mx;
    __syncthreads();
    mx = redm[0];
    for (int w = 1; w < 16; ++w) mx = fmaxf(mx, redm[w]);
    int sh = 0;  // the rows are multiplied by 2^sh
    if (mx > 0.f && mx <= 3.4028235e38f) sh = min(126, max(-126, 14 - ilogbf(mx)));
    if (t == 0) xscale[m] = ldexpf(1.0f, -sh);
    const float up = ldexpf(1.0f, sh);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = t + 1024 * r;
        const float4 nb = make_float4(quad_xor1(yv[r].x), quad_xor1(yv[r].y), quad_xor1(yv[r].z), quad_xor1(yv[r].w));
        if (!(t & 1) && i < n4 && i / 2 < kb8) put(i / 2, pack_x8(yv[r], nb, up));
    }
}

// Each of the 4 waves owns one 64-row group of the block's 256 rows and loads
// its row group's codes straight from the row-interleaved planes (lane l = row
// l, 16 bytes = 32 columns per chunk). One v_permlane32_swap per code-word
// pair turns that into MFMA B operands: after swapping words 0|1 (columns
// 0-7 | 8-15) between lanes l and l + 32, the first result holds rows 0-31
// with columns 0-7 in lanes 0-31 and 8-15 in lanes 32-63 (the 32x32x16 B
// layout of the first 32-row tile), the second the same for rows 32-63. Each
// wave dequantizes only its own rows (no copy shared through LDS), so the
// LDS carries X alone: per K-step a block writes 16 KB of fp16 X and each
// wave reads 16 KB back for 32 MFMAs (128 tokens x 64 rows x 64 columns),
// against 96 KB per 16 MFMAs per wave with fp16 W tiles.
template <class GP, int TM, int D, bool WF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) k_gemm_q4k_pw(GemmArgs ga) {
    constexpr int BM = 32 * TM;
    constexpr int XB = BM * (BK / 8) / 256;  // 8-column X blocks per thread per K-step
    static_assert(XB >= 1 && 4 % D == 0, "shape");
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][BM * LDK];
    __shared__ float xsc[BM];  // the tile's row factors, for the epilogue

    const RplArgs& a = ga.w;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nblk = blockIdx.x, mblk = blockIdx.y, split = blockIdx.z;
    const int sb0 = split * ga.sb_per_split;
    const int sb1 = min(a.nsb, sb0 + ga.sb_per_split);
    const int steps = (sb1 - sb0) * 4;
    const int kb8 = ga.K / 8;
    // Row factors of the tile's tokens, staged once; the main loop's barriers
    // order these writes before the epilogue reads them.
    if (t < BM) xsc[t] = ga.xscale[min(mblk * BM + t, ga.M - 1)];
    const int g = min(nblk * 4 + wave, a.rg_count - 1);  // this wave's row group
    float wk[2] = {1.0f, 1.0f};  // row factors of the lane's rows in the two 32-row tiles
    if constexpr (WF) row_factors(a, g, lane, wk);

    struct Regs {
        typename GP::Ch c[2];  // the step's two chunks of this lane's row
        uint4 xv[XB];          // fp16 X blocks
    };
    auto load = [&](int s, Regs& r) {
        const int sb = sb0 + s / 4;
        const int64_t si = int64_t(g) * a.nsb + sb;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = 2 * (s & 3) + jj;
            r.c[jj] = GP::load(a, rpl_chunk(a, si, j), si, j, lane);
        }
        const int k8 = sb * 32 + (s & 3) * 8;
#pragma unroll
        for (int i = 0; i < XB; ++i) {
            const int f = t + 256 * i, m = min(mblk * BM + f / 8, ga.M - 1);
            r.xv[i] = ga.xh[int64_t(m) * kb8 + k8 + f % 8];
        }
    };

    f32x16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    Regs ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        load(min(d, steps - 1), ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // B operands: [chunk][tile][k16 step] as fp16 in k order [0,2,4,6,1,3,5,7].
    // Step s + 1's are built (VALU) after the barrier, beside step s's MFMAs,
    // so the matrix cores run while the next weights are dequantized.
    half8 bf[2][2][2];
    GP::bops(ring[0].c[0], lane, wk, bf[0]);
    GP::bops(ring[0].c[1], lane, wk, bf[1]);
    for (int s0 = 0; s0 < steps; s0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int s = s0 + d, buf = s & 1;
#pragma unroll
            for (int i = 0; i < XB; ++i) {
                const int f = t + 256 * i;
                *reinterpret_cast<uint4*>(&xs[buf][(f / 8) * LDK + 8 * (f % 8)]) = ring[d].xv[i];
            }
            __builtin_amdgcn_sched_barrier(0);
            load(min(s + D, steps - 1), ring[d]);
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            half8 bn[2][2][2];  // step s + 1 (its codes sit in the next ring slot)
            GP::bops(ring[(d + 1) % D].c[0], lane, wk, bn[0]);
            GP::bops(ring[(d + 1) % D].c[1], lane, wk, bn[1]);
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int ks = 2 * jj + kk;
                    half8 af[TM];
#pragma unroll
                    for (int i = 0; i < TM; ++i)
                        af[i] = *reinterpret_cast<const half8*>(
                            &xs[buf][(i * 32 + (lane & 31)) * LDK + ks * 16 + 8 * (lane >> 5)]);
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int T = 0; T < 2; ++T)
                            acc[i][T] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[jj][T][kk], acc[i][T], 0, 0, 0);
                }
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
                for (int T = 0; T < 2; ++T)
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) bf[jj][T][kk] = bn[jj][T][kk];
        }
    }

    // C[i][j] of a 32x32 tile: lane holds j = lane % 32, i = 8*(r/4) + 4*(lane/32) + r%4.
    float* out = ga.y + int64_t(split) * ga.M * a.rows;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const int n = (nblk * 4 + wave) * 64 + T * 32 + (lane & 31);
            if (n >= a.rows) continue;
            const float wi = WF ? 1.0f / wk[T] : 1.0f;  // the row factor back out (exact: a power of two)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mblk * BM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < ga.M) out[int64_t(m) * a.rows + n] = acc[i][T][r] * wi * xsc[m - mblk * BM];
            }
        }
}

// The token-block GEMM for few tokens (TM 32-token tiles, TM = 1 or 2): one
// block per (64-row group, token block, K split), its W waves splitting the
// split's super-blocks (`per` consecutive ones each). A wave loads its row
// group's codes from the planes as k_gemm_q4k_pw does (B operands through
// lane swaps) and its fp16 X fragments straight from global memory (one
// contiguous 1 KB per wave and load: the A-fragment order of GemmArgs::xh),
// so the main loop has no barrier and no LDS traffic. A step is 64 columns
// (two chunks, four k16 MFMA steps); codes run DC steps ahead of use and X
// fragments (L2 hits: every row group's blocks read the same X) DX steps
// ahead, in register rings. Every weight is dequantized once per token block.
// The W waves' partial tiles meet in LDS after the loop and are added in wave
// order (deterministic), one 32-token tile at a time.
template <class GP, int TM, int DC, int DX, int NT, bool WF>
__global__ void __launch_bounds__(NT) k_gemm_rg(GemmArgs ga, int per) {
    constexpr int BM = 32 * TM;
    static_assert(4 % DC == 0 && 4 % DX == 0, "the rings must divide the 4 steps of a super-block");
    constexpr int DU = DC > DX ? DC : DX;  // loop unroll: both ring positions are compile-time
    extern __shared__ float red[];  // [W][2][16][64] partial tiles of one 32-token tile
    const RplArgs& a = ga.w;
    const int t = threadIdx.x, lane = t & 63, W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: chunk addresses stay scalar
    const int g = blockIdx.x, mblk = blockIdx.y, split = blockIdx.z;
    const int sb0 = split * ga.sb_per_split;
    const int sb1 = min(a.nsb, sb0 + ga.sb_per_split);
    const int wsb0 = sb0 + wave * per;
    const int steps = max(0, min(sb1, wsb0 + per) - wsb0) * 4;
    const int mt = (ga.M + 31) / 32;  // 32-token tiles of the fragment-ordered X
    float wk[2] = {1.0f, 1.0f};  // row factors of the lane's rows in the two 32-row tiles
    if constexpr (WF) row_factors(a, g, lane, wk);

    struct Codes {
        typename GP::Ch c[2];  // the step's two chunks of this lane's row
    };
    struct Xf {
        uint4 v[TM][4];  // A fragments of the step's 4 k16 steps
    };
    auto load_c = [&](int s, Codes& r) {
        const int64_t si = int64_t(g) * a.nsb + wsb0 + s / 4;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = 2 * (s & 3) + jj;
            r.c[jj] = GP::load(a, rpl_chunk(a, si, j), si, j, lane);
        }
    };
    auto load_x = [&](int s, Xf& r) {
        const int64_t q0 = int64_t(wsb0) * 16 + 4 * s;  // first k16 step of the step
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) r.v[i][ks] = ga.xh[((q0 + ks) * mt + mblk * TM + i) * 64 + lane];
    };

    f32x16 acc[TM][2];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    if (steps > 0) {
        Codes cr[DC];
        Xf xr[DX];
#pragma unroll
        for (int d = 0; d < DU; ++d) {
            if (d < DC) load_c(min(d, steps - 1), cr[d % DC]);
            if (d < DX) load_x(min(d, steps - 1), xr[d % DX]);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int s0 = 0; s0 < steps; s0 += DU) {
#pragma unroll
            for (int d = 0; d < DU; ++d) {
                const int s = s0 + d;
                const Codes cc = cr[d % DC];
                const Xf xc = xr[d % DX];
                __builtin_amdgcn_sched_barrier(0);
                load_c(min(s + DC, steps - 1), cr[d % DC]);
                load_x(min(s + DX, steps - 1), xr[d % DX]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    half8 bf[2][2];  // [tile][k16 step]
                    GP::bops(cc.c[jj], lane, wk, bf);
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                        for (int i = 0; i < TM; ++i) {
                            const half8 af = __builtin_bit_cast(half8, xc.v[i][2 * jj + kk]);
#pragma unroll
                            for (int T = 0; T < 2; ++T)
                                acc[i][T] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[T][kk], acc[i][T], 0, 0, 0);
                        }
                }
            }
        }
    }

    // C[i][j] of a 32x32 tile: lane holds j = lane % 32, i = 8*(r/4) + 4*(lane/32) + r%4.
    float* out = ga.y + int64_t(split) * ga.M * a.rows;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        if (i > 0) __syncthreads();  // the previous tile's sums have been read
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const float wi = WF ? 1.0f / wk[T] : 1.0f;  // the row factor back out (exact: a power of two)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[((wave * 2 + T) * 16 + r) * 64 + lane] = acc[i][T][r] * wi;
        }
        __syncthreads();
        for (int v = t; v < 2048; v += 64 * W) {
            const int T = v >> 10, r = (v >> 6) & 15, l = v & 63;
            float sum = 0.f;
            for (int w = 0; w < W; ++w) sum += red[((w * 2 + T) * 16 + r) * 64 + l];
            const int n = g * 64 + T * 32 + (l & 31);
            const int m = mblk * BM + i * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
            if (n < a.rows && m < ga.M) out[int64_t(m) * a.rows + n] = sum * ga.xscale[m];
        }
    }
}

// y[i] = sum_k part[k*n + i], k ascending; each thread owns 4 consecutive
// outputs (float4 when n % 4 == 0 and y is 16-byte aligned; the partials
// always are) and issues up to 8 splits' loads before adding them.
__global__ void __launch_bounds__(256) k_split_sum(const float* __restrict__ part, float* __restrict__ y, int64_t n,
                                                  int splits) {
    const int64_t i4 = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i4 * 4 >= n) return;
    if ((n & 3) || (reinterpret_cast<uintptr_t>(y) & 15)) {  // ragged or unaligned: scalar, in the same order
        for (int64_t i = i4 * 4; i < min<int64_t>(n, i4 * 4 + 4); ++i) {
            float s = 0.f;
            for (int k = 0; k < splits; ++k) s += part[int64_t(k) * n + i];
            y[i] = s;
        }
        return;
    }
    const float4* p = reinterpret_cast<const float4*>(part) + i4;
    const int64_t n4 = n >> 2;
    // Splits in order; each group of 8 loads (clamped to the last split, the
    // extra ones masked out of the sum) is issued before any add.
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = 0; k < splits; k += 8) {
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p[int64_t(min(k + j, splits - 1)) * n4];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (k + j < splits) {
                s.x += v[j].x;
                s.y += v[j].y;
                s.z += v[j].z;
                s.w += v[j].w;
            }
        }
    }
    reinterpret_cast<float4*>(y)[i4] = s;
}

}  // namespace

// Q4_K at every M; every other row-interleaved format from 9 token rows up
// (up to 8 rows, one batched GEMV launch reads the weights once).
bool gemm_supported(const DevBlob& b, int M) {
    if (b.layout != LAYOUT_RPL) return false;
    if (!b.rpl.wrow) return false;  // the gate/up pair images carry no row factors
    return b.fmt == FMT_Q4_K || M > 8;
}

// Which kernel runs a token block, its tile height (bm tokens), the K split
// (splits of sb_per_split super-blocks) and, for k_gemm_rg, its waves per
// block W and super-blocks per wave `per`:
//   * up to 64 tokens: k_gemm_rg (one block per 64-row group, 8 waves
//     splitting K, one or two 32-token tiles), K split over blocks by the
//     fewest passes of the grid per unit of work (below);
//   * 65 to 128 tokens on at least 200 row groups: k_gemm_rg with four
//     32-token tiles (4 waves, one per SIMD), no K split (4096->14336 M = 128
//     43.5 against 45.7 us; with the split, 14336->4096, 49.3 against 45.0);
//   * 65 to 128 tokens on fewer row groups: k_gemm_rg with two 64-token
//     blocks (8 waves, 2 per SIMD), K split as above (14336->4096 M = 128
//     42.1-42.7 against 42.7-43.4 us on k_gemm_q4k_pw split 14 ways);
//   * otherwise k_gemm_q4k_pw (256-row tiles of 128 tokens, one block per
//     CU), K split while whole tiles leave CUs idle.
enum { GEMM_PW = 1, GEMM_RG = 2 };
// k_gemm_rg waves per block: 8 (2 per SIMD) for one or two 32-token tiles,
// 4 (1 per SIMD) for four.
constexpr int rg_waves(int tm) { return tm == 4 ? 4 : 8; }
struct GemmPlan {
    int kind, bm, splits, sb_per_split, W, per;
};
constexpr int kRgMinBlocks = 200;  // row groups on which 128-token k_gemm_rg blocks fill the GPU unsplit
constexpr int64_t kCUs = 256;       // MI355X
GemmPlan gemm_plan(const DevBlob& b, int M) {
    const RplArgs& a = b.rpl;
    GemmPlan p{GEMM_PW, M <= 32 ? 32 : M <= 64 || (M <= 128 && a.rg_count < kRgMinBlocks) ? 64 : 128, 1, a.nsb, 1, 1};
    int want = 1;
    if (M <= 128) {
        // A k_gemm_rg block fills its CU (8 waves of up to 256 registers, or
        // 4 of 512), so the grid runs in ceil(blocks / 256) passes of
        // 1/want of the work each: the split with the fewest passes per unit
        // of work, the smallest of equals (no split sum where a split would
        // only add a pass).
        p.kind = GEMM_RG;
        const int64_t tiles = int64_t(a.rg_count) * ((M + p.bm - 1) / p.bm);
        const int max_split = std::max(1, a.nsb / 8);  // each split >= 8 super-blocks
        double best = 0.0;
        for (int w = 1; w <= max_split; ++w) {
            const double t = double((tiles * w + kCUs - 1) / kCUs) / w;
            if (w == 1 || t < best - 1e-9) {
                best = t;
                want = w;
            }
        }
    } else {
        const int64_t tiles = int64_t((a.rows + 255) / 256) * ((M + p.bm - 1) / p.bm);
        want = int(std::max<int64_t>(1, 256 / tiles));
        want = std::min(want, std::max(1, a.nsb / 2));  // each split >= 2 super-blocks
    }
    p.sb_per_split = (a.nsb + want - 1) / want;
    p.splits = (a.nsb + p.sb_per_split - 1) / p.sb_per_split;
    if (p.kind == GEMM_RG) {
        p.per = (p.sb_per_split + rg_waves(p.bm / 32) - 1) / rg_waves(p.bm / 32);
        p.W = (p.sb_per_split + p.per - 1) / p.per;
    }
    return p;
}

// Scratch floats: the fp16 copy of X (M*K halves), the M row factors, then
// the split-K partials (each piece 256-byte aligned).
size_t gemm_x_floats(const DevBlob& b, int M) {
    return ((size_t(M) + 31) / 32 * 32 * size_t(b.cols) / 2 + 63) / 64 * 64;  // tokens padded to 32 (A fragments)
}
size_t gemm_scale_floats(int M) { return (size_t(M) + 63) / 64 * 64; }
size_t gemm_scratch_floats(const DevBlob& b, int M) {
    const GemmPlan p = gemm_plan(b, M);
    return gemm_x_floats(b, M) + gemm_scale_floats(M) + (p.splits > 1 ? size_t(p.splits) * size_t(M) * size_t(b.rows) : 0);
}

// Calls go.template run<GP>() with the B-operand builder of b's format.
template <class Go>
int with_builder(const DevBlob& b, const Go& go) {
    switch (b.fmt) {
    case FMT_Q2_K: go.template run<GemmKQ<2>>(); return 0;
    case FMT_Q3_K: go.template run<GemmKQ<3>>(); return 0;
    case FMT_Q4_K: go.template run<GemmKQ<4>>(); return 0;
    case FMT_Q5_K: go.template run<GemmKQ<5>>(); return 0;
    case FMT_Q6_K: go.template run<GemmQ6>(); return 0;
    case FMT_Q8_0: go.template run<GemmQ8>(); return 0;
    case FMT_Q4_0: go.template run<GemmB32<4, false, 8, 0x88888888u>>(); return 0;
    case FMT_Q4_1: go.template run<GemmB32<4, true, 0, 0u>>(); return 0;
    case FMT_Q5_0: go.template run<GemmB32<5, false, 16, 0u>>(); return 0;
    case FMT_Q5_1: go.template run<GemmB32<5, true, 0, 0u>>(); return 0;
    case FMT_AFFINE:
        switch (b.block_weights) {
        case 32: go.template run<GemmB32<4, true, 0, 0u, 0>>(); return 0;
        case 64: go.template run<GemmB32<4, true, 0, 0u, 1>>(); return 0;
        case 128: go.template run<GemmB32<4, true, 0, 0u, 2>>(); return 0;
        case 256: go.template run<GemmB32<4, true, 0, 0u, 3>>(); return 0;
        default: return int(hipErrorInvalidValue);
        }
    case FMT_BINARY:
        if (b.block_weights == 128) {
            go.template run<GemmLin<1, false, 1, 2>>();
            return 0;
        }
        [[fallthrough]];
    case FMT_IQ1_S: go.template run<GemmLin<1, false, 1>>(); return 0;
    case FMT_IQ2_XXS: go.template run<GemmLin<2, false, 3>>(); return 0;
    case FMT_IQ2_XS: go.template run<GemmLin<2, true, 3>>(); return 0;
    case FMT_IQ3_XXS: go.template run<GemmLin<3, false, 7>>(); return 0;
    case FMT_IQ3_S: go.template run<GemmLin<3, true, 7>>(); return 0;
    case FMT_IQ4_XS: go.template run<GemmLin<4, true, 15>>(); return 0;
    case FMT_TERNARY: go.template run<GemmLin<2, true, 2>>(); return 0;
    case FMT_IQ4_NL: go.template run<GemmNL>(); return 0;
    default: return int(hipErrorInvalidValue);
    }
}

// k_gemm_q4k_pw with TM 32-token tiles per wave; WF: apply the row factors.
template <int TM, bool WF>
struct PwGo {
    dim3 grid;
    hipStream_t s;
    const GemmArgs& ga;
    template <class GP>
    void run() const {
        hipLaunchKernelGGL((k_gemm_q4k_pw<GP, TM, 4, WF>), grid, dim3(256), 0, s, ga);
    }
};

// k_gemm_rg with TM token tiles per block, `per` super-blocks per wave, W
// waves (at most rg_waves(TM)). Ring depths and block size per token tiles:
// one or two tiles run 8 waves (2 per SIMD, 256 registers each), four tiles 4
// waves (1 per SIMD, whose 512 registers hold the 128 accumulators and deeper
// rings).
template <int TM, bool WF>
struct RgGo {
    dim3 grid;
    int W, per;
    hipStream_t s;
    const GemmArgs& ga;
    template <class GP>
    void run() const {
        constexpr int DC = TM == 2 ? 2 : 4, DX = TM == 1 ? 2 : TM == 2 ? 1 : 2, NT = TM == 4 ? 256 : 512;
        const size_t lds = size_t(W) * 2 * 16 * 64 * sizeof(float);
        hipLaunchKernelGGL((k_gemm_rg<GP, TM, DC, DX, NT, WF>), grid, dim3(unsigned(64 * W)), lds, s, ga, per);
    }
};

template <bool WF>
int launch_tiles(const DevBlob& b, const GemmPlan& p, dim3 grid, hipStream_t s, const GemmArgs& ga) {
    if (p.kind == GEMM_RG)
        return p.bm == 32   ? with_builder(b, RgGo<1, WF>{grid, p.W, p.per, s, ga})
               : p.bm == 64 ? with_builder(b, RgGo<2, WF>{grid, p.W, p.per, s, ga})
                            : with_builder(b, RgGo<4, WF>{grid, p.W, p.per, s, ga});
    return with_builder(b, PwGo<4, WF>{grid, s, ga});
}

bool gemm_x_frag(const DevBlob& b, int M) { return gemm_plan(b, M).kind == GEMM_RG; }

int launch_norm_x_f16r(float* h, const float* a, int a_splits, int64_t a_stride, const float* gamma, float* y, void* xh,
                       float* xscale, int M, int dim, double eps, bool frag, void* stream) {
    if (a_splits < 1 || a_splits > 4 || (a_stride & 3)) return int(hipErrorInvalidValue);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (frag)
        hipLaunchKernelGGL(k_norm_x_f16r<true>, dim3(unsigned((M + 31) / 32 * 32)), dim3(1024), 0, s, h, a, a_splits,
                           a_stride, gamma, y, static_cast<uint4*>(xh), xscale, dim, eps, M);
    else
        hipLaunchKernelGGL(k_norm_x_f16r<false>, dim3(unsigned(M)), dim3(1024), 0, s, h, a, a_splits, a_stride, gamma,
                           y, static_cast<uint4*>(xh), xscale, dim, eps, M);
    return 0;
}

int launch_merge_x_f16r(const float* part, int ks, int n_heads, int hd, int M, bool frag, void* xhv, float* xscale,
                        void* stream) {
    const int kb8 = n_heads * hd / 8;
    if (ks < 1 || ks > 8 || hd % 8 || kb8 > 1024) return int(hipErrorInvalidValue);
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint4* xh = static_cast<uint4*>(xhv);
    const dim3 g(unsigned(frag ? (M + 31) / 32 * 32 : M)), b(256);
    auto go = [&](auto kern) { hipLaunchKernelGGL(kern, g, b, 0, s, part, ks, n_heads, hd, xh, xscale, kb8, M); };
    if (kb8 <= 256) frag ? go(k_merge_x_f16r<1, true>) : go(k_merge_x_f16r<1, false>);
    else if (kb8 <= 512) frag ? go(k_merge_x_f16r<2, true>) : go(k_merge_x_f16r<2, false>);
    else frag ? go(k_merge_x_f16r<4, true>) : go(k_merge_x_f16r<4, false>);
    return 0;
}

void launch_split_sum(const float* part, float* y, int64_t n, int splits, void* stream) {
    hipLaunchKernelGGL(k_split_sum, dim3(unsigned((n / 4 + 1 + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), part, y, n, splits);
}

void gemm_convert_x(const float* d_x, const float* d_u, int cols, int M, bool frag, void* xhv, float* xscale,
                    void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint4* xh = static_cast<uint4*>(xhv);
    const int kb8 = cols / 8;
    if (frag) {
        if (d_u) launch_x_f16r_t<true, true>(d_x, d_u, xh, xscale, M, kb8, s);
        else launch_x_f16r_t<true, false>(d_x, nullptr, xh, xscale, M, kb8, s);
    } else {
        if (d_u) launch_x_f16r_t<false, true>(d_x, d_u, xh, xscale, M, kb8, s);
        else launch_x_f16r_t<false, false>(d_x, nullptr, xh, xscale, M, kb8, s);
    }
}

int launch_gemm_xh(const DevBlob& b, const void* xh, const float* xscale, float* d_y, int M, void* stream,
                   float* d_part, int* d_splits) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!gemm_supported(b, M)) return int(hipErrorInvalidValue);
    const GemmPlan p = gemm_plan(b, M);
    const int bm = p.bm, splits = p.splits;
    if (splits > 1 && !d_part) return int(hipErrorInvalidValue);
    GemmArgs ga;
    ga.w = b.rpl;
    ga.xh = static_cast<const uint4*>(xh);
    ga.xscale = xscale;
    ga.y = splits > 1 ? d_part : d_y;
    ga.M = M;
    ga.K = int(b.cols);
    ga.sb_per_split = p.sb_per_split;
    const dim3 grid(unsigned(p.kind == GEMM_RG ? b.rpl.rg_count : (b.rows + 255) / 256), unsigned((M + bm - 1) / bm),
                    unsigned(splits));
    const int e = b.gemm_row_factors ? launch_tiles<true>(b, p, grid, s, ga) : launch_tiles<false>(b, p, grid, s, ga);
    if (e) return e;
    if (d_splits) *d_splits = splits;
    if (splits > 1 && !d_splits) launch_split_sum(d_part, d_y, int64_t(M) * b.rows, splits, s);
    return int(hipGetLastError());
}

int launch_gemm(const DevBlob& b, const float* d_x, float* d_y, int M, void* stream, float* d_scratch) {
    if (!gemm_supported(b, M) || !d_scratch) return int(hipErrorInvalidValue);
    uint4* xh = reinterpret_cast<uint4*>(d_scratch);
    float* xscale = d_scratch + gemm_x_floats(b, M);
    float* part = xscale + gemm_scale_floats(M);
    gemm_convert_x(d_x, nullptr, int(b.cols), M, gemm_x_frag(b, M), xh, xscale, stream);
    return launch_gemm_xh(b, xh, xscale, d_y, M, stream, part);
}

}  // namespace wv
