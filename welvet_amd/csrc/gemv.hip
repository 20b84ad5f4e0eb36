// gemv.hip — gfx950 kernels of the Dense MatVec path.
//
// Three families:
//   * k_gemv_raw / k_gemvt_raw: decode each weight from the uploaded bytes
//     (LAYOUT_RAW). Any format, any shape, including blocks that straddle rows.
//     Semantics follow the reference decoders element by element
//     (quant/*.go forEach* / unpack*), accumulating in f32.
//   * k_gemv_planar<Policy>: batch-1 decode GEMV on re-laid-out planes
//     (codes plane + scale planes, same byte count as the reference blob).
//     Each lane owns fixed 32-column chunks and keeps that slice of x in
//     VGPRs for the whole launch; waves walk rows, loading 16 B of codes per
//     lane per chunk (coalesced: the 64 lanes of a load read 1 KiB
//     contiguous), unpacking nibbles in registers and reducing row partials
//     with cross-lane shuffles plus LDS when K is split across waves.
//   * k_ternary_i8: the DTypeTernary int8 path (layers/dense/simd.go:130-147):
//     activations absmax-quantized to int8 in LDS, codes unpacked to bytes in
//     registers and multiplied with packed-dot v_dot4_i32_i8; exact int32.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "wv_internal.h"

namespace wv {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}

__device__ __forceinline__ float ld_f32(const uint8_t* p) {
    // 4-byte aligned in every layout that reaches here (block sizes are multiples of 4).
    return *reinterpret_cast<const float*>(p);
}
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// LSB-first bit field [bitpos, bitpos+nbits) of a byte stream, nbits <= 8
// (quant/helpers.go:140-149). Bits past `len` read as 0.
__device__ __forceinline__ uint32_t read_bits(const uint8_t* buf, int64_t len, int64_t bitpos, int nbits) {
    int64_t byte = bitpos >> 3;
    int sh = int(bitpos & 7);
    uint32_t v = byte < len ? buf[byte] : 0u;
    if (sh + nbits > 8 && byte + 1 < len) v |= uint32_t(buf[byte + 1]) << 8;
    return (v >> sh) & ((1u << nbits) - 1u);
}

struct RawArgs {
    const uint8_t* raw;
    int64_t raw_len;
    const float* scales;
    int64_t n_scales;
    int64_t rows, cols;
    int iq_bits, iq_sg;
    int g128;  // BinaryPacked with BlockWeights == 128 (row-aligned groups)
};

template <int F>
struct KSpecC;
template <> struct KSpecC<FMT_Q2_K> { static constexpr int bits = 2, has_dmin = 1, mid = 0; };
template <> struct KSpecC<FMT_Q3_K> { static constexpr int bits = 3, has_dmin = 1, mid = 0; };
template <> struct KSpecC<FMT_Q4_K> { static constexpr int bits = 4, has_dmin = 1, mid = 0; };
template <> struct KSpecC<FMT_Q5_K> { static constexpr int bits = 5, has_dmin = 1, mid = 0; };
template <> struct KSpecC<FMT_Q6_K> { static constexpr int bits = 6, has_dmin = 0, mid = 32; };

// Weight at flat index i = row*cols + col, decoded exactly as the reference.
template <int F>
__device__ __forceinline__ float decode(const RawArgs& a, int64_t i, int64_t row, int64_t col) {
    if constexpr (F == FMT_Q4_0) {  // q4_0.go:93-99
        const uint8_t* o = a.raw + (i >> 5) * 20;
        uint32_t b = o[4 + ((i & 31) >> 1)];
        int q = int((i & 1) ? (b >> 4) : (b & 15u));
        q = q > 7 ? q - 16 : q;
        return float(q) * ld_f32(o);
    } else if constexpr (F == FMT_Q8_0) {  // q8_0.go:58-63
        const uint8_t* o = a.raw + (i >> 5) * 36;
        return float(int8_t(o[4 + (i & 31)])) * ld_f32(o);
    } else if constexpr (F == FMT_Q4_1) {  // q4_1.go:63-72
        const uint8_t* o = a.raw + (i >> 5) * 24;
        uint32_t b = o[8 + ((i & 31) >> 1)];
        uint32_t q = (i & 1) ? (b >> 4) : (b & 15u);
        return ld_f32(o + 4) + float(q) * ld_f32(o);
    } else if constexpr (F == FMT_Q5_0) {  // q5_0.go:55-63
        const uint8_t* o = a.raw + (i >> 5) * 24;
        int q = int(read_bits(o + 4, 20, (i & 31) * 5, 5)) - 16;
        return float(q) * ld_f32(o);
    } else if constexpr (F == FMT_Q5_1) {  // q5_1.go:59-67
        const uint8_t* o = a.raw + (i >> 5) * 28;
        uint32_t q = read_bits(o + 8, 20, (i & 31) * 5, 5);
        return ld_f32(o + 4) + float(q) * ld_f32(o);
    } else if constexpr (F >= FMT_Q2_K && F <= FMT_Q6_K) {  // kquant.go:178-188
        using S = KSpecC<F>;
        constexpr int sbb = 8 + 16 + (S::has_dmin ? 16 : 0) + 256 * S::bits / 8;
        constexpr int qoff = S::has_dmin ? 40 : 24;
        const uint8_t* o = a.raw + (i >> 8) * sbb;
        int k = int(i & 255), g = k >> 4;
        float d = ld_f32(o);
        float sc = d * float(o[8 + g]) / 255.0f;
        if (sc == 0.0f) sc = d / 255.0f;
        uint32_t q = read_bits(o + qoff, sbb - qoff, int64_t(k) * S::bits, S::bits);
        if constexpr (S::has_dmin) {
            float mn = ld_f32(o + 4) * float(int8_t(o[24 + g])) / 127.0f;
            return mn + float(q) * sc;
        } else {
            return sc * float(int(q) - S::mid);
        }
    } else if constexpr (F >= FMT_IQ1_S && F <= FMT_IQ4_XS) {  // iq.go:169-207
        int64_t s = i / a.iq_sg;
        float scale = a.scales[s];
        uint32_t q = read_bits(a.raw, a.raw_len, i * a.iq_bits, a.iq_bits);
        if constexpr (F == FMT_IQ4_NL) {
            return scale * kIQ4NLGrid[q & 15];
        } else {
            if (a.iq_bits == 1) return (q & 1u) ? scale : -scale;
            constexpr float mid = F == FMT_IQ2_XXS || F == FMT_IQ2_XS ? 1.5f
                                : F == FMT_IQ3_XXS || F == FMT_IQ3_S ? 3.5f
                                : F == FMT_IQ4_XS ? 7.5f : 0.5f;
            return scale * (float(q) - mid);
        }
    } else if constexpr (F == FMT_TERNARY) {  // ternary.go:53-82
        int64_t g = i >> 4;
        uint32_t c = (ld_u32(a.raw + g * 4) >> ((i & 15) * 2)) & 3u;
        float s = g < a.n_scales ? a.scales[g] : 1.0f;
        return c == 0 ? -s : (c == 2 ? s : 0.0f);
    } else if constexpr (F == FMT_BINARY) {
        if (a.g128) {  // binary_g128.go:107-139, row-aligned groups
            int64_t wpr = a.cols >> 5, gpr = a.cols >> 7;
            uint32_t word = ld_u32(a.raw + (row * wpr + (col >> 5)) * 4);
            int64_t si = row * gpr + (col >> 7);
            float s = si < a.n_scales ? a.scales[si] : 1.0f;
            return ((word >> (col & 31)) & 1u) ? s : -s;
        }
        int64_t g = i >> 5;  // binary.go:49-75
        uint32_t word = ld_u32(a.raw + g * 4);
        float s = g < a.n_scales ? a.scales[g] : 1.0f;
        return ((word >> (i & 31)) & 1u) ? s : -s;
    } else {
        return 0.0f;
    }
}

// y[b][row] = sum_c w(row,c) x[b][c]; one wave per row, 4 rows per block.
template <int F>
__global__ void __launch_bounds__(256) k_gemv_raw(RawArgs a, const float* __restrict__ x, float* __restrict__ y) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave;
    if (row >= a.rows) return;
    const int b = blockIdx.y;
    const float* xb = x + int64_t(b) * a.cols;
    const int64_t base = row * a.cols;
    float acc = 0.0f;
    for (int64_t c = lane; c < a.cols; c += kWave) acc += decode<F>(a, base + c, row, c) * xb[c];
    acc = wave_sum(acc);
    if (lane == 0) y[int64_t(b) * a.rows + row] = acc;
}

// Partial gx over a row slice: part[(b*nsplit + split)*cols + c] = sum_{r in slice} w(r,c) gy[b][r].
template <int F>
__global__ void __launch_bounds__(256) k_gemvt_raw(RawArgs a, const float* __restrict__ gy, float* __restrict__ part,
                                                  int rows_per_split) {
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int split = blockIdx.y, b = blockIdx.z;
    if (c >= a.cols) return;
    const float* g = gy + int64_t(b) * a.rows;
    const int64_t r0 = int64_t(split) * rows_per_split;
    const int64_t r1 = min<int64_t>(a.rows, r0 + rows_per_split);
    float acc = 0.0f;
    for (int64_t r = r0; r < r1; ++r) acc += decode<F>(a, r * a.cols + c, r, c) * g[r];
    part[(int64_t(b) * gridDim.y + split) * a.cols + c] = acc;
}

__global__ void __launch_bounds__(256) k_gemvt_reduce(const float* __restrict__ part, float* __restrict__ gx,
                                                     int64_t cols, int nsplit) {
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= cols) return;
    float s = 0.0f;
    for (int k = 0; k < nsplit; ++k) s += part[(int64_t(b) * nsplit + k) * cols + c];
    gx[int64_t(b) * cols + c] += s;
}

// ---------------------------------------------------------------------------
// planar kernels
// ---------------------------------------------------------------------------

__device__ __forceinline__ float ub0(uint32_t v) { return float(v & 0xFFu); }
__device__ __forceinline__ float ub1(uint32_t v) { return float((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ub2(uint32_t v) { return float((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ub3(uint32_t v) { return float(v >> 24); }

// sum_k q_k x[k] for 8 unsigned 4-bit codes of one word (code k = nibble k).
__device__ __forceinline__ float dot8_u4(uint32_t w, const float* x) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
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
// sum_k q_k x[k] for 4 unsigned byte codes.
__device__ __forceinline__ float dot4_u8(uint32_t w, const float* x) {
    float a = ub0(w) * x[0];
    a = fmaf(ub1(w), x[1], a);
    a = fmaf(ub2(w), x[2], a);
    a = fmaf(ub3(w), x[3], a);
    return a;
}

struct PlanarArgs {
    const uint8_t* codes;    // row-major code plane
    const uint8_t* codes_hi; // Q6_K: 2-bit high plane
    const float* blk;        // k: (d, dmin) per super-block; Q8_0/Q4_0: scale per block
    const uint32_t* grp;     // k: per-chunk (u0, u1, m0, m1); Q6_K reads u16 pairs
    int64_t nchunks;         // K / 32
};

// Q4_K: chunk = 32 columns = groups (2p, 2p+1) of super-block jc/8.
// w = dmin*m/127 + (d*u/255)*q  (quant/kquant.go:178-188).
struct PolQ4K {
    struct Raw { uint4 c; float2 dd; uint32_t g; };
    static __device__ __forceinline__ Raw load(const PlanarArgs& a, int64_t row, int64_t jc) {
        Raw r;
        const int64_t ci = row * a.nchunks + jc;
        r.c = *reinterpret_cast<const uint4*>(a.codes + ci * 16);
        r.dd = reinterpret_cast<const float2*>(a.blk)[ci >> 3];
        r.g = a.grp[ci];
        return r;
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* x, float sx0, float sx1) {
        const float a0 = dot8_u4(r.c.x, x) + dot8_u4(r.c.y, x + 8);
        const float a1 = dot8_u4(r.c.z, x + 16) + dot8_u4(r.c.w, x + 24);
        const float d255 = r.dd.x * (1.0f / 255.0f), dm127 = r.dd.y * (1.0f / 127.0f);
        const float m0 = float(int8_t(r.g >> 16)), m1 = float(int32_t(r.g) >> 24);
        return d255 * fmaf(ub1(r.g), a1, ub0(r.g) * a0) + dm127 * fmaf(m1, sx1, m0 * sx0);
    }
};

// Q6_K: q = lo4 | hi2 << 4, w = (d*u/255)*(q-32).
// hi plane per chunk: dword t, byte b, bits 2f..2f+1 hold the high bits of the
// weight in byte b of spread word s = 4t+f (s = 2*word + nibble half).
struct PolQ6K {
    struct Raw { uint4 c; uint2 h; float d; uint32_t g; };
    static __device__ __forceinline__ Raw load(const PlanarArgs& a, int64_t row, int64_t jc) {
        Raw r;
        const int64_t ci = row * a.nchunks + jc;
        r.c = *reinterpret_cast<const uint4*>(a.codes + ci * 16);
        r.h = *reinterpret_cast<const uint2*>(a.codes_hi + ci * 8);
        r.d = a.blk[(ci >> 3) * 2];
        r.g = reinterpret_cast<const uint16_t*>(a.grp)[ci];
        return r;
    }
    static __device__ __forceinline__ float dot_word(uint32_t w, uint32_t h, int f0, const float* x) {
        const uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> (2 * f0)) & 0x03030303u) << 4);
        const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (2 * f0 + 2)) & 0x03030303u) << 4);
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
    static __device__ __forceinline__ float dot(const Raw& r, const float* x, float sx0, float sx1) {
        const float a0 = dot_word(r.c.x, r.h.x, 0, x) + dot_word(r.c.y, r.h.x, 2, x + 8);
        const float a1 = dot_word(r.c.z, r.h.y, 0, x + 16) + dot_word(r.c.w, r.h.y, 2, x + 24);
        const float d255 = r.d * (1.0f / 255.0f);
        return d255 * fmaf(ub1(r.g), fmaf(-32.0f, sx1, a1), ub0(r.g) * fmaf(-32.0f, sx0, a0));
    }
};

// Q8_0: 32 int8 codes + f32 scale per block; codes biased by 128 so that the
// byte converts unsigned: sum x*q = sum x*(q+128) - 128*sum x.
struct PolQ8 {
    struct Raw { uint4 c0, c1; float s; };
    static __device__ __forceinline__ Raw load(const PlanarArgs& a, int64_t row, int64_t jc) {
        Raw r;
        const int64_t ci = row * a.nchunks + jc;
        const uint4* p = reinterpret_cast<const uint4*>(a.codes + ci * 32);
        r.c0 = p[0];
        r.c1 = p[1];
        r.s = a.blk[ci];
        return r;
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* x, float sx0, float sx1) {
        const uint32_t B = 0x80808080u;
        float a = dot4_u8(r.c0.x ^ B, x) + dot4_u8(r.c0.y ^ B, x + 4);
        a += dot4_u8(r.c0.z ^ B, x + 8) + dot4_u8(r.c0.w ^ B, x + 12);
        a += dot4_u8(r.c1.x ^ B, x + 16) + dot4_u8(r.c1.y ^ B, x + 20);
        a += dot4_u8(r.c1.z ^ B, x + 24) + dot4_u8(r.c1.w ^ B, x + 28);
        return r.s * fmaf(-128.0f, sx0 + sx1, a);
    }
};

// Q4_0: signed nibble q in [-8,7] stored two's-complement; q ^ 8 = q + 8.
struct PolQ4 {
    struct Raw { uint4 c; float s; };
    static __device__ __forceinline__ Raw load(const PlanarArgs& a, int64_t row, int64_t jc) {
        Raw r;
        const int64_t ci = row * a.nchunks + jc;
        r.c = *reinterpret_cast<const uint4*>(a.codes + ci * 16);
        r.s = a.blk[ci];
        return r;
    }
    static __device__ __forceinline__ float dot(const Raw& r, const float* x, float sx0, float sx1) {
        const uint32_t B = 0x88888888u;
        float a = dot8_u4(r.c.x ^ B, x) + dot8_u4(r.c.y ^ B, x + 8);
        a += dot8_u4(r.c.z ^ B, x + 16) + dot8_u4(r.c.w ^ B, x + 24);
        return r.s * fmaf(-8.0f, sx0 + sx1, a);
    }
};

// Launch geometry: block = KW*RW waves. Wave (kw, rw) owns chunks
// jc = (i*KW + kw)*64 + lane, i < CPL, of every row in its row range.
template <class P, int CPL, int U>
__global__ void __launch_bounds__(512) k_gemv_planar(PlanarArgs a, const float* __restrict__ x, float* __restrict__ y,
                                                    int rows, int KW, int RPW) {
    extern __shared__ float part[];  // [RW*RPW][KW]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kw = wave % KW, rw = wave / KW;
    const int RW = (blockDim.x >> 6) / KW;
    const int b = blockIdx.y;
    const float* xb = x + int64_t(b) * a.nchunks * 32;
    float* yb = y + int64_t(b) * rows;

    float xr[CPL][32];
    float sx[CPL][2];
    int64_t jcs[CPL];
    bool ok[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        jcs[i] = int64_t(i * KW + kw) * kWave + lane;
        ok[i] = jcs[i] < a.nchunks;
        const float4* xp = reinterpret_cast<const float4*>(xb + (ok[i] ? jcs[i] : 0) * 32);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float4 v = ok[i] ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            xr[i][4 * k] = v.x;
            xr[i][4 * k + 1] = v.y;
            xr[i][4 * k + 2] = v.z;
            xr[i][4 * k + 3] = v.w;
        }
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            s0 += xr[i][k];
            s1 += xr[i][16 + k];
        }
        sx[i][0] = s0;
        sx[i][1] = s1;
    }

    const int wg_rows = RW * RPW;
    const int row0 = blockIdx.x * wg_rows + rw * RPW;
    const int row1 = min(rows, row0 + RPW);
    for (int r = row0; r < row1; r += U) {
        typename P::Raw raw[U][CPL];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                if (r + u < row1 && ok[i]) raw[u][i] = P::load(a, r + u, jcs[i]);
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            acc[u] = 0.f;
#pragma unroll
            for (int i = 0; i < CPL; ++i)
                if (r + u < row1 && ok[i]) acc[u] += P::dot(raw[u][i], xr[i], sx[i][0], sx[i][1]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float s = wave_sum(acc[u]);
            if (lane == 0 && r + u < row1) part[(r + u - blockIdx.x * wg_rows) * KW + kw] = s;
        }
    }
    __syncthreads();
    for (int t = threadIdx.x; t < wg_rows; t += blockDim.x) {
        const int row = blockIdx.x * wg_rows + t;
        if (row < rows) {
            float s = 0.f;
            for (int k = 0; k < KW; ++k) s += part[t * KW + k];
            yb[row] = s;
        }
    }
}

// ---------------------------------------------------------------------------
// DTypeTernary int8 path
// ---------------------------------------------------------------------------

// One block computes rows [blockIdx.x*rows_per_block, ...) for batch row blockIdx.y.
// LDS: xq permuted so that byte b of word (g*4+k) is xq[16g + 4b + k], matching
// the byte spread (codes >> 2k) & 0x03030303 of a 16-code dword.
__global__ void __launch_bounds__(256) k_ternary_i8(const uint8_t* __restrict__ codes, float scale, int rows, int K,
                                                   const float* __restrict__ x, float* __restrict__ y,
                                                   int32_t* __restrict__ acc_out, float* __restrict__ act_out,
                                                   int rows_per_block) {
    extern __shared__ uint32_t lds[];  // K/4 words of permuted xq (K%16==0) or K plain bytes
    __shared__ float red_f[4];
    __shared__ int red_i[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.y;
    const float* xb = x + int64_t(b) * K;

    // quantizeActsI8 (layers/dense/simd.go:526-549): absmax, f32 scale, round half away.
    float m = 0.f;
    for (int j = tid; j < K; j += 256) m = fmaxf(m, fabsf(xb[j]));
    m = wave_max(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    float act = m / 127.0f;
    if (act == 0.0f) act = 1.0f;
    const bool fast = (K % 64) == 0;
    uint8_t* l8 = reinterpret_cast<uint8_t*>(lds);
    int sq = 0;
    for (int j = tid; j < K; j += 256) {
        float t = xb[j] / act;
        int q = int(roundf(t));
        q = q > 127 ? 127 : (q < -128 ? -128 : q);
        sq += q;
        const int pos = fast ? ((j >> 4) * 16 + (j & 3) * 4 + ((j & 15) >> 2)) : j;
        l8[pos] = uint8_t(int8_t(q));
    }
    sq = wave_sum_i(sq);
    if (lane == 0) red_i[wave] = sq;
    __syncthreads();
    sq = red_i[0] + red_i[1] + red_i[2] + red_i[3];
    if (act_out && blockIdx.x == 0 && tid == 0) act_out[b] = act;

    const int r0 = blockIdx.x * rows_per_block;
    const int r1 = min(rows, r0 + rows_per_block);
    const int64_t row_bytes = K / 4;
    for (int r = r0 + wave; r < r1; r += 4) {
        int acc = 0;
        if (fast) {
            const uint4* rowp = reinterpret_cast<const uint4*>(codes + int64_t(r) * row_bytes);
            for (int c = lane; c < K / 64; c += kWave) {
                const uint4 v = rowp[c];
                const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t* xw = lds + (c * 4 + d) * 4;
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        acc = __builtin_amdgcn_sdot4(int((wd[d] >> (2 * k)) & 0x03030303u), int(xw[k]), acc, false);
                }
            }
            acc = wave_sum_i(acc) - sq;  // codes are t+1: sum (t+1)*xq - sum xq
        } else {
            const int64_t base = int64_t(r) * K;
            for (int j = lane; j < K; j += kWave) {
                const int64_t i = base + j;
                const int t = int((codes[i >> 2] >> ((i & 3) * 2)) & 3u) - 1;
                acc += t * int(int8_t(l8[j]));
            }
            acc = wave_sum_i(acc);
        }
        if (lane == 0) {
            if (acc_out) acc_out[int64_t(b) * rows + r] = acc;
            if (y) y[int64_t(b) * rows + r] = float(acc) * act * scale;  // simd.go:142
        }
    }
}

RawArgs raw_args(const DevBlob& b) {
    RawArgs a;
    a.raw = b.raw;
    a.raw_len = b.raw_len;
    a.scales = b.scales;
    a.n_scales = b.n_scales;
    a.rows = b.rows;
    a.cols = b.cols;
    a.iq_bits = b.iq_bits;
    a.iq_sg = b.iq_sg;
    a.g128 = (b.fmt == FMT_BINARY && b.block_weights == 128) ? 1 : 0;
    return a;
}

template <int F>
int launch_raw(const DevBlob& b, const float* x, float* y, int batch, hipStream_t s) {
    dim3 grid(unsigned((b.rows + 3) / 4), unsigned(batch));
    hipLaunchKernelGGL(k_gemv_raw<F>, grid, dim3(256), 0, s, raw_args(b), x, y);
    return int(hipGetLastError());
}

template <int F>
int launch_raw_t(const DevBlob& b, const float* gy, float* gx, int batch, hipStream_t s, float* part, int nsplit) {
    const int rps = int((b.rows + nsplit - 1) / nsplit);
    dim3 grid(unsigned((b.cols + 255) / 256), unsigned(nsplit), unsigned(batch));
    hipLaunchKernelGGL(k_gemvt_raw<F>, grid, dim3(256), 0, s, raw_args(b), gy, part, rps);
    hipLaunchKernelGGL(k_gemvt_reduce, dim3(unsigned((b.cols + 255) / 256), unsigned(batch)), dim3(256), 0, s, part,
                       gx, b.cols, nsplit);
    return int(hipGetLastError());
}

using RawFn = int (*)(const DevBlob&, const float*, float*, int, hipStream_t);
using RawTFn = int (*)(const DevBlob&, const float*, float*, int, hipStream_t, float*, int);

template <int F>
constexpr RawFn raw_fn() { return &launch_raw<F>; }

RawFn pick_raw(int fmt) {
    switch (fmt) {
    case FMT_Q4_0: return launch_raw<FMT_Q4_0>;
    case FMT_Q8_0: return launch_raw<FMT_Q8_0>;
    case FMT_Q4_1: return launch_raw<FMT_Q4_1>;
    case FMT_Q5_0: return launch_raw<FMT_Q5_0>;
    case FMT_Q5_1: return launch_raw<FMT_Q5_1>;
    case FMT_Q2_K: return launch_raw<FMT_Q2_K>;
    case FMT_Q3_K: return launch_raw<FMT_Q3_K>;
    case FMT_Q4_K: return launch_raw<FMT_Q4_K>;
    case FMT_Q5_K: return launch_raw<FMT_Q5_K>;
    case FMT_Q6_K: return launch_raw<FMT_Q6_K>;
    case FMT_IQ1_S: return launch_raw<FMT_IQ1_S>;
    case FMT_IQ2_XXS: return launch_raw<FMT_IQ2_XXS>;
    case FMT_IQ2_XS: return launch_raw<FMT_IQ2_XS>;
    case FMT_IQ3_XXS: return launch_raw<FMT_IQ3_XXS>;
    case FMT_IQ3_S: return launch_raw<FMT_IQ3_S>;
    case FMT_IQ4_NL: return launch_raw<FMT_IQ4_NL>;
    case FMT_IQ4_XS: return launch_raw<FMT_IQ4_XS>;
    case FMT_TERNARY: return launch_raw<FMT_TERNARY>;
    case FMT_BINARY: return launch_raw<FMT_BINARY>;
    default: return nullptr;
    }
}
RawTFn pick_raw_t(int fmt) {
    switch (fmt) {
    case FMT_Q4_0: return launch_raw_t<FMT_Q4_0>;
    case FMT_Q8_0: return launch_raw_t<FMT_Q8_0>;
    case FMT_Q4_1: return launch_raw_t<FMT_Q4_1>;
    case FMT_Q5_0: return launch_raw_t<FMT_Q5_0>;
    case FMT_Q5_1: return launch_raw_t<FMT_Q5_1>;
    case FMT_Q2_K: return launch_raw_t<FMT_Q2_K>;
    case FMT_Q3_K: return launch_raw_t<FMT_Q3_K>;
    case FMT_Q4_K: return launch_raw_t<FMT_Q4_K>;
    case FMT_Q5_K: return launch_raw_t<FMT_Q5_K>;
    case FMT_Q6_K: return launch_raw_t<FMT_Q6_K>;
    case FMT_IQ1_S: return launch_raw_t<FMT_IQ1_S>;
    case FMT_IQ2_XXS: return launch_raw_t<FMT_IQ2_XXS>;
    case FMT_IQ2_XS: return launch_raw_t<FMT_IQ2_XS>;
    case FMT_IQ3_XXS: return launch_raw_t<FMT_IQ3_XXS>;
    case FMT_IQ3_S: return launch_raw_t<FMT_IQ3_S>;
    case FMT_IQ4_NL: return launch_raw_t<FMT_IQ4_NL>;
    case FMT_IQ4_XS: return launch_raw_t<FMT_IQ4_XS>;
    case FMT_TERNARY: return launch_raw_t<FMT_TERNARY>;
    case FMT_BINARY: return launch_raw_t<FMT_BINARY>;
    default: return nullptr;
    }
}

PlanarArgs planar_args(const DevBlob& b) {
    PlanarArgs a;
    a.codes = b.codes;
    a.codes_hi = b.codes_hi;
    a.blk = b.blk_scale;
    a.grp = b.grp;
    a.nchunks = b.cols / 32;
    return a;
}

// Chooses chunks-per-lane (CPL) and waves splitting K (KW) so a row's chunks
// are covered, then rows-per-wave so the grid holds ~16 waves per CU.
template <class P>
int launch_planar(const DevBlob& b, const float* x, float* y, int batch, hipStream_t s) {
    const int64_t nch = b.cols / 32;
    int cpl, kw;
    if (nch <= 64) { cpl = 1; kw = 1; }
    else if (nch <= 128) { cpl = 2; kw = 1; }
    else if (nch <= 64 * 8) { cpl = 1; kw = int((nch + 63) / 64); }
    else if (nch <= 128 * 8) { cpl = 2; kw = int((nch + 127) / 128); }
    else if (nch <= 256 * 8) { cpl = 4; kw = int((nch + 255) / 256); }
    else return int(hipErrorInvalidValue);
    const int rw = std::max(1, 4 / kw);
    const int64_t target_waves = 256 * 16;
    int64_t rpw = (b.rows * kw + target_waves - 1) / target_waves;
    rpw = std::max<int64_t>(1, std::min<int64_t>(rpw, 64));
    const int64_t wg_rows = rw * rpw;
    dim3 grid(unsigned((b.rows + wg_rows - 1) / wg_rows), unsigned(batch));
    dim3 block(unsigned(64 * kw * rw));
    const size_t lds = size_t(wg_rows * kw) * sizeof(float);
    const PlanarArgs a = planar_args(b);
    const int R = int(b.rows), RPW = int(rpw);
    switch (cpl) {
    case 1: hipLaunchKernelGGL((k_gemv_planar<P, 1, 4>), grid, block, lds, s, a, x, y, R, kw, RPW); break;
    case 2: hipLaunchKernelGGL((k_gemv_planar<P, 2, 4>), grid, block, lds, s, a, x, y, R, kw, RPW); break;
    default: hipLaunchKernelGGL((k_gemv_planar<P, 4, 2>), grid, block, lds, s, a, x, y, R, kw, RPW); break;
    }
    return int(hipGetLastError());
}

int launch_ternary(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s) {
    const int rows = int(b.rows), K = int(b.cols);
    const int rpb = 16;
    dim3 grid(unsigned((rows + rpb - 1) / rpb), unsigned(batch));
    const size_t lds = size_t((K + 3) / 4) * 4;
    hipLaunchKernelGGL(k_ternary_i8, grid, dim3(256), lds, s, b.codes, b.tensor_scale, rows, K, x, y, acc, act, rpb);
    return int(hipGetLastError());
}

}  // namespace

int launch_matvec(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (b.rows == 0 || batch == 0) return 0;
    switch (b.layout) {
    case LAYOUT_K_PLANAR:
        if (b.fmt == FMT_Q4_K) return launch_planar<PolQ4K>(b, d_x, d_y, batch, s);
        if (b.fmt == FMT_Q6_K) return launch_planar<PolQ6K>(b, d_x, d_y, batch, s);
        return int(hipErrorInvalidValue);
    case LAYOUT_Q8_PLANAR: return launch_planar<PolQ8>(b, d_x, d_y, batch, s);
    case LAYOUT_Q4_PLANAR: return launch_planar<PolQ4>(b, d_x, d_y, batch, s);
    case LAYOUT_TERNARY_I8: return launch_ternary(b, d_x, d_y, nullptr, nullptr, batch, s);
    default: {
        RawFn f = pick_raw(b.fmt);
        if (!f) return int(hipErrorInvalidValue);
        return f(b, d_x, d_y, batch, s);
    }
    }
}

size_t matvec_t_scratch_floats(const DevBlob& b, int batch) {
    const int64_t nsplit = std::max<int64_t>(1, std::min<int64_t>(64, b.rows / 64));
    return size_t(nsplit) * size_t(b.cols) * size_t(batch);
}

int launch_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (b.rows == 0 || batch == 0) return 0;
    if (b.layout != LAYOUT_RAW) return int(hipErrorInvalidValue);
    RawTFn f = pick_raw_t(b.fmt);
    if (!f) return int(hipErrorInvalidValue);
    const int nsplit = int(std::max<int64_t>(1, std::min<int64_t>(64, b.rows / 64)));
    return f(b, d_gy, d_gx, batch, s, d_scratch, nsplit);
}

int launch_ternary_acc(const DevBlob& b, const float* d_x, int32_t* d_acc, float* d_act, int batch, void* stream) {
    if (b.layout != LAYOUT_TERNARY_I8) return int(hipErrorInvalidValue);
    return launch_ternary(b, d_x, nullptr, d_acc, d_act, batch, static_cast<hipStream_t>(stream));
}

}  // namespace wv
