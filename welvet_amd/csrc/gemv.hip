// gemv.hip — gfx950 kernels of the Dense MatVec path.
//
// Three families:
//   * k_gemv_raw16 / k_gemvt_raw16 (cols % 256 == 0) and k_gemv_raw / k_gemvt_raw (any shape,
//     including blocks that straddle rows): the reference layout as uploaded
//     (LAYOUT_RAW), every format; semantics follow the reference decoders
//     (quant/*.go forEach* / unpack*), accumulating in f32.
//   * the row-interleaved fast path lives in gemv_rpl.hip, the weights.Store
//     DTypes (int8 path, f32 and f64 products) in native.hip;
//   * k_bias_act: Dense's bias + activation epilogue for the layouts whose
//     GEMV has no fused one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>

#include "epilogue.h"
#include "wave_ops.h"
#include "wv_internal.h"

namespace wv {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) { return wave_total(v); }
__device__ __forceinline__ int wave_sum_i(int v) { return wave_total_i(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_maximum(v); }

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
    const float* mins;  // AffinePacked biases, one per group of `group` weights
    int64_t group;
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
    } else if constexpr (F == FMT_AFFINE) {  // decodeRowAffine (affine_g64.go:124-161), 4-bit codes
        const uint32_t code = (uint32_t(a.raw[i >> 1]) >> ((i & 1) * 4)) & 15u;
        const int64_t g = i / a.group;  // cols % group == 0: flat group = row * groups_per_row + col / group
        return a.scales[g] * float(code) + a.mins[g];
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

// ---------------------------------------------------------------------------
// Vectorized decode of the reference layout (cols % 256 == 0).
//
// Every format stores, per 16 consecutive weights of a row, an LSB-first run
// of 16 codes of BITS bits (2*BITS bytes, byte aligned) sharing one affine
// map w = alpha * f(q) + beta (f = identity, except the IQ4_NL grid and the
// ternary {-1, 0, +1, 0} table; Q4_0 and Q8_0 become affine through q ^ bias).
// So sum_k w_k x_k = alpha * sum_k f(q_k) x_k + beta * sum_k x_k. A lane takes
// one such 16-weight run at a time for R = 4 rows at once, reusing its 16 x
// values (read through L1) across the rows; the codes come in as aligned
// dwords and are realigned with v_alignbyte and cut with bit-field extracts
// at compile-time offsets.
// ---------------------------------------------------------------------------

struct Grp {
    const uint8_t* codes;  // first code byte (2-byte aligned)
    float alpha, beta;
};

template <int F>
struct RawF;
template <> struct RawF<FMT_Q4_0> {
    static constexpr int BITS = 4;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // q4_0.go:93-99
        const uint8_t* o = a.raw + (f >> 5) * 20;
        const float s = ld_f32(o);
        return {o + 4 + ((f >> 4) & 1) * 8, s, -8.0f * s};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q ^ 8u); }
};
template <> struct RawF<FMT_Q8_0> {
    static constexpr int BITS = 8;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // q8_0.go:58-63
        const uint8_t* o = a.raw + (f >> 5) * 36;
        const float s = ld_f32(o);
        return {o + 4 + ((f >> 4) & 1) * 16, s, -128.0f * s};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q ^ 0x80u); }
};
template <> struct RawF<FMT_Q4_1> {
    static constexpr int BITS = 4;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // q4_1.go:63-72
        const uint8_t* o = a.raw + (f >> 5) * 24;
        return {o + 8 + ((f >> 4) & 1) * 8, ld_f32(o), ld_f32(o + 4)};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};
template <> struct RawF<FMT_Q5_0> {
    static constexpr int BITS = 5;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // q5_0.go:55-63
        const uint8_t* o = a.raw + (f >> 5) * 24;
        const float s = ld_f32(o);
        return {o + 4 + ((f >> 4) & 1) * 10, s, -16.0f * s};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};
template <> struct RawF<FMT_Q5_1> {
    static constexpr int BITS = 5;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // q5_1.go:59-67
        const uint8_t* o = a.raw + (f >> 5) * 28;
        return {o + 8 + ((f >> 4) & 1) * 10, ld_f32(o), ld_f32(o + 4)};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};
template <int F>
struct RawK {  // kquant.go:178-188: sc = d*u/255 (0 -> d/255), w = dmin*m/127 + q*sc, Q6_K: sc*(q - 32)
    using S = KSpecC<F>;
    static constexpr int BITS = S::bits;
    static constexpr int SBB = 8 + 16 + (S::has_dmin ? 16 : 0) + 256 * S::bits / 8;
    static constexpr int QOFF = S::has_dmin ? 40 : 24;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {
        const uint8_t* o = a.raw + (f >> 8) * SBB;
        const int g = int((f >> 4) & 15);
        const float d = ld_f32(o);
        float sc = d * float(o[8 + g]) / 255.0f;
        if (sc == 0.0f) sc = d / 255.0f;
        if constexpr (S::has_dmin) {
            const float mn = ld_f32(o + 4) * float(int8_t(o[24 + g])) / 127.0f;
            return {o + QOFF + g * 2 * BITS, sc, mn};
        } else {
            return {o + QOFF + g * 2 * BITS, sc, -float(S::mid) * sc};
        }
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};
template <> struct RawF<FMT_Q2_K> : RawK<FMT_Q2_K> {};
template <> struct RawF<FMT_Q3_K> : RawK<FMT_Q3_K> {};
template <> struct RawF<FMT_Q4_K> : RawK<FMT_Q4_K> {};
template <> struct RawF<FMT_Q5_K> : RawK<FMT_Q5_K> {};
template <> struct RawF<FMT_Q6_K> : RawK<FMT_Q6_K> {};
template <int F, int B, int SG>
struct RawIQ {  // iq.go:169-207, one scale per SG weights of the flat stream
    static constexpr int BITS = B;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {
        const float s = a.scales[f / SG];
        const uint8_t* c = a.raw + (f * B) / 8;
        if constexpr (B == 1) return {c, 2.0f * s, -s};
        else if constexpr (F == FMT_IQ4_NL) return {c, s, 0.0f};
        else {
            constexpr float mid = B == 2 ? 1.5f : B == 3 ? 3.5f : 7.5f;
            return {c, s, -mid * s};
        }
    }
    static __device__ float fq(uint32_t q, const float* tab) {
        if constexpr (F == FMT_IQ4_NL) return tab[q & 15];  // the grid staged in LDS
        else return float(q);
    }
};
template <> struct RawF<FMT_IQ1_S> : RawIQ<FMT_IQ1_S, 1, 32> {};
template <> struct RawF<FMT_IQ2_XXS> : RawIQ<FMT_IQ2_XXS, 2, 32> {};
template <> struct RawF<FMT_IQ2_XS> : RawIQ<FMT_IQ2_XS, 2, 16> {};
template <> struct RawF<FMT_IQ3_XXS> : RawIQ<FMT_IQ3_XXS, 3, 32> {};
template <> struct RawF<FMT_IQ3_S> : RawIQ<FMT_IQ3_S, 3, 16> {};
template <> struct RawF<FMT_IQ4_NL> : RawIQ<FMT_IQ4_NL, 4, 32> {};
template <> struct RawF<FMT_IQ4_XS> : RawIQ<FMT_IQ4_XS, 4, 16> {};
template <> struct RawF<FMT_TERNARY> {
    static constexpr int BITS = 2;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // ternary.go:53-82
        const int64_t g = f >> 4;
        return {a.raw + g * 4, g < a.n_scales ? a.scales[g] : 1.0f, 0.0f};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return q == 0 ? -1.0f : (q == 2 ? 1.0f : 0.0f); }
};
template <> struct RawF<FMT_AFFINE> {
    static constexpr int BITS = 4;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {  // affine_g64.go:140-160
        const int64_t g = f / a.group;
        return {a.raw + (f >> 1), a.scales[g], a.mins[g]};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};
template <> struct RawF<FMT_BINARY> {
    static constexpr int BITS = 1;
    static __device__ Grp grp(const RawArgs& a, int64_t row, int64_t f) {
        if (a.g128) {  // binary_g128.go:107-139, row-aligned words and groups
            const int64_t col = f - row * a.cols;
            const int64_t si = row * (a.cols >> 7) + (col >> 7);
            const float s = si < a.n_scales ? a.scales[si] : 1.0f;
            return {a.raw + (row * (a.cols >> 5) + (col >> 5)) * 4 + ((col >> 4) & 1) * 2, 2.0f * s, -s};
        }
        const int64_t g = f >> 5;  // binary.go:49-75
        const float s = g < a.n_scales ? a.scales[g] : 1.0f;
        return {a.raw + g * 4 + ((f >> 4) & 1) * 2, 2.0f * s, -s};
    }
    static __device__ float fq(uint32_t q, const float* tab) { return float(q); }
};

// The dword-aligned start of a run's code bytes at p (2-byte aligned) and the
// byte offset of p in it. The start is formed by pointer arithmetic on p, not
// through an integer: an integer round trip loses the global address space,
// and the loads become flat loads, which also count against the LDS counter
// so that every wait on them is a full wait.
__device__ __forceinline__ const uint32_t* run_base(const uint8_t* p, uint32_t& mis) {
    mis = uint32_t(reinterpret_cast<uintptr_t>(p)) & 3u;
    return reinterpret_cast<const uint32_t*>(p - mis);
}
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w, int k) {
    const int bit = k * BITS, wi = bit >> 5, off = bit & 31;
    if (off + BITS <= 32) return (w[wi] >> off) & ((1u << BITS) - 1u);
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], off) & ((1u << BITS) - 1u);
}

// One block = 4 waves = 4/KW groups of R = 4 rows; the KW waves of a group
// take interleaved runs of the same rows (K split inside the block) and
// their row sums meet in LDS in a fixed order.
template <int F, int U, int KW>
__global__ void __launch_bounds__(256) k_gemv_raw16(RawArgs a, const float* __restrict__ x, float* __restrict__ y) {
    using P = RawF<F>;
    constexpr int R = 4;  // rows per wave
    __shared__ float red[4][R];
    __shared__ float tab[16];  // IQ4_NL grid: a per-lane index into a register table would go through scratch
    if constexpr (F == FMT_IQ4_NL) {
        if (threadIdx.x < 16) tab[threadIdx.x] = kIQ4NLGrid[threadIdx.x];
        __syncthreads();
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kp = wave % KW;  // this wave's K part
    const int64_t row0 = (int64_t(blockIdx.x) * (4 / KW) + wave / KW) * R;
    if (KW == 1 && row0 >= a.rows) return;  // with KW > 1 every wave reaches the barrier below
    const int b = blockIdx.y;
    const float* xb = x + int64_t(b) * a.cols;
    const int64_t nsg = a.cols >> 4;
    int64_t rowc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowc[r] = min<int64_t>(row0 + r, a.rows - 1);
    // U runs per lane in flight: every load of U consecutive runs (lane, lane+64, ...)
    // is issued before any of them is used; indices past the row are clamped
    // to its last run (read, not used), so the load phase has no branches.
    constexpr int NB = 2 * P::BITS, NW = (NB + 2 + 3) / 4;
    // Load order (measured at 4096->14336): formats whose header is a plain
    // scale (and min) issue every row's codes first and the headers after;
    // the k-quants (two exact divisions per run), IQ4_NL and Affine keep each
    // row's header arithmetic next to its loads, where it overlaps the other
    // rows' loads (two-phase: Q4_1 -13 %, Q5_0 -12 %, Binary -10 %; Q5_K +26 %).
    constexpr bool kTwoPhase = !(F >= FMT_Q2_K && F <= FMT_Q6_K) && F != FMT_IQ4_NL && F != FMT_AFFINE;
    float acc[R] = {};
    for (int64_t s0 = kp * 64 + lane; s0 < nsg; s0 += 64 * KW * U) {
        float4 xq[U][4];
        Grp g[U][R];
        uint32_t dw[U][R][NW], mis[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c0 = min<int64_t>(s0 + 64 * KW * u, nsg - 1) << 4;
            const float4* xp = reinterpret_cast<const float4*>(xb + c0);
#pragma unroll
            for (int k = 0; k < 4; ++k) xq[u][k] = xp[k];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if constexpr (!kTwoPhase) g[u][r] = P::grp(a, rowc[r], rowc[r] * a.cols + c0);
                const uint32_t* base =
                    run_base(kTwoPhase ? P::grp(a, rowc[r], rowc[r] * a.cols + c0).codes : g[u][r].codes, mis[u][r]);
#pragma unroll
                for (int i = 0; i < NW; ++i) dw[u][r][i] = base[i];
            }
        }
        if constexpr (kTwoPhase) {
            // The loads above used only the codes address of grp(); its header
            // loads and alpha/beta arithmetic follow here, so no header
            // arithmetic waits between one row's loads and the next's.
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t c0 = min<int64_t>(s0 + 64 * KW * u, nsg - 1) << 4;
#pragma unroll
                for (int r = 0; r < R; ++r) g[u][r] = P::grp(a, rowc[r], rowc[r] * a.cols + c0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + 64 * KW * u >= nsg) continue;
            const float xv[16] = {xq[u][0].x, xq[u][0].y, xq[u][0].z, xq[u][0].w, xq[u][1].x, xq[u][1].y,
                                  xq[u][1].z, xq[u][1].w, xq[u][2].x, xq[u][2].y, xq[u][2].z, xq[u][2].w,
                                  xq[u][3].x, xq[u][3].y, xq[u][3].z, xq[u][3].w};
            float xs = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) xs += xv[k];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t w[(NB + 3) / 4];  // the run's bytes realigned to a dword boundary
#pragma unroll
                for (int i = 0; i < (NB + 3) / 4; ++i)
                    w[i] = __builtin_amdgcn_alignbyte(i + 1 < NW ? dw[u][r][i + 1] : 0u, dw[u][r][i], mis[u][r]);
                float d = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) d = fmaf(P::fq(code_at<P::BITS>(w, k), tab), xv[k], d);
                acc[r] = fmaf(g[u][r].alpha, d, fmaf(g[u][r].beta, xs, acc[r]));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[r]);
        if (KW == 1) {
            if (lane == 0 && row0 + r < a.rows) y[int64_t(b) * a.rows + row0 + r] = v;
        } else if (lane == 0) {
            red[wave][r] = v;
        }
    }
    if constexpr (KW > 1) {
        __syncthreads();
        const int t = threadIdx.x;
        if (t < (4 / KW) * R) {
            const int grp = t / R, r = t % R;
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < KW; ++k) v += red[grp * KW + k][r];
            const int64_t row = (int64_t(blockIdx.x) * (4 / KW) + grp) * R + r;
            if (row < a.rows) y[int64_t(b) * a.rows + row] = v;
        }
    }
}

// MatVecT on the reference layout by runs (cols % 256 == 0, the layouts of
// k_gemv_raw16): gx[c] += sum_r w(r,c) gy[r] with w = alpha*f(q) + beta per
// run of 16 columns. Lane = one run of a 64-run column tile (blockIdx.x); the
// kRawTWaves waves of a block take rows r0 + w, r0 + w + kRawTWaves, ... of
// the block's row slice (blockIdx.y). A lane keeps 16 column sums of
// (gy*alpha)*f(q) and one sum of gy*beta for the whole run, with the runs of
// U rows in flight, and the waves' sums meet in LDS in wave order. Several
// slices write part[(b*slices + slice)*cols + c] for k_gemvt_reduce; one
// slice adds to gx directly.
constexpr int kRawTWaves = 8;
template <int F>
__global__ void __launch_bounds__(64 * kRawTWaves) k_gemvt_raw16(RawArgs a, const float* __restrict__ gy,
                                                                  float* __restrict__ gx, float* __restrict__ part,
                                                                  int rows_per_slice) {
    using P = RawF<F>;
    constexpr int WB = kRawTWaves, U = 4;
    constexpr int NB = 2 * P::BITS, NW = (NB + 2 + 3) / 4;
    __shared__ float tab[16];
    __shared__ float red[WB][64 * 16];
    if constexpr (F == FMT_IQ4_NL) {
        if (threadIdx.x < 16) tab[threadIdx.x] = kIQ4NLGrid[threadIdx.x];
        __syncthreads();
    }
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int slice = blockIdx.y, b = blockIdx.z;
    const int64_t nsg = a.cols >> 4;
    const int64_t c0 = min<int64_t>(int64_t(blockIdx.x) * 64 + lane, nsg - 1) << 4;
    const int64_t r0 = int64_t(slice) * rows_per_slice;
    const int64_t r1 = min<int64_t>(a.rows, r0 + rows_per_slice);
    const float* g = gy + int64_t(b) * a.rows;
    float acc[16] = {};
    float off = 0.f;
    for (int64_t rb = r0 + wave; rb < r1; rb += WB * U) {
        // Rows past the slice are clamped to its last row (read, not used).
        // Phase 1 issues the code loads of all U rows (only the codes
        // address of grp() is used, so its header loads and arithmetic are
        // dropped here); phase 2 calls grp() again for alpha and beta, whose
        // header loads queue behind the codes. A barrier keeps each phase's
        // loads ahead of the arithmetic that waits on them.
        int64_t rr[U];
        uint32_t dw[U][NW], mis[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            rr[u] = min<int64_t>(rb + WB * u, r1 - 1);
            const uint32_t* base = run_base(P::grp(a, rr[u], rr[u] * a.cols + c0).codes, mis[u]);
#pragma unroll
            for (int i = 0; i < NW; ++i) dw[u][i] = base[i];
        }
        __builtin_amdgcn_sched_barrier(0);
        Grp gr[U];
        float gv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            gr[u] = P::grp(a, rr[u], rr[u] * a.cols + c0);
            gv[u] = g[rr[u]];
        }
        __builtin_amdgcn_sched_barrier(0);
        // No branch per row: a branch would let the compiler sink that row's
        // loads into it, and the rows' loads would no longer overlap. Rows
        // past the slice add exact zeros (selects, so no 0 * inf).
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool live = rb + WB * u < r1;
            uint32_t w[(NB + 3) / 4];
#pragma unroll
            for (int i = 0; i < (NB + 3) / 4; ++i)
                w[i] = __builtin_amdgcn_alignbyte(i + 1 < NW ? dw[u][i + 1] : 0u, dw[u][i], mis[u]);
            const float coef = live ? gv[u] * gr[u].alpha : 0.f;
            off += live ? gv[u] * gr[u].beta : 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[k] = fmaf(coef, P::fq(code_at<P::BITS>(w, k), tab), acc[k]);
        }
    }
    float* rw = red[wave] + lane * 16;
#pragma unroll
    for (int k = 0; k < 16; ++k) rw[k] = acc[k] + off;
    __syncthreads();
    for (int cc = threadIdx.x; cc < 64 * 16; cc += 64 * WB) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < WB; ++w) v += red[w][cc];
        const int64_t col = int64_t(blockIdx.x) * 1024 + cc;
        if (col >= a.cols) continue;
        if (gridDim.y == 1)
            gx[int64_t(b) * a.cols + col] += v;
        else
            part[(int64_t(b) * gridDim.y + slice) * a.cols + col] = v;
    }
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

__global__ void __launch_bounds__(64) k_gemvt_reduce(const float* __restrict__ part, float* __restrict__ gx,
                                                     int64_t cols, int nsplit) {
    const int64_t c = int64_t(blockIdx.x) * 64 + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= cols) return;
    // Partials are added in split order, then to gx. Each group of 8 loads
    // (clamped to the last split, the extra ones masked out of the sum) and
    // the gx load are issued before any add, so a step with up to 8 splits
    // pays one memory round trip.
    const float* p = part + int64_t(b) * nsplit * cols + c;
    float* g = gx + int64_t(b) * cols + c;
    const float g0 = *g;
    float s = 0.0f;
    for (int k = 0; k < nsplit; k += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p[int64_t(min(k + j, nsplit - 1)) * cols];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (k + j < nsplit) s += v[j];
    }
    *g = g0 + s;
}

// applyBiasAct (layers/dense/dense.go:145-167) over y[batch][rows]: pre =
// f32(y + bias) written to `pre`, post = f32(act(f64(pre))) to `post`. y and
// pre may be the same buffer (in place; each thread reads its element before
// writing it), so neither is declared __restrict__.
__global__ void __launch_bounds__(256) k_bias_act(const float* y, float* pre,
                                                  float* __restrict__ post, const double* __restrict__ bias, int act,
                                                  int64_t rows, int64_t n) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    store_bias_act(pre, post, i, y[i], bias, i % rows, act);
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
    a.mins = b.mins;
    a.group = b.block_weights > 0 ? b.block_weights : 64;
    return a;
}

// The run-vectorized kernel needs whole runs of 16 weights per row and the
// format's standard IQ bit width and scale group (Meta may override them).
template <int F>
bool raw16_ok(const DevBlob& b) {
    if (b.cols % 256 != 0) return false;
    if constexpr (F >= FMT_IQ1_S && F <= FMT_IQ4_XS) {
        IQSpec sp;
        iq_spec(F, sp);
        return b.iq_bits == sp.bits && b.iq_sg == sp.sg;
    }
    if constexpr (F == FMT_BINARY) return b.block_weights != 128 || b.cols % 128 == 0;
    if constexpr (F == FMT_AFFINE) return b.block_weights % 16 == 0;  // a run of 16 never straddles groups
    return true;
}

template <int F>
int launch_raw(const DevBlob& b, const float* x, float* y, int batch, hipStream_t s) {
    if (raw16_ok<F>(b)) {
        // IQ4_NL's grid lookups (LDS) overlap the next runs' loads; for the
        // others the extra registers of 4 runs in flight cost more than they hide.
        constexpr int U = F == FMT_IQ4_NL ? 4 : 1;
        // K parts per row group (measured at 4096->14336): the fewest that give
        // about 4 waves per SIMD, never more parts than the row has runs of 64;
        // IQ4_NL's 4-run ring already holds as many registers as a SIMD has.
        const int64_t quads = (b.rows + 3) / 4, nsg = b.cols / 16;
        int kw = U > 1 || quads >= 4096 ? 1 : (quads * 2 >= 4096 ? 2 : 4);
        while (kw > 1 && nsg < 64 * kw) kw /= 2;
        const dim3 g(unsigned((quads * kw + 3) / 4), unsigned(batch));
        if (kw == 4)
            hipLaunchKernelGGL((k_gemv_raw16<F, U, 4>), g, dim3(256), 0, s, raw_args(b), x, y);
        else if (kw == 2)
            hipLaunchKernelGGL((k_gemv_raw16<F, U, 2>), g, dim3(256), 0, s, raw_args(b), x, y);
        else
            hipLaunchKernelGGL((k_gemv_raw16<F, U, 1>), g, dim3(256), 0, s, raw_args(b), x, y);
        return int(hipGetLastError());
    }
    dim3 grid(unsigned((b.rows + 3) / 4), unsigned(batch));
    hipLaunchKernelGGL(k_gemv_raw<F>, grid, dim3(256), 0, s, raw_args(b), x, y);
    return int(hipGetLastError());
}

// Row slices of the run-vectorized MatVecT: about kRawTBlocks blocks over the
// column tiles (measured on MI355X), at most 128 slices and at least 64 rows
// per slice (so the partials stay small next to the weights).
constexpr int kRawTBlocks = 1024;
int raw_t16_slices(const DevBlob& b) {
    const int64_t tiles = (b.cols / 16 + 63) / 64;
    const int64_t want = (kRawTBlocks + tiles - 1) / tiles;
    return int(std::max<int64_t>(1, std::min<int64_t>({want, 128, b.rows / 64})));
}
// Row splits of the per-weight MatVecT.
int raw_t_splits(const DevBlob& b) { return int(std::max<int64_t>(1, std::min<int64_t>(64, b.rows / 64))); }

template <int F>
int launch_raw_t(const DevBlob& b, const float* gy, float* gx, int batch, hipStream_t s, float* part) {
    if (raw16_ok<F>(b)) {
        const int ns = raw_t16_slices(b);
        const int rps = int((b.rows + ns - 1) / ns);
        const dim3 grid(unsigned((b.cols / 16 + 63) / 64), unsigned(ns), unsigned(batch));
        hipLaunchKernelGGL(k_gemvt_raw16<F>, grid, dim3(64 * kRawTWaves), 0, s, raw_args(b), gy, gx, part, rps);
        if (ns > 1)
            hipLaunchKernelGGL(k_gemvt_reduce, dim3(unsigned((b.cols + 63) / 64), unsigned(batch)), dim3(64), 0, s,
                               part, gx, b.cols, ns);
        return int(hipGetLastError());
    }
    const int nsplit = raw_t_splits(b);
    const int rps = int((b.rows + nsplit - 1) / nsplit);
    dim3 grid(unsigned((b.cols + 255) / 256), unsigned(nsplit), unsigned(batch));
    hipLaunchKernelGGL(k_gemvt_raw<F>, grid, dim3(256), 0, s, raw_args(b), gy, part, rps);
    hipLaunchKernelGGL(k_gemvt_reduce, dim3(unsigned((b.cols + 63) / 64), unsigned(batch)), dim3(64), 0, s, part,
                       gx, b.cols, nsplit);
    return int(hipGetLastError());
}

using RawFn = int (*)(const DevBlob&, const float*, float*, int, hipStream_t);
using RawTFn = int (*)(const DevBlob&, const float*, float*, int, hipStream_t, float*);

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
    case FMT_AFFINE: return launch_raw<FMT_AFFINE>;
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
    case FMT_AFFINE: return launch_raw_t<FMT_AFFINE>;
    default: return nullptr;
    }
}

}  // namespace

size_t matvec_scratch_floats(const DevBlob& b, int batch) { return rpl_scratch_floats(b, batch); }

int launch_matvec(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, float* d_scratch,
                  const BiasAct* ba) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (b.rows == 0 || batch == 0) return 0;
    const bool epi = ba && ba->post;
    // The bias/activation epilogue runs as its own elementwise kernel: fused
    // into the GEMV store, its f64 activations cost the hot kernels ~5 % from
    // code size alone (measured on MI355X) even when unused.
    int e = 0;
    if (b.layout == LAYOUT_RPL) {
        e = launch_rpl(b, d_x, d_y, batch, s, RPL_STORE, nullptr, d_scratch);
    } else if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32) {
        e = launch_native_fwd(b, d_x, d_y, batch, s);
    } else {
        RawFn f = pick_raw(b.fmt);
        if (!f) return int(hipErrorInvalidValue);
        e = f(b, d_x, d_y, batch, s);
    }
    if (e || !epi) return e;
    return launch_bias_act(d_y, d_y, ba->post, ba->bias, ba->act, b.rows, batch, s);
}

int launch_bias_act(const float* d_y, float* d_pre, float* d_post, const double* d_bias, int act, int64_t rows,
                    int batch, void* stream) {
    const int64_t n = rows * int64_t(batch);
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_bias_act, dim3(unsigned((n + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream), d_y,
                       d_pre, d_post, d_bias, act, rows, n);
    return int(hipGetLastError());
}

void launch_gemvt_reduce(const float* part, float* gx, int64_t cols, int nsplit, int batch, void* stream) {
    hipLaunchKernelGGL(k_gemvt_reduce, dim3(unsigned((cols + 63) / 64), unsigned(batch)), dim3(64), 0,
                       static_cast<hipStream_t>(stream), part, gx, cols, nsplit);
}

size_t matvec_t_scratch_floats(const DevBlob& b, int batch) {
    if (batch <= 0) return 0;
    if (b.layout == LAYOUT_RPL) return rpl_t_scratch_floats(b.rpl, batch);
    if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32) return native_t_scratch_floats(b, batch);
    const int64_t n = std::max(raw_t_splits(b), raw_t16_slices(b));  // covers either kernel
    return size_t(n) * size_t(b.cols) * size_t(batch);
}

int launch_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (b.rows == 0 || batch == 0) return 0;
    if (b.layout == LAYOUT_RPL) return launch_rpl_matvec_t(b, d_gy, d_gx, batch, stream, d_scratch);
    if (b.layout == LAYOUT_NARROW || b.layout == LAYOUT_F32)
        return launch_native_t(b, d_gy, d_gx, batch, stream, reinterpret_cast<double*>(d_scratch));
    if (b.layout != LAYOUT_RAW) return int(hipErrorInvalidValue);
    RawTFn f = pick_raw_t(b.fmt);
    if (!f || !d_scratch) return int(hipErrorInvalidValue);
    return f(b, d_gy, d_gx, batch, s, d_scratch);
}

}  // namespace wv
