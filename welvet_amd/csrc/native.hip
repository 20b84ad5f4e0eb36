// native.hip — weights.Store payloads (FormatNone + DType) on the device.
//
// Three computations over the same resident codes:
//   * Dense's int8 path for the narrow DTypes (forwardSIMDNarrowI8 and
//     forwardSIMDInt8, layers/dense/simd.go:130-195, 303-326): activations
//     absmax-quantized to int8 (quantizeActsI8, simd.go:526-549), codes
//     expanded to int8 (expandNarrowToI8, simd.go:149-195), exact int32 dot
//     on v_dot4_i32_i8, y = f32(acc) * actScale * scale;
//   * the f32 FormatNone product (quant/none.go:37-51, Dense's
//     forwardSIMDMasterF32, simd.go:201-214) with f64 accumulation;
//   * weights.Store.MatVec / MatVecT on FormatNone stores
//     (weights/store.go:133-206 -> matVecNativeF64 / matVecTNativeF64,
//     weights/native.go:1120-1158): f64 sums over the decoded weights.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "wave_ops.h"
#include "wv_internal.h"

namespace wv {
namespace {

// Code width and int8 expansion of each narrow DType (expandNarrowToI8,
// layers/dense/simd.go:149-195): value = MUL * u - OFF with u the unsigned
// code after xor XR; Int8 bytes are used as signed values directly.
template <int F>
struct Narrow;
template <> struct Narrow<FMT_NATIVE_INT8> {  // nativeInt8Weights (simd.go:506-511)
    static constexpr int B = 8, MUL = 1, OFF = 0;
    static constexpr uint32_t XR = 0u, MASK = 0xFFFFFFFFu;
};
template <> struct Narrow<FMT_NATIVE_INT4> {  // nibble, q > 7 -> q - 16: (q ^ 8) - 8
    static constexpr int B = 4, MUL = 1, OFF = 8;
    static constexpr uint32_t XR = 0x88888888u, MASK = 0x0F0F0F0Fu;
};
template <> struct Narrow<FMT_NATIVE_INT2> {  // code - 2
    static constexpr int B = 2, MUL = 1, OFF = 2;
    static constexpr uint32_t XR = 0u, MASK = 0x03030303u;
};
template <> struct Narrow<FMT_NATIVE_TERNARY> {  // code - 1 (code 3 -> +2, as expandNarrowToI8)
    static constexpr int B = 2, MUL = 1, OFF = 1;
    static constexpr uint32_t XR = 0u, MASK = 0x03030303u;
};
template <> struct Narrow<FMT_NATIVE_BINARY> {  // bit set -> +1, clear -> -1: 2u - 1
    static constexpr int B = 1, MUL = 2, OFF = 1;
    static constexpr uint32_t XR = 0u, MASK = 0x01010101u;
};

// Unsigned B-bit code of flat element i in the device word order of the
// narrow codes (narrow_permute_words, runtime.hip): word i / E (E = 32/B)
// holds its element j = 4k + b at bits 8b + B*k, i.e. in byte
// 4*(i / E) + (j & 3) at bit B*(j >> 2). Int8 bytes are in element order.
template <int B>
__device__ __forceinline__ uint32_t ncode(const uint8_t* codes, int64_t i) {
    if constexpr (B == 8) {
        return codes[i];
    } else {
        constexpr int E = 32 / B;
        const int j = int(i % E);
        return (uint32_t(codes[(i / E) * 4 + (j & 3)]) >> (B * (j >> 2))) & ((1u << B) - 1u);
    }
}

// int8 value of flat element i (expandNarrowToI8).
template <int F>
__device__ __forceinline__ int narrow_i8(const uint8_t* codes, int64_t i) {
    using N = Narrow<F>;
    if constexpr (N::B == 8) {
        return int(int8_t(codes[i]));
    } else {
        return N::MUL * int(ncode<N::B>(codes, i) ^ (N::XR & ((1u << N::B) - 1u))) - N::OFF;
    }
}

// Four quantized activations (each in [-128, 127]) as the bytes of one dword.
__device__ __forceinline__ uint32_t pack_i8x4(int q0, int q1, int q2, int q3) {
    const uint32_t lo = __builtin_amdgcn_perm(uint32_t(q1), uint32_t(q0), 0x0C0C0400u);  // q0.b0, q1.b0
    const uint32_t hi = __builtin_amdgcn_perm(uint32_t(q3), uint32_t(q2), 0x0C0C0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// quantizeActsI8's q = round-half-away(f32(x / act)) clamped to [-128, 127].
// With inv = v_rcp(act) (1 ulp), t = x * inv is within 4e-5 of RN(x / act)
// while |t| <= 128 (relative 2^-23 + 2^-24 on t, 2^-24 on the quotient), so
// rint(t) is the reference's rounding unless t lies that close to a
// half-integer. Those rare elements, and every element when 1/act overflows
// (max|x| < 127 * 2^-128: thr = -1), are redone by the exact f32 division.
constexpr float kTieWindow = 1.2e-4f;
__device__ __forceinline__ float quant_inv(float act) { return __builtin_amdgcn_rcpf(act); }
__device__ __forceinline__ float quant_thr(float inv) { return inv <= 3.4e38f ? 0.5f - kTieWindow : -1.0f; }
// The rounding of t = x * inv when it is safe (returns false otherwise; NaN
// from inf * 0 or inf - inf fails the test too).
__device__ __forceinline__ bool quant_fast(float x, float inv, float thr, float& r) {
    const float t = x * inv;
    r = rintf(t);
    return fabsf(t - r) <= thr;
}
__device__ __forceinline__ int quant_clamp(float r) {
    const int q = int(r);
    return q > 127 ? 127 : (q < -128 ? -128 : q);
}
// One element, the exact division on a wave-uniform branch (a ballot), so it
// is not if-converted into every element's path.
__device__ __forceinline__ int quant_act(float x, float act, float inv, float thr) {
    float r;
    const bool exact = !quant_fast(x, inv, thr, r);
    if (__builtin_amdgcn_ballot_w64(exact)) {
        if (exact) r = roundf(x / act);
    }
    return quant_clamp(r);
}

// The narrow int8 GEMV when each row is a whole number of 16-byte code
// vectors (K % (128/B) == 0) and K <= 8192. A block of WB = blockDim/64 waves
// (up to 16, sized so the grid is about one block per CU) covers WB*RW rows of
// one batch row; every block quantizes all of x, so more threads per block
// shorten that serial prologue:
//  * x is requested first (NX float4 per thread), then the block's codes (NC
//    uint4 per lane per row), so the activation quantization overlaps the
//    codes' arrival;
//  * absmax over x, act = max/127 (1 if 0), q as quant_act;
//  * xq goes to LDS laid out for the dot: code vector c holds E = 32/B codes
//    per dword; in the device word order dword d, shifted by k*B (k < KS =
//    8/B) and masked, offers in byte b the code of element c*(128/B) + d*E +
//    4k + b, so LDS dword (d*nU + c)*KS + k holds those four xq bytes: the
//    quantized float4 of x that starts at that element, one whole-dword store
//    per float4. Lane c reads its KS dwords per d once for all its rows;
//  * acc = MUL * sum u*xq - OFF * sum xq on v_dot4_i32_i8: exact.
template <int F, int NC, int NX, int RW>
__global__ void __launch_bounds__(1024) k_narrow_i8v(const uint8_t* __restrict__ codes, float scale, int rows, int K,
                                                    const float* __restrict__ x, float* __restrict__ y,
                                                    int32_t* __restrict__ acc_out, float* __restrict__ act_out) {
    using N = Narrow<F>;
    constexpr int B = N::B, KS = 8 / B, E = 32 / B, EU = 128 / B;
    extern __shared__ uint32_t lds[];  // K/4 dwords of xq in the dot layout
    __shared__ float red_f[16];
    const int nt = blockDim.x, WB = nt >> 6;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.y;
    const int r0 = (blockIdx.x * WB + wave) * RW;
    const int nU = K / EU, k4 = K / 4;
    const float4* xb = reinterpret_cast<const float4*>(x + int64_t(b) * K);
    float4 xv[NX];
#pragma unroll
    for (int n = 0; n < NX; ++n) xv[n] = xb[min(tid + nt * n, k4 - 1)];
    __builtin_amdgcn_sched_barrier(0);  // keep the x requests ahead of the codes
    uint4 cv[RW][NC];
#pragma unroll
    for (int rw = 0; rw < RW; ++rw) {
        const uint4* rowp = reinterpret_cast<const uint4*>(codes + int64_t(min(r0 + rw, rows - 1)) * (K / 8 * B));
#pragma unroll
        for (int c = 0; c < NC; ++c) cv[rw][c] = ld_nt16(rowp + min(lane + 64 * c, nU - 1));
    }
    __builtin_amdgcn_sched_barrier(0);
    float m = 0.f;
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        if (tid + nt * n >= k4) xv[n] = make_float4(0.f, 0.f, 0.f, 0.f);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[n].x), fabsf(xv[n].y)), fmaxf(fabsf(xv[n].z), fabsf(xv[n].w))));
    }
    m = wave_maximum(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = wave_maximum(red_f[lane < WB ? lane : 0]);  // one LDS read per lane, then DPP
    float act = m / 127.0f;
    if (act == 0.0f) act = 1.0f;
    const float inv = quant_inv(act), thr = quant_thr(inv);
    // All of this thread's elements on the fast rounding, then one ballot for
    // the rare redo by exact division.
    float rq[NX][4];
    bool redo = false;
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        redo |= !quant_fast(xv[n].x, inv, thr, rq[n][0]);
        redo |= !quant_fast(xv[n].y, inv, thr, rq[n][1]);
        redo |= !quant_fast(xv[n].z, inv, thr, rq[n][2]);
        redo |= !quant_fast(xv[n].w, inv, thr, rq[n][3]);
    }
    if (__builtin_amdgcn_ballot_w64(redo)) {
        if (redo) {
#pragma unroll
            for (int n = 0; n < NX; ++n) {
                const float e4[4] = {xv[n].x, xv[n].y, xv[n].z, xv[n].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float r;
                    if (!quant_fast(e4[t], inv, thr, r)) rq[n][t] = roundf(e4[t] / act);
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        const int i = tid + nt * n;
        if (i >= k4) continue;
        const int e = 4 * i, c = e / EU, r = e % EU, d = r / E, k = (r % E) >> 2;
        lds[(d * nU + c) * KS + k] = pack_i8x4(quant_clamp(rq[n][0]), quant_clamp(rq[n][1]), quant_clamp(rq[n][2]),
                                               quant_clamp(rq[n][3]));
    }
    __syncthreads();
    if (act_out && blockIdx.x == 0 && tid == 0) act_out[b] = act;
    // The wave's lanes read every xq byte exactly once (lane c + 64 j holds code
    // vector c + 64 j), so each lane's share of sum(xq) comes from the same
    // words, by a dot with ones; -OFF * sum(xq) then rides in the row totals.
    uint32_t xw[NC][4][KS];
    int sq = 0;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int k = 0; k < KS; ++k) xw[c][d][k] = lds[(d * nU + min(lane + 64 * c, nU - 1)) * KS + k];
        if (lane + 64 * c < nU) {
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int k = 0; k < KS; ++k) sq = __builtin_amdgcn_sdot4(int(xw[c][d][k]), 0x01010101, sq, false);
        }
    }
    const int osq = N::OFF * sq;
#pragma unroll
    for (int rw = 0; rw < RW; ++rw) {
        int acc = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (lane + 64 * c < nU) {
                const uint32_t wd[4] = {cv[rw][c].x ^ N::XR, cv[rw][c].y ^ N::XR, cv[rw][c].z ^ N::XR,
                                        cv[rw][c].w ^ N::XR};
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int k = 0; k < KS; ++k)
                        acc = __builtin_amdgcn_sdot4(int((wd[d] >> (B * k)) & N::MASK), int(xw[c][d][k]), acc, false);
            }
        }
        acc = wave_total_i(N::MUL * acc - osq);
        const int r = r0 + rw;
        if (lane == 0 && r < rows) {
            if (acc_out) acc_out[int64_t(b) * rows + r] = acc;
            if (y) y[int64_t(b) * rows + r] = float(acc) * act * scale;  // simd.go:142
        }
    }
}

// Rows of whole code vectors longer than k_narrow_i8v takes (K <= 32768): the
// same prologue, LDS layout and dot, one row per wave, each lane walking its
// code vectors c = lane + 64 i four at a time with the next four loaded while
// the current ones are summed.
template <int F, int NX>
__global__ void __launch_bounds__(1024) k_narrow_i8l(const uint8_t* __restrict__ codes, float scale, int rows, int K,
                                                    const float* __restrict__ x, float* __restrict__ y,
                                                    int32_t* __restrict__ acc_out, float* __restrict__ act_out) {
    using N = Narrow<F>;
    constexpr int B = N::B, KS = 8 / B, E = 32 / B, EU = 128 / B, NCI = 4;
    extern __shared__ uint32_t lds[];
    __shared__ float red_f[16];
    const int nt = blockDim.x, WB = nt >> 6;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.y;
    const int r = blockIdx.x * WB + wave;
    const int nU = K / EU, k4 = K / 4;
    const float4* xb = reinterpret_cast<const float4*>(x + int64_t(b) * K);
    float4 xv[NX];
#pragma unroll
    for (int n = 0; n < NX; ++n) xv[n] = xb[min(tid + nt * n, k4 - 1)];
    __builtin_amdgcn_sched_barrier(0);
    const uint4* rowp = reinterpret_cast<const uint4*>(codes + int64_t(min(r, rows - 1)) * (K / 8 * B));
    uint4 cur[NCI];
#pragma unroll
    for (int n = 0; n < NCI; ++n) cur[n] = ld_nt16(rowp + min(lane + 64 * n, nU - 1));
    __builtin_amdgcn_sched_barrier(0);
    float m = 0.f;
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        if (tid + nt * n >= k4) xv[n] = make_float4(0.f, 0.f, 0.f, 0.f);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(xv[n].x), fabsf(xv[n].y)), fmaxf(fabsf(xv[n].z), fabsf(xv[n].w))));
    }
    m = wave_maximum(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = wave_maximum(red_f[lane < WB ? lane : 0]);
    float act = m / 127.0f;
    if (act == 0.0f) act = 1.0f;
    const float inv = quant_inv(act), thr = quant_thr(inv);
    float rq[NX][4];
    bool redo = false;
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        redo |= !quant_fast(xv[n].x, inv, thr, rq[n][0]);
        redo |= !quant_fast(xv[n].y, inv, thr, rq[n][1]);
        redo |= !quant_fast(xv[n].z, inv, thr, rq[n][2]);
        redo |= !quant_fast(xv[n].w, inv, thr, rq[n][3]);
    }
    if (__builtin_amdgcn_ballot_w64(redo)) {
        if (redo) {
#pragma unroll
            for (int n = 0; n < NX; ++n) {
                const float e4[4] = {xv[n].x, xv[n].y, xv[n].z, xv[n].w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    float q;
                    if (!quant_fast(e4[t], inv, thr, q)) rq[n][t] = roundf(e4[t] / act);
                }
            }
        }
    }
#pragma unroll
    for (int n = 0; n < NX; ++n) {
        const int i = tid + nt * n;
        if (i >= k4) continue;
        const int e = 4 * i, c = e / EU, rr = e % EU, d = rr / E, k = (rr % E) >> 2;
        lds[(d * nU + c) * KS + k] = pack_i8x4(quant_clamp(rq[n][0]), quant_clamp(rq[n][1]), quant_clamp(rq[n][2]),
                                               quant_clamp(rq[n][3]));
    }
    __syncthreads();
    if (act_out && blockIdx.x == 0 && tid == 0) act_out[b] = act;
    int acc = 0, sq = 0;
    for (int c0 = 0; c0 < nU; c0 += 64 * NCI) {
        uint4 nxt[NCI];
#pragma unroll
        for (int n = 0; n < NCI; ++n) nxt[n] = ld_nt16(rowp + min(c0 + 64 * NCI + lane + 64 * n, nU - 1));
#pragma unroll
        for (int n = 0; n < NCI; ++n) {
            const int c = c0 + lane + 64 * n;
            if (c < nU) {
                const uint32_t wd[4] = {cur[n].x ^ N::XR, cur[n].y ^ N::XR, cur[n].z ^ N::XR, cur[n].w ^ N::XR};
#pragma unroll
                for (int d = 0; d < 4; ++d)
#pragma unroll
                    for (int k = 0; k < KS; ++k) {
                        const uint32_t xw = lds[(d * nU + c) * KS + k];
                        sq = __builtin_amdgcn_sdot4(int(xw), 0x01010101, sq, false);
                        acc = __builtin_amdgcn_sdot4(int((wd[d] >> (B * k)) & N::MASK), int(xw), acc, false);
                    }
            }
        }
#pragma unroll
        for (int n = 0; n < NCI; ++n) cur[n] = nxt[n];
    }
    acc = wave_total_i(N::MUL * acc - N::OFF * sq);
    if (lane == 0 && r < rows) {
        if (acc_out) acc_out[int64_t(b) * rows + r] = acc;
        if (y) y[int64_t(b) * rows + r] = float(acc) * act * scale;  // simd.go:142
    }
}

// Any shape (K <= 32768): xq in LDS in plain order, one wave per row, codes
// read per element by flat index (rows need not start on a byte).
template <int F>
__global__ void __launch_bounds__(256) k_narrow_i8(const uint8_t* __restrict__ codes, float scale, int rows, int K,
                                                  const float* __restrict__ x, float* __restrict__ y,
                                                  int32_t* __restrict__ acc_out, float* __restrict__ act_out,
                                                  int rows_per_block) {
    extern __shared__ uint32_t lds[];
    __shared__ float red_f[4];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int b = blockIdx.y;
    const float* xb = x + int64_t(b) * K;
    float m = 0.f;
    for (int j = tid; j < K; j += 256) m = fmaxf(m, fabsf(xb[j]));
    m = wave_maximum(m);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    float act = m / 127.0f;
    if (act == 0.0f) act = 1.0f;
    const float inv = quant_inv(act), thr = quant_thr(inv);
    int8_t* l8 = reinterpret_cast<int8_t*>(lds);
    for (int j = tid; j < K; j += 256) l8[j] = int8_t(quant_act(xb[j], act, inv, thr));
    __syncthreads();
    if (act_out && blockIdx.x == 0 && tid == 0) act_out[b] = act;
    const int r0 = blockIdx.x * rows_per_block, r1 = min(rows, r0 + rows_per_block);
    for (int r = r0 + wave; r < r1; r += 4) {
        int acc = 0;
        const int64_t base = int64_t(r) * K;
        for (int j = lane; j < K; j += 64) acc += narrow_i8<F>(codes, base + j) * int(l8[j]);
        acc = wave_total_i(acc);
        if (lane == 0) {
            if (acc_out) acc_out[int64_t(b) * rows + r] = acc;
            if (y) y[int64_t(b) * rows + r] = float(acc) * act * scale;
        }
    }
}

// f32 weight of flat element i, as the Store decoders give it (weightAt,
// weights/decode.go:150-215): f32(q) * scale for the narrow DTypes, Ternary
// codes 0 / 2 -> -scale / +scale and 1, 3 -> 0; the f32 value for LAYOUT_F32.
template <int F>
__device__ __forceinline__ float store_w(const uint8_t* codes, int64_t i, float scale) {
    if constexpr (F == FMT_NONE) {
        return reinterpret_cast<const float*>(codes)[i];
    } else if constexpr (F == FMT_NATIVE_TERNARY) {
        const uint32_t u = ncode<2>(codes, i);
        return u == 0 ? -scale : (u == 2 ? scale : 0.0f);
    } else if constexpr (F == FMT_NATIVE_BINARY) {
        return ncode<1>(codes, i) ? scale : -scale;
    } else {
        return float(narrow_i8<F>(codes, i)) * scale;
    }
}

// y = W x with f64 sums (one wave per row, 4 rows per block): the f32
// FormatNone product (TX = TY = float) and Store.MatVec (TX = TY = double).
template <int F, class TX, class TY>
__global__ void __launch_bounds__(256) k_native_fwd(const uint8_t* __restrict__ codes, float scale, int64_t rows,
                                                   int64_t K, const TX* __restrict__ x, TY* __restrict__ y) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t r = int64_t(blockIdx.x) * 4 + wave;
    const int b = blockIdx.y;
    if (r >= rows) return;
    const TX* xb = x + int64_t(b) * K;
    const int64_t base = r * K;
    double acc = 0.0;
    if constexpr (F == FMT_NONE && sizeof(TX) == 4) {
        if (K % 4 == 0) {  // rows start 16-byte aligned
            typedef float f32x4 __attribute__((ext_vector_type(4)));
            const f32x4* w4 = reinterpret_cast<const f32x4*>(codes) + base / 4;
            const float4* x4 = reinterpret_cast<const float4*>(xb);
            for (int64_t j = lane; j < K / 4; j += 64) {
                const f32x4 w = __builtin_nontemporal_load(w4 + j);
                const float4 v = x4[j];
                acc = fma(double(w.x), double(v.x), acc);
                acc = fma(double(w.y), double(v.y), acc);
                acc = fma(double(w.z), double(v.z), acc);
                acc = fma(double(w.w), double(v.w), acc);
            }
        } else {
            for (int64_t j = lane; j < K; j += 64) acc = fma(double(store_w<F>(codes, base + j, scale)), double(xb[j]), acc);
        }
    } else {
        for (int64_t j = lane; j < K; j += 64) acc = fma(double(store_w<F>(codes, base + j, scale)), double(xb[j]), acc);
    }
    acc = wave_total_f64(acc);
    if (lane == 0) y[int64_t(b) * rows + r] = TY(acc);
}

// Column partials of W^T gy over row slices (f64): thread = column, slice =
// blockIdx.y (rows_per_slice rows in row order), batch = blockIdx.z. Rows
// with gy == 0 are skipped, as matVecTNativeF64 does (weights/native.go:1147).
template <int F, class TG>
__global__ void __launch_bounds__(256) k_native_t(const uint8_t* __restrict__ codes, float scale, int64_t rows,
                                                 int64_t K, const TG* __restrict__ gy, double* __restrict__ part,
                                                 int64_t rows_per_slice) {
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int slice = blockIdx.y, b = blockIdx.z, nslices = gridDim.y;
    if (c >= K) return;
    const int64_t r0 = int64_t(slice) * rows_per_slice, r1 = min(rows, r0 + rows_per_slice);
    const TG* g = gy + int64_t(b) * rows;
    double acc = 0.0;
    for (int64_t r = r0; r < r1; ++r) {
        const double gv = double(g[r]);
        if (gv == 0.0) continue;
        acc = fma(double(store_w<F>(codes, r * K + c, scale)), gv, acc);
    }
    part[(int64_t(b) * nslices + slice) * K + c] = acc;
}

// gx[b][c] = TX(gx[b][c] + sum of the slices' partials in slice order), in f64.
template <class TX>
__global__ void __launch_bounds__(256) k_native_t_sum(const double* __restrict__ part, TX* __restrict__ gx, int64_t K,
                                                     int nslices) {
    const int64_t c = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= K) return;
    const double* p = part + int64_t(b) * nslices * K + c;
    TX* o = gx + int64_t(b) * K + c;
    const double g0 = double(*o);
    // Slices in order; each group of 8 loads (clamped, the extra ones masked
    // out of the sum) and the gx load are issued before any add.
    double s = 0.0;
    for (int k = 0; k < nslices; k += 8) {
        double v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p[int64_t(min(k + j, nslices - 1)) * K];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (k + j < nslices) s += v[j];
    }
    *o = TX(g0 + s);
}

// Launch geometry of k_narrow_i8v: about one block per CU (256), each of WB
// waves (4..16) holding RW rows (1, 2 or 4), and NX float4 of x per thread.
template <int F, int NC, int NX, int RW>
void launch_narrow_g(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s,
                     int wb) {
    const int rows = int(b.rows), K = int(b.cols);
    const int per = wb * RW;
    hipLaunchKernelGGL((k_narrow_i8v<F, NC, NX, RW>), dim3(unsigned((rows + per - 1) / per), unsigned(batch)),
                       dim3(unsigned(64 * wb)), size_t(K), s, b.codes, b.tensor_scale, rows, K, x, y, acc, act);
}

template <int F, int NC, int RW>
void launch_narrow_x(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s,
                     int wb) {
    // NX = float4 of x per thread, exact for 1..4, 6 and 8 (K <= 8192, wb >= 4).
    // NC = RW = 4 holds 16 code vectors per lane: there the block takes enough
    // waves for NX <= 4, which keeps the kernel within its registers.
    if constexpr (NC == 4 && RW == 4) wb = std::max(wb, (int(b.cols) / 4 + 255) / 256);
    const int nx = (int(b.cols) / 4 + 64 * wb - 1) / (64 * wb);
    if (nx <= 1) launch_narrow_g<F, NC, 1, RW>(b, x, y, acc, act, batch, s, wb);
    else if (nx <= 2) launch_narrow_g<F, NC, 2, RW>(b, x, y, acc, act, batch, s, wb);
    else if (nx <= 3) launch_narrow_g<F, NC, 3, RW>(b, x, y, acc, act, batch, s, wb);
    else if (nx <= 4 || (NC == 4 && RW == 4)) launch_narrow_g<F, NC, 4, RW>(b, x, y, acc, act, batch, s, wb);
    else if constexpr (NC < 4 || RW < 4) {
        if (nx <= 6) launch_narrow_g<F, NC, 6, RW>(b, x, y, acc, act, batch, s, wb);
        else launch_narrow_g<F, NC, 8, RW>(b, x, y, acc, act, batch, s, wb);
    }
}

// Block shape of k_narrow_i8v: rows per block ~ rows / 256 (one block per
// CU), as wb waves (4..16) of rw rows each. Measured on the ternary pair:
// 2560 rows run best as 10 waves x 1 row (256 blocks), 6912 rows as 7-8 waves
// x 4 rows (216-247 blocks; 14 x 2 is 5 % slower, 16 x 1 in 432 blocks 25 %).
struct NarrowShape {
    int wb, rw;
};
inline NarrowShape narrow_shape(int rows) {
    const int want = (rows + 255) / 256;
    const int rw = want <= 16 ? 1 : 4;
    return {std::max(4, std::min(16, (want + rw - 1) / rw)), rw};
}

template <int F, int NC>
void launch_narrow_v(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s) {
    if constexpr (NC == 8) {  // 8 code vectors per lane and row (Int8 rows of up to 8192): one row per wave
        launch_narrow_x<F, NC, 1>(b, x, y, acc, act, batch, s, std::max(4, std::min(16, (int(b.rows) + 255) / 256)));
    } else {
        const NarrowShape sh = narrow_shape(int(b.rows));
        if (sh.rw == 1) launch_narrow_x<F, NC, 1>(b, x, y, acc, act, batch, s, sh.wb);
        else if (sh.rw == 2) launch_narrow_x<F, NC, 2>(b, x, y, acc, act, batch, s, sh.wb);
        else launch_narrow_x<F, NC, 4>(b, x, y, acc, act, batch, s, sh.wb);
    }
}

template <int F>
int launch_narrow_f(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s) {
    const int rows = int(b.rows), K = int(b.cols);
    constexpr int EU = 128 / Narrow<F>::B;  // codes per 16-byte vector
    if (K % EU == 0 && K <= 8192) {
        const int nu = K / EU;  // NC = ceil(nu / 64) vectors per lane and row; nu <= 8192 / EU
        if (nu <= 64) launch_narrow_v<F, 1>(b, x, y, acc, act, batch, s);
        else if constexpr (EU <= 64) {
            if (nu <= 128) launch_narrow_v<F, 2>(b, x, y, acc, act, batch, s);
            else if constexpr (EU <= 32) {
                if (nu <= 256) launch_narrow_v<F, 4>(b, x, y, acc, act, batch, s);
                else if constexpr (EU <= 16) launch_narrow_v<F, 8>(b, x, y, acc, act, batch, s);
            }
        }
        return int(hipGetLastError());
    }
    if (K % EU == 0) {  // longer rows of whole code vectors (K <= 32768): one row per wave of 16-wave blocks
        const dim3 g = dim3(unsigned((rows + 15) / 16), unsigned(batch)), blk = dim3(1024);
        const int nx = (K / 4 + 1023) / 1024;
        if (nx <= 4) hipLaunchKernelGGL((k_narrow_i8l<F, 4>), g, blk, size_t(K), s, b.codes, b.tensor_scale, rows, K, x, y, acc, act);
        else hipLaunchKernelGGL((k_narrow_i8l<F, 8>), g, blk, size_t(K), s, b.codes, b.tensor_scale, rows, K, x, y, acc, act);
        return int(hipGetLastError());
    }
    const int rpb = 16;
    const size_t lds = size_t((K + 3) / 4) * 4;
    hipLaunchKernelGGL(k_narrow_i8<F>, dim3(unsigned((rows + rpb - 1) / rpb), unsigned(batch)), dim3(256), lds, s,
                       b.codes, b.tensor_scale, rows, K, x, y, acc, act, rpb);
    return int(hipGetLastError());
}

int launch_narrow(const DevBlob& b, const float* x, float* y, int32_t* acc, float* act, int batch, hipStream_t s) {
    switch (b.fmt) {
    case FMT_NATIVE_INT8: return launch_narrow_f<FMT_NATIVE_INT8>(b, x, y, acc, act, batch, s);
    case FMT_NATIVE_INT4: return launch_narrow_f<FMT_NATIVE_INT4>(b, x, y, acc, act, batch, s);
    case FMT_NATIVE_INT2: return launch_narrow_f<FMT_NATIVE_INT2>(b, x, y, acc, act, batch, s);
    case FMT_NATIVE_TERNARY: return launch_narrow_f<FMT_NATIVE_TERNARY>(b, x, y, acc, act, batch, s);
    case FMT_NATIVE_BINARY: return launch_narrow_f<FMT_NATIVE_BINARY>(b, x, y, acc, act, batch, s);
    default: return int(hipErrorInvalidValue);
    }
}

template <class TX, class TY>
int launch_fwd_t(const DevBlob& b, const TX* x, TY* y, int batch, hipStream_t s) {
    const dim3 g(unsigned((b.rows + 3) / 4), unsigned(batch));
    const float sc = b.tensor_scale;
    switch (b.fmt) {
    case FMT_NONE: hipLaunchKernelGGL((k_native_fwd<FMT_NONE, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    case FMT_NATIVE_INT8: hipLaunchKernelGGL((k_native_fwd<FMT_NATIVE_INT8, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    case FMT_NATIVE_INT4: hipLaunchKernelGGL((k_native_fwd<FMT_NATIVE_INT4, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    case FMT_NATIVE_INT2: hipLaunchKernelGGL((k_native_fwd<FMT_NATIVE_INT2, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    case FMT_NATIVE_TERNARY: hipLaunchKernelGGL((k_native_fwd<FMT_NATIVE_TERNARY, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    case FMT_NATIVE_BINARY: hipLaunchKernelGGL((k_native_fwd<FMT_NATIVE_BINARY, TX, TY>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, x, y); break;
    default: return int(hipErrorInvalidValue);
    }
    return int(hipGetLastError());
}

// Row slices of the transposed products: about 1024 blocks, at least 64 rows each.
int native_t_slices(const DevBlob& b, int batch) {
    const int64_t colb = (b.cols + 255) / 256;
    const int64_t want = (1024 + colb * batch - 1) / (colb * std::max(1, batch));
    return int(std::max<int64_t>(1, std::min<int64_t>({want, 256, b.rows / 64})));
}

template <class TG, class TX>
int launch_t_t(const DevBlob& b, const TG* gy, TX* gx, int batch, hipStream_t s, double* part) {
    if (!part) return int(hipErrorInvalidValue);
    const int ns = native_t_slices(b, batch);
    const int64_t rps = (b.rows + ns - 1) / ns;
    const dim3 g(unsigned((b.cols + 255) / 256), unsigned(ns), unsigned(batch));
    const float sc = b.tensor_scale;
    switch (b.fmt) {
    case FMT_NONE: hipLaunchKernelGGL((k_native_t<FMT_NONE, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    case FMT_NATIVE_INT8: hipLaunchKernelGGL((k_native_t<FMT_NATIVE_INT8, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    case FMT_NATIVE_INT4: hipLaunchKernelGGL((k_native_t<FMT_NATIVE_INT4, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    case FMT_NATIVE_INT2: hipLaunchKernelGGL((k_native_t<FMT_NATIVE_INT2, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    case FMT_NATIVE_TERNARY: hipLaunchKernelGGL((k_native_t<FMT_NATIVE_TERNARY, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    case FMT_NATIVE_BINARY: hipLaunchKernelGGL((k_native_t<FMT_NATIVE_BINARY, TG>), g, dim3(256), 0, s, b.codes, sc, b.rows, b.cols, gy, part, rps); break;
    default: return int(hipErrorInvalidValue);
    }
    hipLaunchKernelGGL(k_native_t_sum<TX>, dim3(unsigned((b.cols + 255) / 256), unsigned(batch)), dim3(256), 0, s, part,
                       gx, b.cols, ns);
    return int(hipGetLastError());
}

}  // namespace

int launch_narrow_acc(const DevBlob& b, const float* d_x, int32_t* d_acc, float* d_act_scale, int batch, void* stream) {
    if (b.layout != LAYOUT_NARROW) return int(hipErrorInvalidValue);
    return launch_narrow(b, d_x, nullptr, d_acc, d_act_scale, batch, static_cast<hipStream_t>(stream));
}

int launch_native_fwd(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (b.layout == LAYOUT_NARROW) return launch_narrow(b, d_x, d_y, nullptr, nullptr, batch, s);
    if (b.layout == LAYOUT_F32) return launch_fwd_t<float, float>(b, d_x, d_y, batch, s);
    return int(hipErrorInvalidValue);
}

int launch_store_f64(const DevBlob& b, const double* d_x, double* d_y, void* stream) {
    if (b.layout != LAYOUT_NARROW && b.layout != LAYOUT_F32) return int(hipErrorInvalidValue);
    return launch_fwd_t<double, double>(b, d_x, d_y, 1, static_cast<hipStream_t>(stream));
}

size_t store_t_scratch_floats(const DevBlob& b) { return native_t_scratch_floats(b, 1); }

int launch_store_t_f64(const DevBlob& b, const double* d_gy, double* d_gx, void* stream, double* d_scratch) {
    if (b.layout != LAYOUT_NARROW && b.layout != LAYOUT_F32) return int(hipErrorInvalidValue);
    return launch_t_t<double, double>(b, d_gy, d_gx, 1, static_cast<hipStream_t>(stream), d_scratch);
}

// f64 partials: two floats of scratch each.
size_t native_t_scratch_floats(const DevBlob& b, int batch) {
    if (batch <= 0) return 0;
    return 2 * size_t(native_t_slices(b, batch)) * size_t(b.cols) * size_t(batch);
}

int launch_native_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, double* d_scratch) {
    if (b.layout != LAYOUT_NARROW && b.layout != LAYOUT_F32) return int(hipErrorInvalidValue);
    return launch_t_t<float, float>(b, d_gy, d_gx, batch, static_cast<hipStream_t>(stream), d_scratch);
}

}  // namespace wv
