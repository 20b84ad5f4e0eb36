// decode.hip — one greedy decode step of welvet's transformer decoder on the
// device: embedding row, per layer RMSNorm -> Q/K/V GEMVs -> RoPE + KV-cache
// append -> GQA attention -> O GEMV + residual -> RMSNorm -> gate/up GEMVs
// with SiLU(gate)*up -> down GEMV + residual; final RMSNorm, LM head, argmax
// (model/transformer/forward.go:26-90 for one new token; layers/mha/cpu.go,
// attn.go, rope.go; layers/swiglu/cpu.go; layers/rmsnorm/cpu.go).
//
// Everything stays in HBM between kernels. The position and the input token
// live in device memory, so the whole step can be captured once into a HIP
// graph and replayed: the step ends by writing its argmax into the input
// token slot and (optionally) advancing the position, so replays generate
// tokens with no host round trip. Projections on the row-interleaved layout
// fold the residual add and SiLU(gate)*up into the GEMV's output store.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/welvet_hip.h"
#include "rt_internal.h"
#include "wave_ops.h"

namespace wv {
namespace {

constexpr int kChunk = 32;  // KV positions per attention block

// h = table[token] (embedding lookup, clamped token id). Block 0 also builds
// this step's RoPE table: angle_d = pos / theta^(2d/hd) with theta^(2d/hd)
// precomputed on the host as the reference computes it (f64 math.Pow,
// layers/mha/rope.go:14), cs[d] = (cos, sin) in f64.
__global__ void __launch_bounds__(256) k_embed(const float* __restrict__ table, const int32_t* __restrict__ tok,
                                               float* __restrict__ h, int hidden, int vocab,
                                               const double* __restrict__ freq_div, double2* __restrict__ cs,
                                               int half, const int32_t* __restrict__ d_pos, float* __restrict__ ss) {
    const int t = min(max(*tok, 0), vocab - 1);
    for (int i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256)
        h[i] = table[int64_t(t) * hidden + i];
    if (ss) {  // sums of h^2 per 16 elements, for the first layer's fused RMSNorm
        const int i = blockIdx.x * 256 + threadIdx.x;
        const float v = i < hidden ? table[int64_t(t) * hidden + i] : 0.f;
        const float q = row_sum16(v * v);
        if ((threadIdx.x & 15) == 0 && i < hidden) ss[i >> 4] = q;
    }
    if (blockIdx.x == 0) {
        const double pos = double(*d_pos);
        for (int d = threadIdx.x; d < half; d += 256) {
            const double angle = pos / freq_div[d];
            cs[d] = make_double2(cos(angle), sin(angle));
        }
    }
}

// y = f32((x * inv) * gamma), inv = 1 / sqrt(sum(x^2)/dim + eps) in f64
// (layers/rmsnorm/cpu.go:70-85). gamma == nullptr means ones. Each thread
// loads its float4s once (dim % 4 == 0, dim <= 4 * 4096) and keeps them.
__global__ void __launch_bounds__(1024) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ gamma,
                                                  float* __restrict__ y, int dim, double eps) {
    __shared__ double part[16];
    x += int64_t(blockIdx.x) * dim;  // one row per block (the prompt forward normalizes n rows)
    y += int64_t(blockIdx.x) * dim;
    constexpr int R = 4;
    const int n4 = dim / 4;
    float4 xv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 1024 * r;
        xv[r] = i < n4 ? reinterpret_cast<const float4*>(x)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    double s = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r)
        s += double(xv[r].x) * xv[r].x + double(xv[r].y) * xv[r].y + double(xv[r].z) * xv[r].z +
             double(xv[r].w) * xv[r].w;
    s = wave_total_f64(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < 16; ++w) tot += part[w];
    const double inv = 1.0 / sqrt(tot / double(dim) + eps);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 1024 * r;
        if (i >= n4) break;
        const float4 g = gamma ? reinterpret_cast<const float4*>(gamma)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
        float4 o;
        o.x = float(double(xv[r].x) * inv * double(g.x));
        o.y = float(double(xv[r].y) * inv * double(g.y));
        o.z = float(double(xv[r].z) * inv * double(g.z));
        o.w = float(double(xv[r].w) * inv * double(g.w));
        reinterpret_cast<float4*>(y)[i] = o;
    }
}

// h += a (the residual add, per element as k_add), the updated rows written
// back, then the RMSNorm of them into y as k_rmsnorm: the prompt forward's add
// and norm in one pass over the rows. a and y may be the same rows: a block
// reads its row of a before the barrier and writes y after it.
__global__ void __launch_bounds__(1024) k_add_rmsnorm(float* __restrict__ h, const float* a,
                                                      const float* __restrict__ gamma, float* y, int dim, double eps) {
    __shared__ double part[16];
    h += int64_t(blockIdx.x) * dim;
    a += int64_t(blockIdx.x) * dim;
    y += int64_t(blockIdx.x) * dim;
    constexpr int R = 4;
    const int n4 = dim / 4;
    float4 xv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 1024 * r;
        xv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < n4) {
            const float4 hv = reinterpret_cast<const float4*>(h)[i], av = reinterpret_cast<const float4*>(a)[i];
            xv[r] = make_float4(hv.x + av.x, hv.y + av.y, hv.z + av.z, hv.w + av.w);
        }
    }
    double s = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r)
        s += double(xv[r].x) * xv[r].x + double(xv[r].y) * xv[r].y + double(xv[r].z) * xv[r].z +
             double(xv[r].w) * xv[r].w;
    s = wave_total_f64(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < 16; ++w) tot += part[w];
    const double inv = 1.0 / sqrt(tot / double(dim) + eps);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = threadIdx.x + 1024 * r;
        if (i >= n4) break;
        reinterpret_cast<float4*>(h)[i] = xv[r];
        const float4 g = gamma ? reinterpret_cast<const float4*>(gamma)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
        float4 o;
        o.x = float(double(xv[r].x) * inv * double(g.x));
        o.y = float(double(xv[r].y) * inv * double(g.y));
        o.z = float(double(xv[r].z) * inv * double(g.z));
        o.w = float(double(xv[r].w) * inv * double(g.w));
        reinterpret_cast<float4*>(y)[i] = o;
    }
}

// The KV caches are head-major, [n_kv][max_seq][HD], so the K (and V) rows of
// one chunk of one head are one contiguous kChunk*HD*4-byte run.
//
// Flash-decoding partials for one KV head and one chunk of kChunk positions:
// the G = n_heads / n_kv query heads that share the KV head read its K and V
// rows once (layers/mha/attn.go:40-118: score = q.k * scale over the causal
// positions kPos <= pos, max-subtracted softmax, sum of p * v). Per (head,
// chunk) it writes o[HD] (unnormalised), the chunk max m and sum l.
//
// RoPE and the KV append are folded in: q arrives unrotated and each block
// rotates its G heads in LDS with this step's cos/sin table; the block whose
// chunk holds position pos rotates the new k row of its KV head, uses it and
// the new v row in place of the cache's row pos, and writes both to the cache
// (layers/mha/cpu.go:178-193, rope.go:6-21).
//
// Every block computes only after its own data arrives, so the step costs
// about the last block's arrival plus one block's compute: q and the cos/sin
// pairs are requested first, then K, then V, so the q rotation, the K tile
// and the scores proceed while V is still in flight.
template <int HD>
__global__ void __launch_bounds__(256) k_attn_part(const float* __restrict__ q, float* __restrict__ kc,
                                                   float* __restrict__ vc, const int32_t* __restrict__ d_pos,
                                                   float* __restrict__ part, int n_heads, int n_kv, int max_seq,
                                                   int n_chunks, float scale, const float* __restrict__ k_new,
                                                   const float* __restrict__ v_new, const double2* __restrict__ cs) {
    constexpr int C = kChunk, Q4 = HD / 4, H2 = HD / 2;
    constexpr int NL = C * Q4 / 256;         // float4 of K (and of V) per thread
    constexpr int QP = (8 * H2 + 255) / 256;    // q rotation pairs per thread (up to 8 heads per KV head)
    static_assert(NL >= 1 && C == 32, "chunk shape");
    // K tile: the score pass gives position p to lanes p and p + 32, one half
    // of the head dimensions each. The upper half of a row starts HO words in
    // (HO = 32 mod 64) and rows are KLD = 1 mod 32 words apart, so the 64 lanes
    // of a read hit 64 different banks (and each 32-lane half 32 different
    // banks): with the halves HD/2 apart they met in pairs.
    constexpr int HO = H2 % 64 == 32 ? H2 : H2 + 32, KLD = HO + H2 + 1;
    __shared__ float ktile[C * KLD];
    __shared__ __attribute__((aligned(16))) float vtile[C * HD];
    __shared__ __attribute__((aligned(16))) float es[8][C];
    extern __shared__ float qs[];  // [G][HD]
    const int kvh = blockIdx.x, c = blockIdx.y;
    const int G = n_heads / n_kv;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = *d_pos;
    const int kv_len = min(pos + 1, max_seq);
    const int p0 = c * C;
    const int nvalid = min(C, kv_len - p0);
    if (nvalid <= 0) return;  // past the causal end: the combine reads only the chunks below kv_len
    const int pnew = pos % max_seq - p0;  // row of this step's k/v inside the chunk (if in [0, C))
    const bool has_new = pnew >= 0 && pnew < C;
    float qa[QP], qb[QP];
    double2 rq[QP];
    const float* qh = q + kvh * G * HD;
#pragma unroll
    for (int j = 0; j < QP; ++j) {
        const int i = min(t + 256 * j, G * H2 - 1), g = i / H2, d = i % H2;
        qa[j] = qh[g * HD + d];
        qb[j] = qh[g * HD + d + H2];
        rq[j] = cs[d];
    }
    __builtin_amdgcn_sched_barrier(0);
    // K and V rows of the chunk (rows past the end are clamped to the last valid one and get zero weight)
    float4 kv4[NL], vv4[NL];
    const float4* kb = reinterpret_cast<const float4*>(kc + (int64_t(kvh) * max_seq + p0) * HD);
    const float4* vb = reinterpret_cast<const float4*>(vc + (int64_t(kvh) * max_seq + p0) * HD);
#pragma unroll
    for (int r = 0; r < NL; ++r) {
        const int i = t + 256 * r;
        kv4[r] = kb[min(i / Q4, nvalid - 1) * Q4 + i % Q4];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NL; ++r) {
        const int i = t + 256 * r;
        vv4[r] = vb[min(i / Q4, nvalid - 1) * Q4 + i % Q4];
    }
    __builtin_amdgcn_sched_barrier(0);
    // q heads of this KV group, rotated: one thread per pair (g, d < HD/2)
#pragma unroll
    for (int j = 0; j < QP; ++j) {
        const int i = t + 256 * j;
        if (i < G * H2) {
            const int g = i / H2, d = i % H2;
            const double v0 = qa[j], v1 = qb[j];
            qs[g * HD + d] = float(v0 * rq[j].x - v1 * rq[j].y);
            qs[g * HD + d + H2] = float(v0 * rq[j].y + v1 * rq[j].x);
        }
    }
    // K tile (row pnew comes from this step's k below). Element stores keep
    // the loaded arrays in registers.
#pragma unroll
    for (int r = 0; r < NL; ++r) {
        const int i = t + 256 * r;
        if (i / Q4 == pnew) continue;
        const int c4 = 4 * (i % Q4);
        float* row = ktile + (i / Q4) * KLD + (c4 < H2 ? c4 : c4 - H2 + HO);
        row[0] = kv4[r].x;
        row[1] = kv4[r].y;
        row[2] = kv4[r].z;
        row[3] = kv4[r].w;
    }
    float4 vnew = make_float4(0.f, 0.f, 0.f, 0.f);
    if (has_new && t < Q4) {  // this step's row: rotated k and v, into the tiles and the cache
        const int d0 = 4 * t;
        const float* kn = k_new + kvh * HD;
        float kr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = d0 + e, dm = d % H2;
            const double2 rc = cs[dm];
            const double a0 = kn[dm], a1 = kn[dm + H2];
            kr[e] = d < H2 ? float(a0 * rc.x - a1 * rc.y) : float(a0 * rc.y + a1 * rc.x);
        }
        vnew = reinterpret_cast<const float4*>(v_new + kvh * HD)[t];
        float* row = ktile + pnew * KLD + (d0 < H2 ? d0 : d0 - H2 + HO);
        row[0] = kr[0];
        row[1] = kr[1];
        row[2] = kr[2];
        row[3] = kr[3];
        const int64_t crow = (int64_t(kvh) * max_seq + pos % max_seq) * HD;
        reinterpret_cast<float4*>(kc + crow)[t] = make_float4(kr[0], kr[1], kr[2], kr[3]);
        reinterpret_cast<float4*>(vc + crow)[t] = vnew;
    }
    __syncthreads();
    // scores: one wave per query head; lanes p and p + 32 take the lower and
    // upper half of position p's dimensions
    for (int g = wave; g < G; g += 4) {
        const int p = lane & 31, h = lane >> 5;
        const float* kr = ktile + p * KLD + h * HO;
        const float4* qg = reinterpret_cast<const float4*>(qs + g * HD + h * H2);
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
        for (int d4 = 0; d4 < H2 / 4; ++d4) {
            const float4 qv = qg[d4];
            float& a = s4[d4 & 3];
            a = fmaf(qv.x, kr[4 * d4], a);
            a = fmaf(qv.y, kr[4 * d4 + 1], a);
            a = fmaf(qv.z, kr[4 * d4 + 2], a);
            a = fmaf(qv.w, kr[4 * d4 + 3], a);
        }
        float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        s = reduce_scatter32(s, s);  // + the other half (lane ^ 32)
        s = p < nvalid ? s * scale : -INFINITY;
        const float m = wave_maximum(s);
        const float e = (p < nvalid && h == 0) ? expf(s - m) : 0.f;
        const float l = wave_total(e);
        if (h == 0) es[g][p] = e;
        if (lane == 0) {
            float* o = part + (int64_t(kvh * G + g) * n_chunks + c) * (HD + 2);
            o[HD] = m;
            o[HD + 1] = l;
        }
    }
#pragma unroll
    for (int r = 0; r < NL; ++r) {
        const int i = t + 256 * r;
        if (i / Q4 == pnew) continue;
        float* vr = vtile + 4 * i;
        vr[0] = vv4[r].x;
        vr[1] = vv4[r].y;
        vr[2] = vv4[r].z;
        vr[3] = vv4[r].w;
    }
    if (has_new && t < Q4) {
        float* vr = vtile + pnew * HD + 4 * t;
        vr[0] = vnew.x;
        vr[1] = vnew.y;
        vr[2] = vnew.z;
        vr[3] = vnew.w;
    }
    __syncthreads();
    // o[d] = sum_p e_p v[p][d] over all C rows (e_p = 0 past the end)
    for (int g = wave; g < G; g += 4) {
        float* o = part + (int64_t(kvh * G + g) * n_chunks + c) * (HD + 2);
        const float4* e4 = reinterpret_cast<const float4*>(es[g]);
#pragma unroll
        for (int d = lane; d < HD; d += 64) {
            float a4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
            for (int p4 = 0; p4 < C / 4; ++p4) {
                const float4 ev = e4[p4];
                float& a = a4[p4 & 3];
                a = fmaf(ev.x, vtile[(4 * p4) * HD + d], a);
                a = fmaf(ev.y, vtile[(4 * p4 + 1) * HD + d], a);
                a = fmaf(ev.z, vtile[(4 * p4 + 2) * HD + d], a);
                a = fmaf(ev.w, vtile[(4 * p4 + 3) * HD + d], a);
            }
            o[d] = (a4[0] + a4[1]) + (a4[2] + a4[3]);
        }
    }
}

// Lane-group sums for k_attn_reg. pair_scatter<B> is one reduce-scatter step
// over the lanes that differ in lane bit B: lanes with the bit clear return
// a + a(partner), the others b + b(partner). Bits 5 and 4 use gfx950's lane
// swaps; bits 3..0 use DPP (row_ror 8, half_mirror, quad xor 2, quad xor 1).
// half_mirror pairs l with l ^ 7, which differs in bit 2: applied top-down
// after bits 4 and 3 and before bits 1 and 0, the pairs still tile every
// 8-lane group, so the steps sum over all of it.
template <int B>
__device__ __forceinline__ float lane_partner(float v) {
    static_assert(B >= 0 && B <= 3, "DPP partner");
    if constexpr (B == 3) return row_xor8(v);
    else if constexpr (B == 2) return half_mirror(v);
    else if constexpr (B == 1) return quad_xor2(v);
    else return quad_xor1(v);
}
template <int B>
__device__ __forceinline__ float pair_scatter(float a, float b, int lane) {
    if constexpr (B == 5) return reduce_scatter32(a, b);
    else if constexpr (B == 4) return reduce_scatter16(a, b);
    else {
        const bool hi = (lane >> B) & 1;
        const float keep = hi ? b : a, send = hi ? a : b;
        return keep + lane_partner<B>(send);
    }
}
// Sum over lane bits B..0 into every lane.
template <int B>
__device__ __forceinline__ float group_allsum(float s) {
    if constexpr (B < 0) return s;
    else return group_allsum<B - 1>(s + lane_partner<B>(s));
}
// Totals of v[0..M) over the lanes that differ in lane bits B..0 (M a power of
// two <= 2^(B+1)): bits B, B-1, ... scatter while more than one value is left
// and the bits below that add. Lane l returns the total of v[i] for i given
// by its bits B..B-log2(M)+1, highest bit most significant.
template <int B, int M, int N>
__device__ __forceinline__ float group_scatter(float (&v)[N], int lane) {
    if constexpr (M == 1) {
        return group_allsum<B>(v[0]);
    } else {
#pragma unroll
        for (int j = 0; j < M / 2; ++j) v[j] = pair_scatter<B>(v[j], v[j + M / 2], lane);
        return group_scatter<B - 1, M / 2>(v, lane);
    }
}
// Max and sum over each 32-lane half of the wave, in every lane of the half.
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, quad_xor1(v));
    v = fmaxf(v, quad_xor2(v));
    v = fmaxf(v, half_mirror(v));
    v = fmaxf(v, row_xor8(v));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_wave_sum(float v) {
    v = group_allsum<3>(v);
    return reduce_scatter16(v, v);
}

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }

// The flash-decoding partials of k_attn_part for G = 1, 2, 4 or 8 query heads
// per KV head, computed from registers: K and V stay where they are loaded and
// only the q heads, the scores and the partial outputs pass through LDS.
//
// Thread t holds column t % Q4 (4 dims) of rows t / Q4 + r * RS (r < NL) of
// the chunk, Q4 = HD/4 lanes to a row, so the loads are the chunk's
// contiguous K (then V) run. Scores: each thread forms the NV = NL*G 4-dim
// partial dots of its rows and heads, and a reduce-scatter over the Q4 lanes
// of its row group leaves every (row, head) total in a lane (about 2 VALU
// operations per value instead of a shared K tile). Softmax: one 32-lane half
// wave per head. Output: each thread sums e[g][row] * v[row] over its NL rows
// for G heads x 4 dims, a reduce-scatter over the lane bits that select the
// row inside the wave halves the values, and the four waves' parts are added
// in LDS in wave order.
template <int HD, int G>
__global__ void __launch_bounds__(256) k_attn_reg(const float* __restrict__ q, float* __restrict__ kc,
                                                  float* __restrict__ vc, const int32_t* __restrict__ d_pos,
                                                  float* __restrict__ part, int max_seq, int n_chunks, float scale,
                                                  const float* __restrict__ k_new, const float* __restrict__ v_new,
                                                  const double2* __restrict__ cs) {
    constexpr int C = kChunk, Q4 = HD / 4, H2 = HD / 2, LQ = ilog2(Q4);
    constexpr int RS = 256 / Q4;  // rows between one thread's rows
    constexpr int NL = C / RS;    // rows per thread
    constexpr int NV = NL * G;    // partial dots per thread
    constexpr int NO = 4 * G;     // partial outputs per thread (G heads x 4 dims)
    constexpr int LR = 6 - LQ;    // lane bits that select the row inside a wave
    constexpr int NR = NO >> LR;  // partial outputs per lane after the in-wave row sum
    constexpr int QP = (G * H2 + 255) / 256;
    static_assert(C == 32 && NL >= 1 && NV <= Q4 && NR >= 1 && (G == 1 || G == 2 || G == 4 || G == 8), "shape");
    __shared__ __attribute__((aligned(16))) float qs[G * HD];
    __shared__ float ss[G][C];
    __shared__ float red[4][NR][64];
    const int kvh = blockIdx.x, c = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = *d_pos;
    const int kv_len = min(pos + 1, max_seq);
    const int p0 = c * C;
    const int nvalid = min(C, kv_len - p0);
    if (nvalid <= 0) return;  // past the causal end: the combine reads only the chunks below kv_len
    const int pnew = pos % max_seq - p0;
    const bool has_new = pnew >= 0 && pnew < C;
    const int col = t % Q4, row0 = t / Q4, d0 = 4 * col;
    // q pairs of this KV group, this step's k and v column (the block holding pos)
    float qa[QP], qb[QP];
    double2 rq[QP];
    const float* qh = q + kvh * G * HD;
#pragma unroll
    for (int j = 0; j < QP; ++j) {
        const int i = min(t + 256 * j, G * H2 - 1), g = i / H2, d = i % H2;
        qa[j] = qh[g * HD + d];
        qb[j] = qh[g * HD + d + H2];
        rq[j] = cs[d];
    }
    float4 ka = make_float4(0.f, 0.f, 0.f, 0.f), kb4 = ka, vnew = ka;
    double2 rk[4] = {};
    if (has_new) {
        const int dm = d0 % H2;
        ka = *reinterpret_cast<const float4*>(k_new + kvh * HD + dm);
        kb4 = *reinterpret_cast<const float4*>(k_new + kvh * HD + dm + H2);
        vnew = *reinterpret_cast<const float4*>(v_new + kvh * HD + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) rk[e] = cs[dm + e];
    }
    __builtin_amdgcn_sched_barrier(0);
    float4 kv4[NL], vv4[NL];
    const float4* kb = reinterpret_cast<const float4*>(kc + (int64_t(kvh) * max_seq + p0) * HD);
    const float4* vb = reinterpret_cast<const float4*>(vc + (int64_t(kvh) * max_seq + p0) * HD);
#pragma unroll
    for (int r = 0; r < NL; ++r) kv4[r] = ld_nt16(kb + min(row0 + RS * r, nvalid - 1) * Q4 + col);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < NL; ++r) vv4[r] = ld_nt16(vb + min(row0 + RS * r, nvalid - 1) * Q4 + col);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < QP; ++j) {
        const int i = t + 256 * j;
        if (i < G * H2) {
            const int g = i / H2, d = i % H2;
            const double v0 = qa[j], v1 = qb[j];
            qs[g * HD + d] = float(v0 * rq[j].x - v1 * rq[j].y);
            qs[g * HD + d + H2] = float(v0 * rq[j].y + v1 * rq[j].x);
        }
    }
    __syncthreads();
    float4 qv[G];
#pragma unroll
    for (int g = 0; g < G; ++g) qv[g] = *reinterpret_cast<const float4*>(qs + g * HD + d0);
    if (has_new) {  // the rotated new k and the new v replace the cache's row pnew, and are appended to the cache
        float x0[4] = {ka.x, ka.y, ka.z, ka.w}, x1[4] = {kb4.x, kb4.y, kb4.z, kb4.w};
        float kr[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // keeps the widening here: hoisted next to the loads it would wait
            // for them before the K and V loads are issued
            asm volatile("" : "+v"(x0[e]), "+v"(x1[e]));
            const double a0 = x0[e], a1 = x1[e];
            kr[e] = d0 < H2 ? float(a0 * rk[e].x - a1 * rk[e].y) : float(a0 * rk[e].y + a1 * rk[e].x);
        }
        const float4 knew = make_float4(kr[0], kr[1], kr[2], kr[3]);
#pragma unroll
        for (int r = 0; r < NL; ++r) {
            const bool mine = row0 + RS * r == pnew;
            kv4[r].x = mine ? kr[0] : kv4[r].x;
            kv4[r].y = mine ? kr[1] : kv4[r].y;
            kv4[r].z = mine ? kr[2] : kv4[r].z;
            kv4[r].w = mine ? kr[3] : kv4[r].w;
            vv4[r].x = mine ? vnew.x : vv4[r].x;
            vv4[r].y = mine ? vnew.y : vv4[r].y;
            vv4[r].z = mine ? vnew.z : vv4[r].z;
            vv4[r].w = mine ? vnew.w : vv4[r].w;
        }
        if (pnew >= row0 && (pnew - row0) % RS == 0) {
            const int64_t crow = (int64_t(kvh) * max_seq + pos % max_seq) * HD;
            *reinterpret_cast<float4*>(kc + crow + d0) = knew;
            *reinterpret_cast<float4*>(vc + crow + d0) = vnew;
        }
    }
    // scores
    float sv[NV];
#pragma unroll
    for (int r = 0; r < NL; ++r)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float a = qv[g].x * kv4[r].x;
            a = fmaf(qv[g].y, kv4[r].y, a);
            a = fmaf(qv[g].z, kv4[r].z, a);
            sv[r * G + g] = fmaf(qv[g].w, kv4[r].w, a);
        }
    {
        const float s = group_scatter<LQ - 1, NV>(sv, lane);
        constexpr int DUP = Q4 / NV;  // lanes holding each total
        if (col % DUP == 0) {
            const int vi = col / DUP, r = vi / G, g = vi % G, row = row0 + RS * r;
            ss[g][row] = row < nvalid ? s * scale : -INFINITY;
        }
    }
    __syncthreads();
    // softmax over the chunk: head `wave` in the lower half wave, head wave + 4
    // in the upper one (for G <= 4 it repeats the lower half's head and stores nothing)
    if (wave < G) {
        const int p = lane & 31, g = wave + 4 * (lane >> 5);
        const int gs = g < G ? g : wave;
        {
            const float s = ss[gs][p];
            const float m = half_wave_max(s);
            const float e = p < nvalid ? expf(s - m) : 0.f;
            const float l = half_wave_sum(e);
            if (g < G) {
                ss[g][p] = e;
                if (p == 0) {
                    float* o = part + (int64_t(kvh * G + g) * n_chunks + c) * (HD + 2);
                    o[HD] = m;
                    o[HD + 1] = l;
                }
            }
        }
    }
    __syncthreads();
    // o[g][d] = sum_p e[g][p] v[p][d]
    float acc[NO];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < NL; ++r) {
            const float w = ss[g][row0 + RS * r];
            a[0] = fmaf(w, vv4[r].x, a[0]);
            a[1] = fmaf(w, vv4[r].y, a[1]);
            a[2] = fmaf(w, vv4[r].z, a[2]);
            a[3] = fmaf(w, vv4[r].w, a[3]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * g + e] = a[e];
    }
#pragma unroll
    for (int j = 0; j < NO / 2; ++j) acc[j] = pair_scatter<5>(acc[j], acc[j + NO / 2], lane);
    if constexpr (LR == 2) {
#pragma unroll
        for (int j = 0; j < NO / 4; ++j) acc[j] = pair_scatter<4>(acc[j], acc[j + NO / 4], lane);
    }
#pragma unroll
    for (int j = 0; j < NR; ++j) red[wave][j][lane] = acc[j];
    __syncthreads();
    for (int o = t; o < G * HD; o += 256) {
        const int g = o / HD, d = o % HD, vi = 4 * g + (d & 3);
        int ln = d / 4 + 32 * (vi / (NO / 2)), j = vi % (NO / 2);
        if constexpr (LR == 2) {
            ln += 16 * (j / (NO / 4));
            j %= NO / 4;
        }
        const float s = (red[0][j][ln] + red[1][j][ln]) + (red[2][j][ln] + red[3][j][ln]);
        part[(int64_t(kvh * G + g) * n_chunks + c) * (HD + 2) + d] = s;
    }
}

// out[h][d] = sum_c o_c[d] e^{m_c - M} / sum_c l_c e^{m_c - M} over the nc
// chunks below kv_len, for nc <= 64*NCL. Block (h, dq) takes dims 64dq..64dq+63
// of head h (two blocks per head at HD = 128, so each CU pulls in half the
// partials). Every load is issued up front: lane j of the wave holds the
// weights of chunks j, j+64, ... (DPP max and sum), wave w accumulates chunks
// w, w+4, ... of its dim in order with each weight broadcast by readlane, and
// the four waves' sums are added in LDS.
template <int HD, int NCL>
__global__ void __launch_bounds__(256) k_attn_combine(const float* __restrict__ part, float* __restrict__ out,
                                                      int n_chunks, const int32_t* __restrict__ d_pos, int max_seq) {
    constexpr int PW = 16 * NCL;
    __shared__ float red[4][64];
    const int h = blockIdx.x, dq = blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float* ph = part + int64_t(h) * n_chunks * (HD + 2);
    float mc[NCL], lc[NCL];
#pragma unroll
    for (int j = 0; j < NCL; ++j) {
        const int cl = min(lane + 64 * j, n_chunks - 1);
        mc[j] = ph[cl * (HD + 2) + HD];
        lc[j] = ph[cl * (HD + 2) + HD + 1];
    }
    float ov[PW];
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const int cc = min(wave + 4 * k, n_chunks - 1);
        ov[k] = ph[cc * (HD + 2) + 64 * dq + lane];
    }
    const int kv_len = min(*d_pos + 1, max_seq);
    const int nc = min(n_chunks, (kv_len + kChunk - 1) / kChunk);
#pragma unroll
    for (int j = 0; j < NCL; ++j) {
        const bool live = lane + 64 * j < nc;
        mc[j] = live ? mc[j] : -INFINITY;
        lc[j] = live ? lc[j] : 0.f;
    }
    float m = mc[0];
#pragma unroll
    for (int j = 1; j < NCL; ++j) m = fmaxf(m, mc[j]);
    const float M = wave_maximum(m);
    float w[NCL], lw = 0.f;
#pragma unroll
    for (int j = 0; j < NCL; ++j) {
        w[j] = lane + 64 * j < nc ? expf(mc[j] - M) : 0.f;
        lw += lc[j] * w[j];
    }
    const float L = wave_total(lw);
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < PW; ++k) {
        const int cc = wave + 4 * k;
        if (cc < nc) {
            const float wk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[(4 * k) / 64]), cc % 64));
            acc = fmaf(ov[k], wk, acc);
        }
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (t < 64) out[h * HD + 64 * dq + t] = ((red[0][t] + red[1][t]) + (red[2][t] + red[3][t])) * (L > 0.f ? 1.0f / L : 0.f);
}

// The same for any nc <= 2048: thread c owns chunks c, c+256, ... for the max
// and the weights; chunks are summed in order, eight loads in flight.
__global__ void __launch_bounds__(256) k_attn_combine_long(const float* __restrict__ part, float* __restrict__ out,
                                                           int hd, int n_chunks, const int32_t* __restrict__ d_pos,
                                                           int max_seq) {
    constexpr int R = 8;
    __shared__ float wsc[256 * R];
    __shared__ float red[4];
    const int h = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int kv_len = min(*d_pos + 1, max_seq);
    const int nc = min(n_chunks, (kv_len + kChunk - 1) / kChunk);
    const float* ph = part + int64_t(h) * n_chunks * (hd + 2);
    float mloc[R], lloc[R];
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int c = t + 256 * r;
        mloc[r] = c < nc ? ph[c * (hd + 2) + hd] : -INFINITY;
        lloc[r] = c < nc ? ph[c * (hd + 2) + hd + 1] : 0.f;
        M = fmaxf(M, mloc[r]);
    }
    M = wave_maximum(M);
    if (lane == 0) red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float L = 0.f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int c = t + 256 * r;
        const float w = c < nc ? expf(mloc[r] - M) : 0.f;
        if (c < nc) wsc[c] = w;
        L += lloc[r] * w;
    }
    L = wave_total(L);
    if (lane == 0) red[wave] = L;
    __syncthreads();
    L = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    for (int d = t; d < hd; d += 256) {
        float acc = 0.f;
        int c = 0;
        for (; c + 8 <= nc; c += 8) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ph[(c + i) * (hd + 2) + d];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc = fmaf(v[i], wsc[c + i], acc);
        }
        for (; c < nc; ++c) acc = fmaf(ph[c * (hd + 2) + d], wsc[c], acc);
        out[h * hd + d] = acc * inv;
    }
}

__global__ void __launch_bounds__(256) k_add(float* __restrict__ y, const float* __restrict__ a, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) y[i] += a[i];
}

// out = silu(g) * u (layers/swiglu/cpu.go:41-53)
__global__ void __launch_bounds__(256) k_silu_mul(const float* __restrict__ g, const float* __restrict__ u,
                                                  float* __restrict__ out, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float x = g[i];
        out[i] = x / (1.0f + expf(-x)) * u[i];
    }
}

// next = argmax(logits) (lowest index on ties), recorded as generated token
// number *nstep; the next step's input token becomes `next`, and the
// position advances when `advance` is set. state = {pos, tok, next, nstep}.
__global__ void __launch_bounds__(1024) k_argmax_advance(const float* __restrict__ logits, int n,
                                                         int32_t* __restrict__ state, int32_t* __restrict__ gen,
                                                         int gen_cap, int advance) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float v = -INFINITY;
    int idx = 0x7fffffff;
    auto take = [&](float x, int i) {
        if (x > v || (x == v && i < idx)) {
            v = x;
            idx = i;
        }
    };
    // float4 loads, U per thread issued before any compare, so a pass costs
    // one memory round trip (32000 logits: one pass of 8 per thread).
    constexpr int U = 8;
    const int n4 = n >> 2;
    const float4* l4 = reinterpret_cast<const float4*>(logits);
    for (int base = 0; base < n4; base += 1024 * U) {
        float4 r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i4 = base + u * 1024 + int(threadIdx.x);
            r[u] = i4 < n4 ? l4[i4] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = 4 * (base + u * 1024 + int(threadIdx.x));
            if (i < 4 * n4) {
                take(r[u].x, i);
                take(r[u].y, i + 1);
                take(r[u].z, i + 2);
                take(r[u].w, i + 3);
            }
        }
    }
    for (int i = 4 * n4 + int(threadIdx.x); i < n; i += 1024) take(logits[i], i);
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(v, m, 64);
        const int oi = __shfl_xor(idx, m, 64);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = v;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (bv[w] > v || (bv[w] == v && bi[w] < idx)) {
                v = bv[w];
                idx = bi[w];
            }
        state[2] = idx;
        state[1] = idx;
        const int k = state[3];
        if (k < gen_cap) gen[k] = idx;
        state[3] = k + 1;
        if (advance) state[0] += 1;
    }
}

// ---------------------------------------------------------------------------
// Prompt (multi-token) forward: ForwardTokens over a block of n tokens
// ---------------------------------------------------------------------------

// H[s] = table[tok[s]] for the n prompt rows (token ids clamped as k_embed does).
__global__ void __launch_bounds__(256) k_embed_rows(const float* __restrict__ table, const int32_t* __restrict__ tok,
                                                    float* __restrict__ h, int hidden, int vocab) {
    const int s = blockIdx.y;
    const int t = min(max(tok[s], 0), vocab - 1);
    for (int i = blockIdx.x * 256 + threadIdx.x; i < hidden; i += gridDim.x * 256)
        h[int64_t(s) * hidden + i] = table[int64_t(t) * hidden + i];
}

// RoPE and the KV append for prompt row s at position pos0 + s
// (layers/mha/cpu.go:178-193, rope.go:6-21): the row's q heads are rotated in
// place, its k heads rotated and, with its v heads, written to the caches at
// that position. Angles and the rotation in f64 as in k_embed / k_attn_reg:
// angle_d = pos / theta^(2d/hd), (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos).
// SPLIT: the rows are the unsummed K-split slices of the Q|K|V stack GEMM
// (`splits` of them, at most 4, pstride floats apart, rows [q|k|v] of qs
// floats) and are added in split order on load; the rotated q goes to q.
// Block (s, y) takes every gridDim.y-th pass over the row's heads (a short
// prompt spreads a row over several blocks).
template <bool SPLIT>
__global__ void __launch_bounds__(256) k_rope_kv_rows(float* __restrict__ q, const float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ part,
                                                      int splits, int64_t pstride, float* __restrict__ kc,
                                                      float* __restrict__ vc, const double* __restrict__ freq_div,
                                                      int n_heads, int n_kv, int hd, int max_seq, int pos0, int qs,
                                                      int kvs) {
    // qs, kvs: row strides of q and of k, v (one [n][q|k|v] block, or three)
    const int s = blockIdx.x, half = hd / 2, pos = pos0 + s;
    const int kvd = n_kv * hd;
    float* qr = q + int64_t(s) * qs;
    const float* kr = k + int64_t(s) * kvs;
    const float* vr = v + int64_t(s) * kvs;
    const float* pr = SPLIT ? part + int64_t(s) * qs : nullptr;
    // element j of the row's q, k or v (off: the column where its part starts)
    auto rd = [&](const float* r, int off, int j) {
        if constexpr (!SPLIT) {
            return r[j];
        } else {
            float p[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (t < splits) p[t] = pr[int64_t(t) * pstride + off + j];
            float x = p[0];
#pragma unroll
            for (int t = 1; t < 4; ++t)
                if (t < splits) x += p[t];
            return x;
        }
    };
    const int koff = n_heads * hd, voff = koff + kvd;
    // the angle depends on the position and the dim only: each thread takes
    // one dim (half divides 256: head dims 64 and 128) and every HG-th head
    const int HG = 256 / half, d = threadIdx.x % half;
    const double angle = double(pos) / freq_div[d];
    const double c = cos(angle), sn = sin(angle);
    for (int hh = threadIdx.x / half + HG * blockIdx.y; hh < n_heads + n_kv; hh += HG * gridDim.y) {
        if (hh < n_heads) {
            const double x0 = rd(qr, 0, hh * hd + d), x1 = rd(qr, 0, hh * hd + d + half);
            qr[hh * hd + d] = float(x0 * c - x1 * sn);
            qr[hh * hd + d + half] = float(x0 * sn + x1 * c);
        } else {
            const int g = hh - n_heads;
            const double x0 = rd(kr, koff, g * hd + d), x1 = rd(kr, koff, g * hd + d + half);
            float* crow = kc + (int64_t(g) * max_seq + pos) * hd;
            crow[d] = float(x0 * c - x1 * sn);
            crow[d + half] = float(x0 * sn + x1 * c);
        }
    }
    for (int i = threadIdx.x + 256 * blockIdx.y; i < kvd; i += 256 * gridDim.y) {
        const int g = i / hd, d = i % hd;
        vc[(int64_t(g) * max_seq + pos) * hd + d] = rd(vr, voff, i);
    }
}

// Causal GQA attention for prompt row s (position pos0 + s) over the cache,
// which already holds the K and V rows of every prompt position
// (layers/mha/attn.go:40-118 with the causal mask kPos <= qPos): block (kvh, s)
// serves the G = n_heads / n_kv query heads of KV head kvh. Keys go in chunks
// of 64 with an online softmax in f32: scores q.k * scale, the running max
// and sum per head, the output rescaled when the max grows; out = sum p v / sum p.
template <int HD>
__global__ void __launch_bounds__(256) k_attn_prefill(const float* __restrict__ q, const float* __restrict__ kc,
                                                      const float* __restrict__ vc, float* __restrict__ out,
                                                      int n_heads, int n_kv, int max_seq, int pos0, float scale,
                                                      int qstr) {
    constexpr int CH = 64, GM = 8, PG = 256 / HD;  // PG: heads a thread's output dim serves per pass
    __shared__ __attribute__((aligned(16))) float qs[GM * HD];
    __shared__ float ps[GM][CH];
    __shared__ float alpha_s[GM], l_s[GM];
    const int G = n_heads / n_kv;
    // the last rows (the longest key ranges) start first
    const int kvh = blockIdx.x, s = gridDim.y - 1 - blockIdx.y, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int qd = n_heads * HD;
    const int kv_len = pos0 + s + 1;
    for (int i = t; i < G * HD; i += 256) qs[i] = q[int64_t(s) * qstr + int64_t(kvh) * G * HD + i];  // qstr: q's row stride
    const float* kb = kc + int64_t(kvh) * max_seq * HD;
    const float* vb = vc + int64_t(kvh) * max_seq * HD;
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};  // heads wave and wave + 4
    float acc[GM / PG];
#pragma unroll
    for (int i = 0; i < GM / PG; ++i) acc[i] = 0.f;
    const int d = t % HD;
    __syncthreads();
    for (int c0 = 0; c0 < kv_len; c0 += CH) {
        // scores of (head g, key c0 + j)
        for (int i = t; i < G * CH; i += 256) {
            const int g = i / CH, j = i % CH, key = c0 + j;
            float sc = -INFINITY;
            if (key < kv_len) {
                const float4* kr = reinterpret_cast<const float4*>(kb + int64_t(key) * HD);
                const float4* qv = reinterpret_cast<const float4*>(qs + g * HD);
                float a = 0.f;
#pragma unroll 8
                for (int e = 0; e < HD / 4; ++e) {
                    const float4 kk = kr[e], qq = qv[e];
                    a = fmaf(qq.x, kk.x, a);
                    a = fmaf(qq.y, kk.y, a);
                    a = fmaf(qq.z, kk.z, a);
                    a = fmaf(qq.w, kk.w, a);
                }
                sc = a * scale;
            }
            ps[g][j] = sc;
        }
        __syncthreads();
        // online softmax: wave w owns heads w and w + 4
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int g = wave + 4 * r;
            if (g < G) {
                const float sv = ps[g][lane];
                const float m_new = fmaxf(m_run[r], wave_maximum(sv));
                const float p = sv == -INFINITY ? 0.f : expf(sv - m_new);
                const float alpha = m_run[r] == -INFINITY ? 0.f : expf(m_run[r] - m_new);
                l_run[r] = l_run[r] * alpha + wave_total(p);
                m_run[r] = m_new;
                ps[g][lane] = p;
                if (lane == 0) alpha_s[g] = alpha;
            }
        }
        __syncthreads();
        // acc[g] = acc[g] * alpha_g + sum_j p[g][j] v[c0 + j][d]
        const int nj = min(CH, kv_len - c0);
#pragma unroll
        for (int i = 0; i < GM / PG; ++i) {
            const int g = t / HD + PG * i;
            if (g < G) acc[i] *= alpha_s[g];
        }
        for (int j = 0; j < nj; ++j) {
            const float vv = vb[int64_t(c0 + j) * HD + d];
#pragma unroll
            for (int i = 0; i < GM / PG; ++i) {
                const int g = t / HD + PG * i;
                if (g < G) acc[i] = fmaf(ps[g][j], vv, acc[i]);
            }
        }
        __syncthreads();
    }
    if (lane == 0) {
        if (wave < G) l_s[wave] = l_run[0];
        if (wave + 4 < G) l_s[wave + 4] = l_run[1];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < GM / PG; ++i) {
        const int g = t / HD + PG * i;
        if (g < G) out[int64_t(s) * qd + (int64_t(kvh) * G + g) * HD + d] = acc[i] / l_s[g];
    }
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// The same causal GQA attention for a whole prompt block on f32 MFMA
// (v_mfma_f32_32x32x2_f32: f32 products and sums, so the scores carry no
// fp16 rounding), flash-attention style. Block (kvh, qb) takes prompt rows
// qb*QP .. qb*QP + QP - 1 (QP = 128 / G positions) for the G query heads of KV
// head kvh: 4 waves of 32 rows, row R = 32*wave + lane % 32 -> position
// qb*QP + R / G, head kvh*G + R % G. Key tiles of 32 positions, up to the
// block's last position, go through LDS once for all 128 rows:
//   * S^T = K Q^T (keys x rows): A = K from LDS (lane l: key l % 32, dims
//     (HD/2)*(l/32) + st), B = Q^T from registers (the lane's own row, the same
//     dims, pre-scaled by 1/sqrt(HD)); the accumulator holds, in lane l, row
//     l % 32 and keys 8*(r/4) + 4*(l/32) + r%4 of the tile (r < 16);
//   * so each lane's softmax is over its own registers plus the partner lane
//     l ^ 32 (one lane swap for the max and one for the sum), with the running
//     max, sum and rescale per row in the lane that owns the row;
//   * O^T += V^T P^T (dims x rows): A = V^T from LDS (stored transposed, keys
//     contiguous), B = P^T, which is the lane's probability registers as they
//     stand: step st pairs keys 8*(st/4) + 4*h + st%4, h = 0, 1 (lane halves).
// Keys past the causal end are masked to -inf; key rows past the last
// written cache row load that row instead (never stale memory), weighted 0.
template <int HD, int G>
__global__ void __launch_bounds__(256) k_attn_prefill_mf(const float* __restrict__ q, const float* __restrict__ kc,
                                                         const float* __restrict__ vc, float* __restrict__ out, int n,
                                                         int n_heads, int max_seq, int pos0, float scale, int qstr) {
    constexpr int QP = 128 / G, KT = 32, HH = HD / 2, NT = HD / 32;
    constexpr int KS = HD + 4;   // K row stride in LDS (floats)
    constexpr int VS = KT + 4;   // V^T row stride (one row per dim)
    __shared__ __attribute__((aligned(16))) float ks[KT * KS];
    __shared__ __attribute__((aligned(16))) float vt[HD * VS];
    // The last position blocks walk the most key tiles: they take the first
    // block ids, so that they start first and the short ones fill in behind.
    const int kvh = blockIdx.x, qb = gridDim.y - 1 - blockIdx.y;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, h = lane >> 5, j = lane & 31;
    const int R = 32 * wave + j;
    const int srow = min(qb * QP + R / G, n - 1);  // prompt row of this lane's query row (clamped rows store nothing)
    const bool live = qb * QP + R / G < n;
    const int head = kvh * G + R % G;
    const int qd = n_heads * HD;
    const int p_row = pos0 + srow;  // this row's position: keys 0..p_row
    const int last_pos = pos0 + min(n, qb * QP + QP) - 1;  // the block's last position
    // Q^T operand: this row's dims HH*h .. HH*h + HH - 1, scaled
    float qv[HH];
    {
        const float4* qr = reinterpret_cast<const float4*>(q + int64_t(srow) * qstr + int64_t(head) * HD + HH * h);
#pragma unroll
        for (int i = 0; i < HH / 4; ++i) {
            const float4 v4 = qr[i];
            qv[4 * i] = v4.x * scale;
            qv[4 * i + 1] = v4.y * scale;
            qv[4 * i + 2] = v4.z * scale;
            qv[4 * i + 3] = v4.w * scale;
        }
    }
    f32x16 o[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[nt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float* kb = kc + int64_t(kvh) * max_seq * HD;
    const float* vb = vc + int64_t(kvh) * max_seq * HD;
    const int ntiles = last_pos / KT + 1;
    for (int kt = 0; kt < ntiles; ++kt) {
        __syncthreads();  // the previous tile's readers are done
        // K rows into ks (row-major), V rows into vt (transposed: vt[dim][key])
        for (int i = t; i < KT * HD / 4; i += 256) {
            const int key = i / (HD / 4), c4 = i % (HD / 4);
            const int krow = min(kt * KT + key, last_pos);
            const float4 kk = reinterpret_cast<const float4*>(kb + int64_t(krow) * HD)[c4];
            const float4 vv = reinterpret_cast<const float4*>(vb + int64_t(krow) * HD)[c4];
            *reinterpret_cast<float4*>(&ks[key * KS + 4 * c4]) = kk;
            vt[(4 * c4) * VS + key] = vv.x;
            vt[(4 * c4 + 1) * VS + key] = vv.y;
            vt[(4 * c4 + 2) * VS + key] = vv.z;
            vt[(4 * c4 + 3) * VS + key] = vv.w;
        }
        __syncthreads();
        // S^T = K Q^T
        f32x16 sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
        const float* krow = ks + j * KS + HH * h;
#pragma unroll
        for (int st4 = 0; st4 < HH / 4; ++st4) {
            const float4 k4 = *reinterpret_cast<const float4*>(krow + 4 * st4);
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.x, qv[4 * st4], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.y, qv[4 * st4 + 1], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.z, qv[4 * st4 + 2], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(k4.w, qv[4 * st4 + 3], sacc, 0, 0, 0);
        }
        // mask, running max and sum of this lane's row
        float pv[16];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kt * KT + 8 * (r >> 2) + 4 * h + (r & 3);
            pv[r] = key <= p_row ? sacc[r] : -INFINITY;
            mt = fmaxf(mt, pv[r]);
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const float m_new = fmaxf(m_run, mt);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = pv[r] == -INFINITY ? 0.f : expf(pv[r] - m_new);
            ps += pv[r];
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
            ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[nt][r] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const float4 v4 = *reinterpret_cast<const float4*>(&vt[(32 * nt + j) * VS + 8 * a4 + 4 * h]);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4.x, pv[4 * a4], o[nt], 0, 0, 0);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4.y, pv[4 * a4 + 1], o[nt], 0, 0, 0);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4.z, pv[4 * a4 + 2], o[nt], 0, 0, 0);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(v4.w, pv[4 * a4 + 3], o[nt], 0, 0, 0);
            }
        }
    }
    if (!live) return;
    // lane l holds O^T[32nt + 8(r/4) + 4h + r%4][row l % 32]: four consecutive dims per r/4
    const float inv = 1.0f / l_run;
    float* orow = out + int64_t(srow) * qd + int64_t(head) * HD;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            *reinterpret_cast<float4*>(orow + 32 * nt + 8 * a + 4 * h) =
                make_float4(o[nt][4 * a] * inv, o[nt][4 * a + 1] * inv, o[nt][4 * a + 2] * inv, o[nt][4 * a + 3] * inv);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

// x = hi + lo to about 2^-16 relative: hi the nearest bf16, lo the nearest
// bf16 to the exact f32 remainder.
__device__ __forceinline__ void bf16_split(float x, __bf16& hi, __bf16& lo) {
    hi = __bf16(x);
    lo = __bf16(x - float(hi));
}

// k_attn_prefill_mf's attention with its products on bf16 MFMA
// (v_mfma_f32_32x32x16_bf16) in three terms: every f32 operand is split as
// hi + lo (bf16_split) and a product taken as hi*hi + hi*lo + lo*hi with f32
// sums, about 2^-16 relative per product against f32's 2^-24, in 48 MFMAs
// per key tile and wave instead of 128 f32 ones (each 5.3 times the cost).
// The prompt forward uses it where the block's projections run on the fp16
// GEMM (the 2e-3 bar); blocks on the f32 GEMVs keep the f32 kernel. Same
// block, row and tile mapping, softmax and masking as k_attn_prefill_mf; the
// K tile is staged as bf16 hi and lo rows, V^T likewise, and Q^T as hi and
// lo registers. A lane half h holds k slots 8h .. 8h+7 of each 16-deep MFMA
// step: dims 16s + 8h + b of K and Q in S^T = K Q^T; for O^T += V^T P^T the
// keys 16s + 4h + b (b < 4) and 16s + 8 + 4h + b - 4 (b >= 4), the order in
// which the lane's probability registers stand.
// KSPLIT: block z of gridDim.z takes the z-th of gridDim.z even ranges of its
// key tiles and stores, per row and head, the unnormalized output, the
// running max (log2 units) and the running sum to part ([z][n][heads][HD + 4],
// 16-byte rows: the output, then the max and the sum)
// for k_attn_prefill_merge; a range past a row's causal end leaves max
// -inf and sum 0, and range 0 always holds key 0.
template <int HD, int G, bool KSPLIT = false>
__global__ void __launch_bounds__(256) k_attn_prefill_bf(const float* __restrict__ q, const float* __restrict__ kc,
                                                         const float* __restrict__ vc, float* __restrict__ out, int n,
                                                         int n_heads, int max_seq, int pos0, float scale, int qstr,
                                                         float* __restrict__ part) {
    constexpr int QP = 128 / G, KT = 32, NT = HD / 32, NS = HD / 16;
    constexpr int KSB = HD + 8;  // bf16 K row stride in LDS
    constexpr int VSB = KT + 8;  // bf16 V^T row stride (one row per dim)
    // two tile buffers: tile kt + 1 is loaded while tile kt is used
    __shared__ __attribute__((aligned(16))) __bf16 khi[2][KT * KSB];
    __shared__ __attribute__((aligned(16))) __bf16 klo[2][KT * KSB];
    __shared__ __attribute__((aligned(16))) __bf16 vhi[2][HD * VSB];
    __shared__ __attribute__((aligned(16))) __bf16 vlo[2][HD * VSB];
    // V^T element (dim, key): the 4-key blocks of a dim's row are XOR-swizzled
    // by (dim / 16) % 8, so that the 32 dims one staging store writes (4c4 + e,
    // c4 < 32, one key) fall in distinct banks (unswizzled, 20 c4 dwords apart
    // mod 64, 8 lanes share a bank); a 4-key block stays contiguous for the
    // 8-byte operand reads.
    auto vt_at = [](int dim, int key) { return dim * VSB + ((((key >> 2) ^ (dim >> 4)) & 7) << 2) + (key & 3); };
    const int kvh = blockIdx.x, qb = gridDim.y - 1 - blockIdx.y;  // longest key ranges first
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, h = lane >> 5, j = lane & 31;
    const int R = 32 * wave + j;
    const int srow = min(qb * QP + R / G, n - 1);  // prompt row of this lane's query row (clamped rows store nothing)
    const bool live = qb * QP + R / G < n;
    const int head = kvh * G + R % G;
    const int qd = n_heads * HD;
    const int p_row = pos0 + srow;
    const int last_pos = pos0 + min(n, qb * QP + QP) - 1;
    // Q^T operand: this row's dims 16s + 8h .. 16s + 8h + 7 per step s, scaled, split
    // scores in log2 units (1/sqrt(HD) * log2(e) folded into Q), so each
    // exponential is one v_exp_f32
    const float scale2 = scale * 1.44269504088896341f;
    bf16x8 qh[NS], ql[NS];
    {
        const float* qr = q + int64_t(srow) * qstr + int64_t(head) * HD + 8 * h;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const float4 a = *reinterpret_cast<const float4*>(qr + 16 * st);
            const float4 b = *reinterpret_cast<const float4*>(qr + 16 * st + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 hi, lo;
                bf16_split(v[e] * scale2, hi, lo);
                qh[st][e] = hi;
                ql[st][e] = lo;
            }
        }
    }
    f32x16 o[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[nt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float* kb = kc + int64_t(kvh) * max_seq * HD;
    const float* vb = vc + int64_t(kvh) * max_seq * HD;
    const int ntiles = last_pos / KT + 1;
    int kt0 = 0, kt1 = ntiles;  // this block's key tiles
    if constexpr (KSPLIT) {
        const int per = (ntiles + int(gridDim.z) - 1) / int(gridDim.z);
        kt0 = min(ntiles, int(blockIdx.z) * per);
        kt1 = min(ntiles, kt0 + per);
    }
    constexpr int NI = KT * HD / 4 / 256;  // float4 items of K (and of V) per thread and tile
    float4 pk[NI], pv[NI];
    auto gload = [&](int kt) {
#pragma unroll
        for (int u = 0; u < NI; ++u) {
            const int i = t + 256 * u, key = i / (HD / 4), c4 = i % (HD / 4);
            const int krow = min(kt * KT + key, last_pos);
            pk[u] = reinterpret_cast<const float4*>(kb + int64_t(krow) * HD)[c4];
            pv[u] = reinterpret_cast<const float4*>(vb + int64_t(krow) * HD)[c4];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int u = 0; u < NI; ++u) {
            const int i = t + 256 * u, key = i / (HD / 4), c4 = i % (HD / 4);
            const float kv[4] = {pk[u].x, pk[u].y, pk[u].z, pk[u].w}, vw[4] = {pv[u].x, pv[u].y, pv[u].z, pv[u].w};
            bf16x4 k_h, k_l;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                __bf16 hi, lo;
                bf16_split(kv[e], hi, lo);
                k_h[e] = hi;
                k_l[e] = lo;
                bf16_split(vw[e], hi, lo);
                const int vi = vt_at(4 * c4 + e, key);
                vhi[buf][vi] = hi;
                vlo[buf][vi] = lo;
            }
            *reinterpret_cast<bf16x4*>(&khi[buf][key * KSB + 4 * c4]) = k_h;
            *reinterpret_cast<bf16x4*>(&klo[buf][key * KSB + 4 * c4]) = k_l;
        }
    };
    if (!KSPLIT || kt0 < kt1) {  // an unsplit block always has a tile
        gload(kt0);
        lstore(0);
    }
    __syncthreads();
    for (int kt = kt0; kt < kt1; ++kt) {
        const int buf = (kt - kt0) & 1;
        if (kt + 1 < kt1) gload(kt + 1);  // in flight through this tile's MFMAs
        // S^T = K Q^T
        f32x16 sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
        for (int st = 0; st < NS; ++st) {
            const bf16x8 a_h = *reinterpret_cast<const bf16x8*>(&khi[buf][j * KSB + 16 * st + 8 * h]);
            const bf16x8 a_l = *reinterpret_cast<const bf16x8*>(&klo[buf][j * KSB + 16 * st + 8 * h]);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, qh[st], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, ql[st], sacc, 0, 0, 0);
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, qh[st], sacc, 0, 0, 0);
        }
        // mask, running max and sum of this lane's row
        float pv[16];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = kt * KT + 8 * (r >> 2) + 4 * h + (r & 3);
            pv[r] = key <= p_row ? sacc[r] : -INFINITY;
            mt = fmaxf(mt, pv[r]);
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
            mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
        }
        const float m_new = fmaxf(m_run, mt);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = pv[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pv[r] - m_new);
            ps += pv[r];
        }
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(ps), __float_as_uint(ps), false, false);
            ps = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run = l_run * alpha + ps;
        m_run = m_new;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[nt][r] *= alpha;
        // O^T += V^T P^T, two 16-key steps
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            bf16x8 p_h, p_l;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                __bf16 hi, lo;
                bf16_split(pv[8 * st + e], hi, lo);
                p_h[e] = hi;
                p_l[e] = lo;
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int dim = 32 * nt + j, v0 = vt_at(dim, 16 * st + 4 * h), v1 = vt_at(dim, 16 * st + 8 + 4 * h);
                const bf16x4 h0 = *reinterpret_cast<const bf16x4*>(&vhi[buf][v0]);
                const bf16x4 h1 = *reinterpret_cast<const bf16x4*>(&vhi[buf][v1]);
                const bf16x4 l0 = *reinterpret_cast<const bf16x4*>(&vlo[buf][v0]);
                const bf16x4 l1 = *reinterpret_cast<const bf16x4*>(&vlo[buf][v1]);
                const bf16x8 a_h = {h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                const bf16x8 a_l = {l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, p_h, o[nt], 0, 0, 0);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_h, p_l, o[nt], 0, 0, 0);
                o[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_l, p_h, o[nt], 0, 0, 0);
            }
        }
        if (kt + 1 < kt1) lstore(buf ^ 1);  // the other buffer's readers finished before the last barrier
        __syncthreads();
    }
    if (!live) return;
    // lane l holds O^T[32nt + 8(r/4) + 4h + r%4][row l % 32]: four consecutive dims per r/4
    if constexpr (KSPLIT) {
        float* prow = part + ((int64_t(blockIdx.z) * n + srow) * n_heads + head) * (HD + 4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int a = 0; a < 4; ++a)
                *reinterpret_cast<float4*>(prow + 32 * nt + 8 * a + 4 * h) =
                    make_float4(o[nt][4 * a], o[nt][4 * a + 1], o[nt][4 * a + 2], o[nt][4 * a + 3]);
        if (h == 0) {
            prow[HD] = m_run;
            prow[HD + 1] = l_run;
        }
        return;
    }
    const float inv = 1.0f / l_run;
    float* orow = out + int64_t(srow) * qd + int64_t(head) * HD;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int a = 0; a < 4; ++a)
            *reinterpret_cast<float4*>(orow + 32 * nt + 8 * a + 4 * h) =
                make_float4(o[nt][4 * a] * inv, o[nt][4 * a + 1] * inv, o[nt][4 * a + 2] * inv, o[nt][4 * a + 3] * inv);
}

// The key-split prompt attention's rows: per (row, head), the ks ranges'
// outputs o_z, maxima m_z (log2 units) and sums l_z meet as
// sum_z 2^(m_z - M) o_z / sum_z 2^(m_z - M) l_z, M = max_z m_z (ranges with
// m_z = -inf count 0). One block per (row, head), one thread per dim, every
// range's values loaded before the first add.
template <int HD>
__global__ void __launch_bounds__(HD) k_attn_prefill_merge(const float* __restrict__ part, float* __restrict__ out,
                                                           int n, int n_heads, int ks) {
    constexpr int KS = 8;
    const int s = blockIdx.x, head = blockIdx.y, dim = threadIdx.x;
    float mv[KS], lv[KS], ov[KS];
#pragma unroll
    for (int z = 0; z < KS; ++z) {
        if (z < ks) {
            const float* p = part + ((int64_t(z) * n + s) * n_heads + head) * (HD + 4);
            mv[z] = p[HD];
            lv[z] = p[HD + 1];
            ov[z] = p[dim];
        }
    }
    float M = mv[0];
#pragma unroll
    for (int z = 1; z < KS; ++z)
        if (z < ks) M = fmaxf(M, mv[z]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int z = 0; z < KS; ++z) {
        if (z < ks && mv[z] != -INFINITY) {
            const float w = exp2f(mv[z] - M);
            num = fmaf(w, ov[z], num);
            den = fmaf(w, lv[z], den);
        }
    }
    out[(int64_t(s) * n_heads + head) * HD + dim] = num / den;
}

// ---------------------------------------------------------------------------
// Decoder object
// ---------------------------------------------------------------------------

struct Layer {
    DevBlob w[7];  // q, k, v, o, gate, up, down
    // Decoder-owned fused copies (row-interleaved blobs only): Q|K|V stacked
    // (one launch writes q, k, v contiguously) and gate/up row pairs (one
    // launch with the SwiGLU epilogue).
    DevBlob qkv{}, gu{};
    bool has_qkv = false, has_gu = false;
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    float* kc = nullptr;
    float* vc = nullptr;
    bool set = false;
};

struct Decoder {
    wv_decoder_config c{};
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<Layer> layers;
    DevBlob lm{};
    bool lm_set = false;
    float* final_norm = nullptr;  // allocated once; used while has_final_norm
    bool has_final_norm = false;
    float* embed = nullptr;
    float* gemv_scratch = nullptr;  // K-split partials of the projections (decoder-owned)
    size_t gemv_scratch_floats = 0;
    // activations and state
    float *h = nullptr, *n = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr;
    float *g = nullptr, *u = nullptr, *logits = nullptr, *part = nullptr;
    int32_t* d_state = nullptr;  // {pos, token, next, step}
    int32_t* d_pos = nullptr;    // = d_state
    int32_t* d_tok = nullptr;    // = d_state + 1
    int32_t* d_gen = nullptr;    // [max_seq] generated tokens
    float* ss_a = nullptr;       // [hidden/16] partial sums of h^2 for the attention norm / final norm
    float* ss_b = nullptr;       // [hidden/16] partial sums of h^2 for the FFN norm
    bool fused_norm = false;     // every norm folded into its consumer GEMV
    double* freq_div = nullptr;  // [head_dim/2] theta^(2d/hd)
    double2* cs = nullptr;       // [head_dim/2] this step's (cos, sin)
    int n_chunks = 0;
    std::vector<void*> allocs;
    bool use_graph = false;
    int graph_advance = -1;
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    // prompt forward (wv_decoder_prefill): rows of every prompt token, grown on demand
    int pcap = 0;
    float *ph = nullptr, *pn = nullptr, *pq = nullptr, *pk = nullptr, *pv = nullptr, *patt = nullptr;
    float *pg = nullptr, *pu = nullptr, *pt = nullptr, *pscratch = nullptr;
    float* pxh = nullptr;  // the fp16 GEMM operand shared by the projections of one input, then its row factors
    int32_t* ptok = nullptr;
    size_t pscratch_floats = 0, pxh_floats = 0;
};

std::mutex g_dmu;
std::unordered_map<uint64_t, Decoder*> g_decs;
uint64_t g_dnext = 1;

Decoder* find(uint64_t h) {
    std::lock_guard<std::mutex> lk(g_dmu);
    auto it = g_decs.find(h);
    return it == g_decs.end() ? nullptr : it->second;
}

int dalloc(Decoder& d, void** p, size_t bytes, const char* what) {
    hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 256));
    if (e != hipSuccess) return rt_hip_fail(e, what);
    d.allocs.push_back(*p);
    return WV_OK;
}

void drop_fused(Layer& ly) {
    if (ly.has_qkv) (void)hipFree(ly.qkv.base);
    if (ly.has_gu) (void)hipFree(ly.gu.base);
    ly.has_qkv = ly.has_gu = false;
}

void drop_graph(Decoder& d) {
    if (d.exec) (void)hipGraphExecDestroy(d.exec);
    if (d.graph) (void)hipGraphDestroy(d.graph);
    d.exec = nullptr;
    d.graph = nullptr;
}

void drop_prefill(Decoder& d) {
    for (void* p : {static_cast<void*>(d.ph), static_cast<void*>(d.pn), static_cast<void*>(d.pq),
                    static_cast<void*>(d.pk), static_cast<void*>(d.pv), static_cast<void*>(d.patt),
                    static_cast<void*>(d.pg), static_cast<void*>(d.pu), static_cast<void*>(d.pt),
                    static_cast<void*>(d.pscratch), static_cast<void*>(d.pxh), static_cast<void*>(d.ptok)})
        if (p) (void)hipFree(p);
    d.ph = d.pn = d.pq = d.pk = d.pv = d.patt = d.pg = d.pu = d.pt = d.pscratch = d.pxh = nullptr;
    d.ptok = nullptr;
    d.pcap = 0;
    d.pscratch_floats = d.pxh_floats = 0;
}

void release(Decoder* d) {
    drop_graph(*d);
    drop_prefill(*d);
    if (d->gemv_scratch) (void)hipFree(d->gemv_scratch);
    for (Layer& ly : d->layers) drop_fused(ly);
    for (void* p : d->allocs) (void)hipFree(p);
    if (d->stream) (void)hipStreamDestroy(d->stream);
    delete d;
}

// y (op)= W x for one projection: fused epilogue on the row-interleaved layout,
// separate elementwise kernels otherwise.
int proj(Decoder& d, const DevBlob& w, const float* x, float* y, int mode, const float* aux, float* tmp) {
    if (w.layout == LAYOUT_RPL) return launch_rpl(w, x, y, 1, d.stream, mode, aux, d.gemv_scratch);
    const int rows = int(w.rows);
    float* out = mode == RPL_STORE ? y : tmp;
    int e = launch_matvec(w, x, out, 1, d.stream, d.gemv_scratch);
    if (e) return e;
    if (mode == RPL_ADD) hipLaunchKernelGGL(k_add, dim3((rows + 255) / 256), dim3(256), 0, d.stream, y, tmp, rows);
    if (mode == RPL_SILU_MUL)
        hipLaunchKernelGGL(k_silu_mul, dim3((rows + 255) / 256), dim3(256), 0, d.stream, aux, tmp, y, rows);
    return int(hipGetLastError());
}

// Enqueues one whole step on d.stream (token and position from device memory).
// The combine variant is fixed by the chunk count the cache can reach.
void launch_combine(Decoder& d, int hd) {
    const dim3 grid(unsigned(d.c.n_heads)), grid2(unsigned(d.c.n_heads), unsigned(hd / 64));  // grid2: k_attn_combine
    const int nc = d.n_chunks;
    if (nc <= 64 && hd == 128)
        hipLaunchKernelGGL((k_attn_combine<128, 1>), grid2, dim3(256), 0, d.stream, d.part, d.att, nc, d.d_pos, d.c.max_seq);
    else if (nc <= 64)
        hipLaunchKernelGGL((k_attn_combine<64, 1>), grid2, dim3(256), 0, d.stream, d.part, d.att, nc, d.d_pos, d.c.max_seq);
    else if (nc <= 128 && hd == 128)
        hipLaunchKernelGGL((k_attn_combine<128, 2>), grid2, dim3(256), 0, d.stream, d.part, d.att, nc, d.d_pos, d.c.max_seq);
    else if (nc <= 128)
        hipLaunchKernelGGL((k_attn_combine<64, 2>), grid2, dim3(256), 0, d.stream, d.part, d.att, nc, d.d_pos, d.c.max_seq);
    else
        hipLaunchKernelGGL(k_attn_combine_long, grid, dim3(256), 0, d.stream, d.part, d.att, hd, nc, d.d_pos, d.c.max_seq);
}

// Attention partials of one layer: the register kernel for G = 1, 2, 4, 8
// query heads per KV head, the LDS-tile kernel otherwise.
void launch_attn(Decoder& d, Layer& ly, int G, float scale) {
    const wv_decoder_config& c = d.c;
    const dim3 ag(unsigned(c.n_kv_heads), unsigned(d.n_chunks));
    auto reg = [&](auto kern) {
        hipLaunchKernelGGL(kern, ag, dim3(256), 0, d.stream, d.q, ly.kc, ly.vc, d.d_pos, d.part, c.max_seq,
                           d.n_chunks, scale, d.k, d.v, d.cs);
    };
    if (c.head_dim == 128) {
        switch (G) {
            case 1: return reg(k_attn_reg<128, 1>);
            case 2: return reg(k_attn_reg<128, 2>);
            case 4: return reg(k_attn_reg<128, 4>);
            case 8: return reg(k_attn_reg<128, 8>);
        }
    } else {
        switch (G) {
            case 1: return reg(k_attn_reg<64, 1>);
            case 2: return reg(k_attn_reg<64, 2>);
            case 4: return reg(k_attn_reg<64, 4>);
            case 8: return reg(k_attn_reg<64, 8>);
        }
    }
    const size_t qsh = size_t(G) * c.head_dim * sizeof(float);
    if (c.head_dim == 128)
        hipLaunchKernelGGL(k_attn_part<128>, ag, dim3(256), qsh, d.stream, d.q, ly.kc, ly.vc, d.d_pos, d.part,
                           c.n_heads, c.n_kv_heads, c.max_seq, d.n_chunks, scale, d.k, d.v, d.cs);
    else
        hipLaunchKernelGGL(k_attn_part<64>, ag, dim3(256), qsh, d.stream, d.q, ly.kc, ly.vc, d.d_pos, d.part,
                           c.n_heads, c.n_kv_heads, c.max_seq, d.n_chunks, scale, d.k, d.v, d.cs);
}

int enqueue_step(Decoder& d, int advance) {
    const wv_decoder_config& c = d.c;
    const int hd = c.head_dim;
    const float scale = float(1.0 / std::sqrt(double(hd)));
    const int G = c.n_heads / c.n_kv_heads;
    const bool fn = d.fused_norm;
    const int nss = c.hidden / 16;  // sum-of-squares partials per 16 rows
    hipLaunchKernelGGL(k_embed, dim3((c.hidden + 255) / 256), dim3(256), 0, d.stream, d.embed, d.d_tok, d.h, c.hidden,
                       c.vocab, d.freq_div, d.cs, hd / 2, d.d_pos, fn ? d.ss_a : nullptr);
    float* tmp = d.logits;  // scratch for the non-fused projection epilogues (>= max(rows) floats)
    auto normed = [&](const float* gamma, const float* ss, int mode, float* ss_out) {
        RplExtra ex;
        ex.mode = mode;
        ex.nrm_gamma = gamma;
        ex.nrm_ss = ss;
        ex.nrm_n = nss;
        ex.nrm_eps = c.rms_eps;
        ex.ss_out = ss_out;
        ex.partial = d.gemv_scratch;
        return ex;
    };
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = d.layers[L];
        int e = 0;
        if (fn) {
            e = launch_rpl_ex(ly.qkv, d.h, d.q, 1, d.stream, normed(ly.attn_norm, d.ss_a, RPL_STORE, nullptr));
        } else {
            hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, d.stream, d.h, ly.attn_norm, d.n, c.hidden, c.rms_eps);
            if (ly.has_qkv) {
                e = launch_rpl(ly.qkv, d.n, d.q, 1, d.stream, RPL_STORE, nullptr, d.gemv_scratch);  // q, k, v are contiguous
            } else {
                e = proj(d, ly.w[0], d.n, d.q, RPL_STORE, nullptr, tmp);
                if (!e) e = proj(d, ly.w[1], d.n, d.k, RPL_STORE, nullptr, tmp);
                if (!e) e = proj(d, ly.w[2], d.n, d.v, RPL_STORE, nullptr, tmp);
            }
        }
        if (e) return e;
        launch_attn(d, ly, G, scale);
        launch_combine(d, hd);
        if (fn) {
            e = launch_rpl_ex(ly.w[3], d.att, d.h, 1, d.stream, normed(nullptr, nullptr, RPL_ADD, d.ss_b));
            if (!e) e = launch_rpl_ex(ly.gu, d.h, d.u, 1, d.stream, normed(ly.ffn_norm, d.ss_b, RPL_SWIGLU, nullptr));
            if (!e) e = launch_rpl_ex(ly.w[6], d.u, d.h, 1, d.stream, normed(nullptr, nullptr, RPL_ADD, d.ss_a));
            if (e) return e;
            continue;
        }
        e = proj(d, ly.w[3], d.att, d.h, RPL_ADD, nullptr, tmp);
        if (e) return e;
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, d.stream, d.h, ly.ffn_norm, d.n, c.hidden, c.rms_eps);
        if (ly.has_gu) {
            e = launch_rpl(ly.gu, d.n, d.u, 1, d.stream, RPL_SWIGLU, nullptr, d.gemv_scratch);
        } else {
            e = proj(d, ly.w[4], d.n, d.g, RPL_STORE, nullptr, tmp);
            if (!e) e = proj(d, ly.w[5], d.n, d.u, RPL_SILU_MUL, d.g, tmp);
        }
        if (!e) e = proj(d, ly.w[6], d.u, d.h, RPL_ADD, nullptr, tmp);
        if (e) return e;
    }
    int e = 0;
    if (fn && d.has_final_norm) {
        e = launch_rpl_ex(d.lm, d.h, d.logits, 1, d.stream, normed(d.final_norm, d.ss_a, RPL_STORE, nullptr));
    } else {
        const float* fin = d.h;
        if (d.has_final_norm) {
            hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, d.stream, d.h, d.final_norm, d.n, c.hidden,
                               c.rms_eps);
            fin = d.n;
        }
        e = proj(d, d.lm, fin, d.logits, RPL_STORE, nullptr, nullptr);
    }
    if (e) return e;
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, d.stream, d.logits, c.vocab, d.d_state, d.d_gen,
                       c.max_seq, advance);
    return int(hipGetLastError());
}

// Every norm can be folded into its consumer when all projections are on the
// row-interleaved layout with Q|K|V and gate/up fused (the residual GEMVs then
// produce the sums of squares the next norm needs).
bool can_fuse_norms(const Decoder& d) {
    if (d.c.hidden % 256) return false;
    for (const Layer& ly : d.layers)
        if (!ly.has_qkv || !ly.has_gu || ly.w[3].layout != LAYOUT_RPL || ly.w[6].layout != LAYOUT_RPL) return false;
    return d.lm.layout == LAYOUT_RPL;
}

int ready(Decoder& d) {
    for (int L = 0; L < d.c.n_layers; ++L)
        if (!d.layers[L].set) return rt_fail(WV_E_ARG, "decoder: layer %d has no weights (wv_decoder_set_layer)", L);
    if (!d.lm_set || !d.embed) return rt_fail(WV_E_ARG, "decoder: no LM head / embedding (wv_decoder_set_output)");
    const bool fn = can_fuse_norms(d);
    if (fn != d.fused_norm) drop_graph(d);
    d.fused_norm = fn;
    // K-split scratch of the widest projection plan; a captured graph holds
    // its address, so growing it means capturing again.
    size_t need = matvec_scratch_floats(d.lm, 1);
    for (const Layer& ly : d.layers) {
        for (const DevBlob& w : ly.w) need = std::max(need, matvec_scratch_floats(w, 1));
        if (ly.has_qkv) need = std::max(need, matvec_scratch_floats(ly.qkv, 1));
        if (ly.has_gu) need = std::max(need, matvec_scratch_floats(ly.gu, 1));
    }
    if (need > d.gemv_scratch_floats) {
        drop_graph(d);
        if (d.gemv_scratch) (void)hipFree(d.gemv_scratch);
        d.gemv_scratch = nullptr;
        d.gemv_scratch_floats = 0;
        const hipError_t e = hipMalloc(&d.gemv_scratch, need * sizeof(float));
        if (e != hipSuccess) {
            d.gemv_scratch = nullptr;
            return rt_hip_fail(e, "decoder: projection scratch");
        }
        d.gemv_scratch_floats = need;
    }
    return WV_OK;
}

// One projection of a prompt block: the prefill GEMM where the blob has one,
// the batched GEMVs otherwise.
// The GEMM input of a prompt block's projection: its f32 rows (x, and u for
// the SwiGLU product silu(x) * u) and the operand order of the fp16 copy in
// d.pxh. Consecutive projections of one input (Q, K, V; gate and up) find the
// copy made and convert nothing.
struct PrefillX {
    const float* x = nullptr;
    const float* u = nullptr;
    int64_t cols = 0;
    int frag = -1;
};

// y = W x for n prompt rows; with u the input is silu(x) * u. The GEMM takes
// the shared fp16 copy of its input (made here when cx does not hold it);
// other blobs take the batched GEMV on f32 rows, with tmp holding the SwiGLU
// rows. With `splits`, a K-split GEMM of at most 4 splits leaves its
// unsummed slices in d.pscratch and stores their count (1: y holds the
// result); more splits are summed into y here.
int prefill_proj(Decoder& d, PrefillX& cx, const DevBlob& w, const float* x, const float* u, float* y, int n,
                 float* tmp, int* splits = nullptr) {
    if (splits) *splits = 1;
    if (gemm_supported(w, n)) {
        const int frag = gemm_x_frag(w, n) ? 1 : 0;
        if (cx.x != x || cx.u != u || cx.cols != w.cols || cx.frag != frag) {
            gemm_convert_x(x, u, int(w.cols), n, frag != 0, d.pxh, d.pxh + gemm_x_floats(w, n), d.stream);
            cx = PrefillX{x, u, w.cols, frag};
        }
        const int e = launch_gemm_xh(w, d.pxh, d.pxh + gemm_x_floats(w, n), y, n, d.stream, d.pscratch, splits);
        if (!e && splits && *splits > 4) {
            launch_split_sum(d.pscratch, y, int64_t(n) * w.rows, *splits, d.stream);
            *splits = 1;
        }
        return e;
    }
    const float* xin = x;
    if (u) {
        const int64_t nin = int64_t(n) * w.cols;
        hipLaunchKernelGGL(k_silu_mul, dim3(unsigned((nin + 255) / 256)), dim3(256), 0, d.stream, x, u, tmp, int(nin));
        xin = tmp;
    }
    return launch_matvec(w, xin, y, n, d.stream, d.pscratch);
}

// Key splits of the bf16x3 prompt attention: its (KV head, 128 / G position)
// blocks, when under one pass of the GPU, each take ks ranges of their key
// tiles, ks = min(8, 256 / blocks, key tiles of the longest range); the
// pos0-free bound sizes the scratch.
int attn_key_splits(const wv_decoder_config& c, int n, int pos0) {
    const int G = c.n_heads / c.n_kv_heads;
    const int64_t blocks = int64_t(c.n_kv_heads) * ((n + 128 / G - 1) / (128 / G));
    const int64_t tiles = pos0 < 0 ? 8 : (int64_t(pos0) + n - 1) / 32 + 1;
    return int(std::max<int64_t>(1, std::min<int64_t>({8, 256 / std::max<int64_t>(blocks, 1), tiles})));
}
size_t attn_part_floats(const wv_decoder_config& c, int n) {
    const int ks = attn_key_splits(c, n, -1);
    return ks > 1 ? size_t(ks) * n * c.n_heads * (c.head_dim + 4) : 0;
}

size_t prefill_proj_scratch(const DevBlob& w, int n) {
    return gemm_supported(w, n) ? gemm_scratch_floats(w, n) : matvec_scratch_floats(w, n);
}

int ensure_prefill(Decoder& d, int n) {
    const wv_decoder_config& c = d.c;
    size_t need_s = 0;
    size_t need_x = 0;  // the widest fp16 copy of a GEMM input, then its row factors
    for (const Layer& ly : d.layers) {
        auto need = [&](const DevBlob& w) {
            need_s = std::max(need_s, prefill_proj_scratch(w, n));
            if (gemm_supported(w, n)) need_x = std::max(need_x, gemm_x_floats(w, n) + gemm_scale_floats(n));
        };
        for (const DevBlob& w : ly.w) need(w);
        if (ly.has_qkv) need(ly.qkv);
    }
    need_s = std::max(need_s, attn_part_floats(c, n));  // the key-split attention's ranges (between RoPE and O)
    if (n <= d.pcap && need_s <= d.pscratch_floats && need_x <= d.pxh_floats) return WV_OK;
    drop_prefill(d);
    const size_t qd = size_t(c.n_heads) * c.head_dim, kvd = size_t(c.n_kv_heads) * c.head_dim;
    const size_t wide = std::max({size_t(c.hidden), size_t(c.ffn), qd});
    struct {
        void** p;
        size_t bytes;
    } bufs[] = {{reinterpret_cast<void**>(&d.ph), n * size_t(c.hidden) * 4},
                {reinterpret_cast<void**>(&d.pn), n * size_t(c.hidden) * 4},
                {reinterpret_cast<void**>(&d.pq), n * (qd + 2 * kvd) * 4},  // q | k | v rows of the fused GEMM
                {reinterpret_cast<void**>(&d.pk), n * kvd * 4},
                {reinterpret_cast<void**>(&d.pv), n * kvd * 4},
                {reinterpret_cast<void**>(&d.patt), n * qd * 4},
                {reinterpret_cast<void**>(&d.pg), n * size_t(c.ffn) * 4},
                {reinterpret_cast<void**>(&d.pu), n * size_t(c.ffn) * 4},
                {reinterpret_cast<void**>(&d.pt), n * wide * 4},
                {reinterpret_cast<void**>(&d.pscratch), std::max<size_t>(need_s, 1) * 4},
                {reinterpret_cast<void**>(&d.pxh), std::max<size_t>(need_x, 1) * 4},
                {reinterpret_cast<void**>(&d.ptok), size_t(n) * 4}};
    for (auto& b : bufs) {
        const hipError_t e = hipMalloc(b.p, std::max<size_t>(b.bytes, 256));
        if (e != hipSuccess) {
            *b.p = nullptr;
            drop_prefill(d);
            return rt_hip_fail(e, "wv_decoder_prefill: buffers");
        }
    }
    d.pcap = n;
    d.pscratch_floats = std::max<size_t>(need_s, 1);
    d.pxh_floats = std::max<size_t>(need_x, 1);
    return WV_OK;
}

// ForwardTokens over n prompt tokens at positions pos0 .. pos0+n-1
// (model/transformer/forward.go:26-90 with the whole block): per layer
// RMSNorm of every row, Q/K/V for the block, RoPE and the KV append, causal
// attention, O + residual, RMSNorm, SwiGLU + residual; then the final norm,
// LM head and argmax of the last row into the decoder state (state[2]).
// The MFMA attention of a prompt block, for head dims 64 and 128 and 1, 2, 4
// or 8 query heads per KV head (bf: the bf16x3 products of k_attn_prefill_bf,
// else f32), q's rows qstr floats apart; false: the shape takes k_attn_prefill.
// The key-split attention's ranges merged into the f32 rows d.patt.
void launch_attn_merge(Decoder& d, int n, int ks) {
    const wv_decoder_config& c = d.c;
    if (c.head_dim == 128)
        hipLaunchKernelGGL(k_attn_prefill_merge<128>, dim3(unsigned(n), unsigned(c.n_heads)), dim3(128), 0, d.stream,
                           d.pscratch, d.patt, n, c.n_heads, ks);
    else
        hipLaunchKernelGGL(k_attn_prefill_merge<64>, dim3(unsigned(n), unsigned(c.n_heads)), dim3(64), 0, d.stream,
                           d.pscratch, d.patt, n, c.n_heads, ks);
}

// With ks_out, a key-split launch leaves its ranges in d.pscratch unmerged
// and stores their count there (1: d.patt holds the rows).
bool launch_attn_prefill_mf(Decoder& d, Layer& ly, const float* q, int qstr, int n, int pos0, float scale, bool bf,
                            int* ks_out = nullptr) {
    const wv_decoder_config& c = d.c;
    const int G = c.n_heads / c.n_kv_heads, hd = c.head_dim;
    if ((hd != 64 && hd != 128) || (G != 1 && G != 2 && G != 4 && G != 8)) return false;
    const int ks = bf ? attn_key_splits(c, n, pos0) : 1;
    const dim3 grid(unsigned(c.n_kv_heads), unsigned((n + 128 / G - 1) / (128 / G)), unsigned(ks));
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, d.stream, q, ly.kc, ly.vc, d.patt, n, c.n_heads, c.max_seq, pos0,
                           scale, qstr);
    };
    auto gob = [&](auto kern, auto kern_split) {
        if (ks == 1)
            hipLaunchKernelGGL(kern, grid, dim3(256), 0, d.stream, q, ly.kc, ly.vc, d.patt, n, c.n_heads, c.max_seq,
                               pos0, scale, qstr, nullptr);
        else
            hipLaunchKernelGGL(kern_split, grid, dim3(256), 0, d.stream, q, ly.kc, ly.vc, d.patt, n, c.n_heads,
                               c.max_seq, pos0, scale, qstr, d.pscratch);
    };
    if (hd == 128) {
        switch (G) {
        case 1: bf ? gob(k_attn_prefill_bf<128, 1>, k_attn_prefill_bf<128, 1, true>) : go(k_attn_prefill_mf<128, 1>); break;
        case 2: bf ? gob(k_attn_prefill_bf<128, 2>, k_attn_prefill_bf<128, 2, true>) : go(k_attn_prefill_mf<128, 2>); break;
        case 4: bf ? gob(k_attn_prefill_bf<128, 4>, k_attn_prefill_bf<128, 4, true>) : go(k_attn_prefill_mf<128, 4>); break;
        default: bf ? gob(k_attn_prefill_bf<128, 8>, k_attn_prefill_bf<128, 8, true>) : go(k_attn_prefill_mf<128, 8>); break;
        }
    } else {
        switch (G) {
        case 1: bf ? gob(k_attn_prefill_bf<64, 1>, k_attn_prefill_bf<64, 1, true>) : go(k_attn_prefill_mf<64, 1>); break;
        case 2: bf ? gob(k_attn_prefill_bf<64, 2>, k_attn_prefill_bf<64, 2, true>) : go(k_attn_prefill_mf<64, 2>); break;
        case 4: bf ? gob(k_attn_prefill_bf<64, 4>, k_attn_prefill_bf<64, 4, true>) : go(k_attn_prefill_mf<64, 4>); break;
        default: bf ? gob(k_attn_prefill_bf<64, 8>, k_attn_prefill_bf<64, 8, true>) : go(k_attn_prefill_mf<64, 8>); break;
        }
    }
    if (ks_out) *ks_out = ks;
    else if (ks > 1) launch_attn_merge(d, n, ks);
    return true;
}

int enqueue_prefill(Decoder& d, int n, int pos0) {
    const wv_decoder_config& c = d.c;
    const int hd = c.head_dim, hidden = c.hidden;
    const float scale = float(1.0 / std::sqrt(double(hd)));
    hipLaunchKernelGGL(k_embed_rows, dim3(unsigned((hidden + 255) / 256), unsigned(n)), dim3(256), 0, d.stream, d.embed,
                       d.ptok, d.ph, hidden, c.vocab);
    // The fp16 operand order a projection's GEMM reads (1: A fragments, 0:
    // row-major), or -1 for the batched GEMV; where every GEMM after a norm
    // reads one order, the norm writes that operand itself
    auto xorder = [&](const DevBlob& w) { return gemm_supported(w, n) ? (gemm_x_frag(w, n) ? 1 : 0) : -1; };
    float* xscale = d.pxh + (d.layers.empty() ? 0 : gemm_x_floats(d.layers[0].w[0], n));  // cols = hidden
    // The Q|K|V stack, O and down projections may leave up to 4 unsummed
    // K-split slices in d.pscratch for the kernel after them to add (RoPE; the
    // fused norm: down_splits, o_splits > 1); other consumers get them summed
    // first
    const int64_t nh = int64_t(n) * hidden;
    int down_splits = 1;
    auto sum_splits = [&](int& splits, float* y) {
        if (splits > 1) launch_split_sum(d.pscratch, y, nh, splits, d.stream);
        splits = 1;
    };
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = d.layers[L];
        const bool fused = ly.has_qkv && gemm_supported(ly.qkv, n);
        const int qkv_x = fused ? xorder(ly.qkv)
                          : xorder(ly.w[1]) == xorder(ly.w[0]) && xorder(ly.w[2]) == xorder(ly.w[0]) ? xorder(ly.w[0])
                                                                                                       : -1;
        PrefillX cx;
        // h += the previous layer's down projection (in pn, or its split
        // slices), then the norm: into Q, K and V's fp16 operand where they
        // all read one, else f32
        if (qkv_x >= 0) {
            const float* a = L == 0 ? nullptr : down_splits > 1 ? d.pscratch : d.pn;
            if (const int e = launch_norm_x_f16r(d.ph, a, down_splits, nh, ly.attn_norm, nullptr, d.pxh, xscale, n,
                                                 hidden, c.rms_eps, qkv_x == 1, d.stream))
                return e;
            down_splits = 1;
            cx = PrefillX{d.pn, nullptr, hidden, qkv_x};
        } else if (L == 0) {
            hipLaunchKernelGGL(k_rmsnorm, dim3(unsigned(n)), dim3(1024), 0, d.stream, d.ph, ly.attn_norm, d.pn, hidden,
                               c.rms_eps);
        } else {
            sum_splits(down_splits, d.pn);
            hipLaunchKernelGGL(k_add_rmsnorm, dim3(unsigned(n)), dim3(1024), 0, d.stream, d.ph, d.pn, ly.attn_norm, d.pn,
                               hidden, c.rms_eps);
        }
        // Q, K and V: one GEMM on the decoder's Q|K|V stack (rows [n][q|k|v]) where
        // it carries the row factors, else three projections sharing one fp16
        // copy of the normed rows
        const int qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
        float *q = d.pq, *k = d.pk, *v = d.pv;
        int qstr = qd, kvstr = kvd, e = 0, qkv_splits = 1;
        if (fused) {
            e = prefill_proj(d, cx, ly.qkv, d.pn, nullptr, d.pq, n, d.pt, &qkv_splits);
            k = d.pq + qd;
            v = k + kvd;
            qstr = kvstr = qd + 2 * kvd;
        } else {
            e = prefill_proj(d, cx, ly.w[0], d.pn, nullptr, d.pq, n, d.pt);
            if (!e) e = prefill_proj(d, cx, ly.w[1], d.pn, nullptr, d.pk, n, d.pt);
            if (!e) e = prefill_proj(d, cx, ly.w[2], d.pn, nullptr, d.pv, n, d.pt);
        }
        if (e) return e;
        // up to 256 / n blocks per row, at most one per pass over the heads
        const int passes = (c.n_heads + c.n_kv_heads + 256 / (hd / 2) - 1) / (256 / (hd / 2));
        const dim3 rg(unsigned(n), unsigned(std::max(1, std::min(passes, 256 / n))));
        if (qkv_splits > 1)
            hipLaunchKernelGGL(k_rope_kv_rows<true>, rg, dim3(256), 0, d.stream, q, k, v, d.pscratch,
                               qkv_splits, int64_t(n) * qstr, ly.kc, ly.vc, d.freq_div, c.n_heads, c.n_kv_heads, hd,
                               c.max_seq, pos0, qstr, kvstr);
        else
            hipLaunchKernelGGL(k_rope_kv_rows<false>, rg, dim3(256), 0, d.stream, q, k, v, nullptr, 1,
                               int64_t(0), ly.kc, ly.vc, d.freq_div, c.n_heads, c.n_kv_heads, hd, c.max_seq, pos0, qstr,
                               kvstr);
        // bf16x3 products where Q, K and V came from the fp16 GEMM (the 2e-3 bar)
        const bool bf = fused || (gemm_supported(ly.w[0], n) && gemm_supported(ly.w[1], n) && gemm_supported(ly.w[2], n));
        int attn_ks = 1;
        if (!launch_attn_prefill_mf(d, ly, q, qstr, n, pos0, scale, bf, &attn_ks)) {
            const dim3 ag(unsigned(c.n_kv_heads), unsigned(n));
            if (hd == 128)
                hipLaunchKernelGGL(k_attn_prefill<128>, ag, dim3(256), 0, d.stream, q, ly.kc, ly.vc, d.patt,
                                   c.n_heads, c.n_kv_heads, c.max_seq, pos0, scale, qstr);
            else
                hipLaunchKernelGGL(k_attn_prefill<64>, ag, dim3(256), 0, d.stream, q, ly.kc, ly.vc, d.patt,
                                   c.n_heads, c.n_kv_heads, c.max_seq, pos0, scale, qstr);
        }
        cx = PrefillX{};
        if (attn_ks > 1) {
            // the key ranges merged straight into the O projection's fp16
            // operand where it runs on the GEMM, else into the f32 rows
            bool merged = false;
            if (gemm_supported(ly.w[3], n)) {
                const int fr = gemm_x_frag(ly.w[3], n) ? 1 : 0;
                merged = launch_merge_x_f16r(d.pscratch, attn_ks, c.n_heads, hd, n, fr != 0, d.pxh,
                                             d.pxh + gemm_x_floats(ly.w[3], n), d.stream) == 0;
                if (merged) cx = PrefillX{d.patt, nullptr, ly.w[3].cols, fr};
            }
            if (!merged) launch_attn_merge(d, n, attn_ks);
        }
        int o_splits = 1;
        e = prefill_proj(d, cx, ly.w[3], d.patt, nullptr, d.pt, n, nullptr, &o_splits);
        if (e) return e;
        // h += O att (in pt, or its split slices), then the norm (into gate
        // and up's fp16 operand where both read one)
        cx = PrefillX{};  // gate and up share one fp16 copy
        if (const int gu_x = xorder(ly.w[4]); gu_x >= 0 && xorder(ly.w[5]) == gu_x) {
            e = launch_norm_x_f16r(d.ph, o_splits > 1 ? d.pscratch : d.pt, o_splits, nh, ly.ffn_norm, nullptr, d.pxh,
                                   xscale, n, hidden, c.rms_eps, gu_x == 1, d.stream);
            if (e) return e;
            cx = PrefillX{d.pn, nullptr, hidden, gu_x};
        } else {
            sum_splits(o_splits, d.pt);
            hipLaunchKernelGGL(k_add_rmsnorm, dim3(unsigned(n)), dim3(1024), 0, d.stream, d.ph, d.pt, ly.ffn_norm, d.pn,
                               hidden, c.rms_eps);
        }
        e = prefill_proj(d, cx, ly.w[4], d.pn, nullptr, d.pg, n, d.pt);
        if (!e) e = prefill_proj(d, cx, ly.w[5], d.pn, nullptr, d.pu, n, d.pt);
        if (e) return e;
        cx = PrefillX{};
        // down(silu(gate) * up), added by the next norm
        e = prefill_proj(d, cx, ly.w[6], d.pg, d.pu, d.pn, n, d.pt, &down_splits);
        if (e) return e;
    }
    // the last layer's residual add, for the one row the LM head reads
    sum_splits(down_splits, d.pn);
    hipLaunchKernelGGL(k_add, dim3(unsigned((hidden + 255) / 256)), dim3(256), 0, d.stream,
                       d.ph + int64_t(n - 1) * hidden, d.pn + int64_t(n - 1) * hidden, hidden);
    const float* last = d.ph + int64_t(n - 1) * hidden;
    const float* fin = last;
    if (d.has_final_norm) {
        hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), 0, d.stream, last, d.final_norm, d.n, hidden, c.rms_eps);
        fin = d.n;
    }
    const int e = proj(d, d.lm, fin, d.logits, RPL_STORE, nullptr, nullptr);
    if (e) return e;
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, d.stream, d.logits, c.vocab, d.d_state, d.d_gen,
                       c.max_seq, 0);
    return int(hipGetLastError());
}

int run_steps(Decoder& d, int n_steps, int advance) {
    if (!d.use_graph) {
        for (int i = 0; i < n_steps; ++i) {
            const int e = enqueue_step(d, advance);
            if (e) return rt_hip_fail(hipError_t(e), "decoder step: launch");
        }
        return WV_OK;
    }
    if (!d.exec || d.graph_advance != advance) {
        drop_graph(d);
        hipError_t e = hipStreamBeginCapture(d.stream, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return rt_hip_fail(e, "decoder: begin capture");
        const int k = enqueue_step(d, advance);
        hipGraph_t g = nullptr;
        e = hipStreamEndCapture(d.stream, &g);
        if (k) {
            if (g) (void)hipGraphDestroy(g);
            return rt_hip_fail(hipError_t(k), "decoder: captured launch");
        }
        if (e != hipSuccess) return rt_hip_fail(e, "decoder: end capture");
        e = hipGraphInstantiate(&d.exec, g, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            (void)hipGraphDestroy(g);
            return rt_hip_fail(e, "decoder: instantiate");
        }
        d.graph = g;
        d.graph_advance = advance;
    }
    for (int i = 0; i < n_steps; ++i) {
        hipError_t e = hipGraphLaunch(d.exec, d.stream);
        if (e != hipSuccess) return rt_hip_fail(e, "decoder: graph launch");
    }
    return WV_OK;
}

}  // namespace
}  // namespace wv

using namespace wv;

extern "C" {

int wv_decoder_create(const wv_decoder_config* cfg, uint64_t* handle) {
    if (!cfg || !handle) return rt_fail(WV_E_ARG, "wv_decoder_create: nil argument");
    const wv_decoder_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.ffn <= 0 || c.vocab <= 0 ||
        c.max_seq <= 0)
        return rt_fail(WV_E_SHAPE, "wv_decoder_create: non-positive dimension");
    if (c.head_dim != 64 && c.head_dim != 128) return rt_fail(WV_E_SHAPE, "wv_decoder_create: head_dim %d (64 or 128)", c.head_dim);
    if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 8)
        return rt_fail(WV_E_SHAPE, "wv_decoder_create: %d heads over %d KV heads", c.n_heads, c.n_kv_heads);
    if (c.rope_theta <= 0 || c.rms_eps <= 0) return rt_fail(WV_E_ARG, "wv_decoder_create: rope_theta and rms_eps must be > 0");
    if (c.hidden % 4 || c.hidden > 16384) return rt_fail(WV_E_SHAPE, "wv_decoder_create: hidden %d (a multiple of 4, <= 16384)", c.hidden);
    if (c.max_seq > kChunk * 2048) return rt_fail(WV_E_SHAPE, "wv_decoder_create: max_seq %d > %d", c.max_seq, kChunk * 2048);
    int rc = rt_ensure_init();
    if (rc) return rc;
    Decoder* d = new Decoder();
    d->c = c;
    d->device = rt_current_device();
    d->layers.resize(size_t(c.n_layers));
    d->n_chunks = (c.max_seq + kChunk - 1) / kChunk;
    hipError_t e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete d;
        return rt_hip_fail(e, "wv_decoder_create: stream");
    }
    const size_t kv_dim = size_t(c.n_kv_heads) * c.head_dim, q_dim = size_t(c.n_heads) * c.head_dim;
    const size_t wide = std::max({size_t(c.hidden), q_dim, size_t(c.ffn), size_t(c.vocab)});
    struct B { float** p; size_t n; };
    B bufs[] = {{&d->h, size_t(c.hidden)}, {&d->n, size_t(c.hidden)}, {&d->q, q_dim + 2 * kv_dim},
                {&d->ss_a, size_t(c.hidden / 16 + 1)}, {&d->ss_b, size_t(c.hidden / 16 + 1)},
                {&d->att, q_dim}, {&d->g, size_t(c.ffn)}, {&d->u, size_t(c.ffn)}, {&d->logits, wide},
                {&d->part, size_t(c.n_heads) * d->n_chunks * (c.head_dim + 2)}};
    for (B& b : bufs) {
        rc = dalloc(*d, reinterpret_cast<void**>(b.p), b.n * sizeof(float), "wv_decoder_create: buffers");
        if (rc) {
            release(d);
            return rc;
        }
    }
    d->k = d->q + q_dim;  // q | k | v contiguous, as the fused QKV projection writes them
    d->v = d->k + kv_dim;
    void* ints = nullptr;
    rc = dalloc(*d, &ints, (4 + size_t(c.max_seq)) * sizeof(int32_t), "wv_decoder_create: state");
    if (rc) {
        release(d);
        return rc;
    }
    void* tabs = nullptr;
    rc = dalloc(*d, &tabs, size_t(c.head_dim / 2) * (sizeof(double) + sizeof(double2)), "wv_decoder_create: RoPE table");
    if (rc) {
        release(d);
        return rc;
    }
    d->cs = static_cast<double2*>(tabs);
    d->freq_div = reinterpret_cast<double*>(d->cs + c.head_dim / 2);
    {
        std::vector<double> fd(size_t(c.head_dim / 2));
        for (int i = 0; i < c.head_dim / 2; ++i) fd[size_t(i)] = std::pow(c.rope_theta, double(2 * i) / double(c.head_dim));
        e = hipMemcpy(d->freq_div, fd.data(), fd.size() * sizeof(double), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            release(d);
            return rt_hip_fail(e, "wv_decoder_create: RoPE table");
        }
    }
    d->d_state = static_cast<int32_t*>(ints);
    d->d_pos = d->d_state;
    d->d_tok = d->d_state + 1;
    d->d_gen = d->d_state + 4;
    for (int L = 0; L < c.n_layers; ++L) {
        Layer& ly = d->layers[L];
        const size_t cache = size_t(c.max_seq) * kv_dim * sizeof(float);
        rc = dalloc(*d, reinterpret_cast<void**>(&ly.kc), cache, "wv_decoder_create: K cache");
        if (!rc) rc = dalloc(*d, reinterpret_cast<void**>(&ly.vc), cache, "wv_decoder_create: V cache");
        if (!rc) rc = dalloc(*d, reinterpret_cast<void**>(&ly.attn_norm), size_t(c.hidden) * 4, "wv_decoder_create: norms");
        if (!rc) rc = dalloc(*d, reinterpret_cast<void**>(&ly.ffn_norm), size_t(c.hidden) * 4, "wv_decoder_create: norms");
        if (!rc) {
            e = hipMemsetAsync(ly.kc, 0, cache, d->stream);
            if (e == hipSuccess) e = hipMemsetAsync(ly.vc, 0, cache, d->stream);
            if (e != hipSuccess) rc = rt_hip_fail(e, "wv_decoder_create: clear cache");
        }
        if (rc) {
            release(d);
            return rc;
        }
    }
    e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) {
        release(d);
        return rt_hip_fail(e, "wv_decoder_create: sync");
    }
    std::lock_guard<std::mutex> lk(g_dmu);
    *handle = g_dnext++;
    g_decs[*handle] = d;
    return WV_OK;
}

int wv_decoder_set_layer(uint64_t dec, int32_t layer, const uint64_t* blobs, const float* attn_norm,
                         const float* ffn_norm) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_set_layer: unknown decoder %llu", (unsigned long long)dec);
    if (!blobs || !attn_norm || !ffn_norm) return rt_fail(WV_E_ARG, "wv_decoder_set_layer: nil argument");
    const wv_decoder_config& c = d->c;
    if (layer < 0 || layer >= c.n_layers) return rt_fail(WV_E_ARG, "wv_decoder_set_layer: layer %d of %d", layer, c.n_layers);
    const int64_t q_dim = int64_t(c.n_heads) * c.head_dim, kv_dim = int64_t(c.n_kv_heads) * c.head_dim;
    const int64_t want[7][2] = {{q_dim, c.hidden}, {kv_dim, c.hidden}, {kv_dim, c.hidden}, {c.hidden, q_dim},
                                {c.ffn, c.hidden}, {c.ffn, c.hidden}, {c.hidden, c.ffn}};
    static const char* names[7] = {"Q", "K", "V", "O", "gate", "up", "down"};
    Layer& ly = d->layers[layer];
    DevBlob nw[7];
    for (int i = 0; i < 7; ++i) {
        DevBlob b;
        if (!rt_lookup(blobs[i], b)) return rt_fail(WV_E_HANDLE, "wv_decoder_set_layer: %s blob %llu unknown", names[i], (unsigned long long)blobs[i]);
        if (b.rows != want[i][0] || b.cols != want[i][1])
            return rt_fail(WV_E_SHAPE, "wv_decoder_set_layer: %s is %lldx%lld, want %lldx%lld", names[i], (long long)b.rows,
                           (long long)b.cols, (long long)want[i][0], (long long)want[i][1]);
        nw[i] = b;
    }
    (void)hipSetDevice(d->device);
    // A captured step reads this layer's old weights and fused copies: drop
    // it, and keep the layer unusable until every part below succeeded.
    drop_graph(*d);
    ly.set = false;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e == hipSuccess) e = hipMemcpy(ly.attn_norm, attn_norm, size_t(c.hidden) * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(ly.ffn_norm, ffn_norm, size_t(c.hidden) * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_set_layer: norms");
    drop_fused(ly);
    for (int i = 0; i < 7; ++i) ly.w[i] = nw[i];
    const DevBlob* w = ly.w;
    auto rpl_same = [&](int i, int j) {
        return w[i].layout == LAYOUT_RPL && w[j].layout == LAYOUT_RPL && w[i].fmt == w[j].fmt;
    };
    if (rpl_same(0, 1) && rpl_same(0, 2) && w[0].rows % 64 == 0 && w[1].rows % 64 == 0) {
        const int k = rpl_fuse_rows(w, 3, ly.qkv, d->stream);
        if (k != hipSuccess) return rt_hip_fail(hipError_t(k), "wv_decoder_set_layer: fuse Q|K|V");
        ly.has_qkv = true;
    }
    if (rpl_same(4, 5) && w[4].rows % 32 == 0) {
        const int k = rpl_fuse_pairs(w[4], w[5], ly.gu, d->stream);
        if (k != hipSuccess) return rt_hip_fail(hipError_t(k), "wv_decoder_set_layer: fuse gate/up");
        ly.has_gu = true;
    }
    ly.set = true;
    return WV_OK;
}

int wv_decoder_set_output(uint64_t dec, uint64_t lm_head, const float* final_norm, const float* embedding) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_set_output: unknown decoder %llu", (unsigned long long)dec);
    if (!embedding) return rt_fail(WV_E_ARG, "wv_decoder_set_output: nil embedding table");
    const wv_decoder_config& c = d->c;
    DevBlob b;
    if (!rt_lookup(lm_head, b)) return rt_fail(WV_E_HANDLE, "wv_decoder_set_output: LM head blob unknown");
    if (b.rows != c.vocab || b.cols != c.hidden)
        return rt_fail(WV_E_SHAPE, "wv_decoder_set_output: LM head is %lldx%lld, want %dx%d", (long long)b.rows,
                       (long long)b.cols, c.vocab, c.hidden);
    (void)hipSetDevice(d->device);
    // A captured step holds the old head, norm and table: capture again, and
    // keep the output unusable until the copies below succeeded.
    drop_graph(*d);
    d->lm_set = false;
    int rc = WV_OK;
    if (final_norm && !d->final_norm) rc = dalloc(*d, reinterpret_cast<void**>(&d->final_norm), size_t(c.hidden) * 4, "final norm");
    if (!rc && !d->embed) rc = dalloc(*d, reinterpret_cast<void**>(&d->embed), size_t(c.vocab) * c.hidden * 4, "embedding");
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize(d->stream);
    if (e == hipSuccess && final_norm) e = hipMemcpy(d->final_norm, final_norm, size_t(c.hidden) * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(d->embed, embedding, size_t(c.vocab) * c.hidden * 4, hipMemcpyHostToDevice);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_set_output: copy");
    d->has_final_norm = final_norm != nullptr;  // NULL: no final norm (forward.go:80-86)
    d->lm = b;
    d->lm_set = true;
    return WV_OK;
}

int wv_decoder_set_kv(uint64_t dec, int32_t layer, int32_t first_pos, int32_t n_pos, const float* k, const float* v) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_set_kv: unknown decoder %llu", (unsigned long long)dec);
    const wv_decoder_config& c = d->c;
    if (layer < 0 || layer >= c.n_layers || !k || !v) return rt_fail(WV_E_ARG, "wv_decoder_set_kv: bad layer or nil rows");
    if (first_pos < 0 || n_pos < 0 || int64_t(first_pos) + n_pos > c.max_seq)
        return rt_fail(WV_E_SHAPE, "wv_decoder_set_kv: rows %d..%d outside max_seq %d", first_pos, first_pos + n_pos, c.max_seq);
    const size_t hd = size_t(c.head_dim), kv_dim = size_t(c.n_kv_heads) * hd;
    (void)hipSetDevice(d->device);
    hipError_t e = hipSuccess;
    // host rows [pos][kv head][hd] -> device head-major [kv head][max_seq][hd]
    for (int kh = 0; kh < c.n_kv_heads && e == hipSuccess && n_pos > 0; ++kh) {
        const size_t dst = (size_t(kh) * c.max_seq + size_t(first_pos)) * hd;
        e = hipMemcpy2D(d->layers[layer].kc + dst, hd * 4, k + kh * hd, kv_dim * 4, hd * 4, size_t(n_pos),
                        hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy2D(d->layers[layer].vc + dst, hd * 4, v + kh * hd, kv_dim * 4, hd * 4, size_t(n_pos),
                            hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_set_kv: copy");
    return WV_OK;
}

int wv_decoder_use_graph(uint64_t dec, int32_t enable) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_use_graph: unknown decoder %llu", (unsigned long long)dec);
    d->use_graph = enable != 0;
    return WV_OK;
}

int wv_decoder_generate(uint64_t dec, int32_t token, int32_t pos, int32_t n_steps, int32_t advance_pos,
                        int32_t* tokens_out, float* last_logits) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_generate: unknown decoder %llu", (unsigned long long)dec);
    const wv_decoder_config& c = d->c;
    if (n_steps < 0 || n_steps > c.max_seq) return rt_fail(WV_E_ARG, "wv_decoder_generate: step count %d outside 0..max_seq", n_steps);
    if (pos < 0 || int64_t(pos) + (advance_pos ? n_steps : 1) > c.max_seq)
        return rt_fail(WV_E_SHAPE, "wv_decoder_generate: positions %d.. exceed max_seq %d", pos, c.max_seq);
    int rc = ready(*d);
    if (rc) return rc;
    (void)hipSetDevice(d->device);
    const int32_t init[4] = {pos, token, -1, 0};
    hipError_t e = hipMemcpyAsync(d->d_state, init, sizeof init, hipMemcpyHostToDevice, d->stream);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_generate: state");
    rc = run_steps(*d, n_steps, advance_pos ? 1 : 0);
    if (rc) return rc;
    if (tokens_out && n_steps > 0) {
        e = hipMemcpyAsync(tokens_out, d->d_gen, size_t(n_steps) * sizeof(int32_t), hipMemcpyDeviceToHost, d->stream);
        if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_generate: tokens");
    }
    if (last_logits && n_steps > 0) {
        e = hipMemcpyAsync(last_logits, d->logits, size_t(c.vocab) * 4, hipMemcpyDeviceToHost, d->stream);
        if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_generate: logits");
    }
    e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_generate: sync");
    return WV_OK;
}

int wv_decoder_prefill(uint64_t dec, const int32_t* tokens, int32_t n_tokens, int32_t pos0, int32_t* next_token,
                       float* last_logits) {
    Decoder* d = find(dec);
    if (!d) return rt_fail(WV_E_HANDLE, "wv_decoder_prefill: unknown decoder %llu", (unsigned long long)dec);
    const wv_decoder_config& c = d->c;
    if (!tokens || n_tokens <= 0) return rt_fail(WV_E_ARG, "wv_decoder_prefill: empty ids");  // forward.go:35-37
    if (pos0 < 0 || int64_t(pos0) + n_tokens > c.max_seq)
        return rt_fail(WV_E_SHAPE, "wv_decoder_prefill: seq %d at position %d > MaxSeqLen %d", n_tokens, pos0, c.max_seq);
    int rc = ready(*d);
    if (rc) return rc;
    (void)hipSetDevice(d->device);
    rc = ensure_prefill(*d, n_tokens);
    if (rc) return rc;
    hipError_t e = hipMemcpyAsync(d->ptok, tokens, size_t(n_tokens) * 4, hipMemcpyHostToDevice, d->stream);
    const int32_t init[4] = {pos0 + n_tokens - 1, 0, -1, 0};
    if (e == hipSuccess) e = hipMemcpyAsync(d->d_state, init, sizeof init, hipMemcpyHostToDevice, d->stream);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_prefill: tokens");
    const int k = enqueue_prefill(*d, n_tokens, pos0);
    if (k) return rt_hip_fail(hipError_t(k), "wv_decoder_prefill: launch");
    int32_t st[4] = {0, 0, 0, 0};
    e = hipMemcpyAsync(st, d->d_state, sizeof st, hipMemcpyDeviceToHost, d->stream);
    if (e == hipSuccess && last_logits)
        e = hipMemcpyAsync(last_logits, d->logits, size_t(c.vocab) * 4, hipMemcpyDeviceToHost, d->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(d->stream);
    if (e != hipSuccess) return rt_hip_fail(e, "wv_decoder_prefill: results");
    if (next_token) *next_token = st[2];
    return WV_OK;
}

int wv_decoder_free(uint64_t dec) {
    Decoder* d = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_dmu);
        auto it = g_decs.find(dec);
        if (it == g_decs.end()) return rt_fail(WV_E_HANDLE, "wv_decoder_free: unknown decoder %llu", (unsigned long long)dec);
        d = it->second;
        g_decs.erase(it);
    }
    (void)hipSetDevice(d->device);
    (void)hipStreamSynchronize(d->stream);
    release(d);
    return WV_OK;
}

}  // extern "C"
