// wave_ops.h — cross-lane reductions of a 64-lane wavefront on DPP.
//
// A ds_bpermute butterfly (what __shfl_xor compiles to) costs one LDS round
// trip per step; these reductions run on the VALU instead: row_shr 1, 2, 4, 8
// leaves each 16-lane row's total in its lane 15, row_bcast 15 and 31 carry
// the row totals up, and lane 63 ends with the wave's total, which readlane
// returns to every lane as a uniform value. Every lane of the wave must be
// active. Sums associate differently from a butterfly (f32 results may differ
// in the last bits; integer results are identical).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace wv {

// DPP controls (GFX9 encoding).
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

// A 16-byte load with the non-temporal hint, for data read once per launch
// (weights, the KV cache): on MI355X it streams 38.5 MB in 6.8 us against
// 7.2 us for a plain load.
__device__ __forceinline__ uint4 ld_nt16(const uint4* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 ld_nt16(const float4* p) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Value of `v` from another lane per the DPP control; lanes without a source
// (outside the row, or masked off) get `fill`.
template <int Ctrl, int RowMask = 0xf, int BankMask = 0xf>
__device__ __forceinline__ int dpp_i(int fill, int v) {
    return __builtin_amdgcn_update_dpp(fill, v, Ctrl, RowMask, BankMask, false);
}

__device__ __forceinline__ int wave_total_i(int v) {
    v += dpp_i<kDppRowShr1>(0, v);
    v += dpp_i<kDppRowShr2>(0, v);
    v += dpp_i<kDppRowShr4, 0xf, 0xe>(0, v);
    v += dpp_i<kDppRowShr8, 0xf, 0xc>(0, v);
    v += dpp_i<kDppRowBcast15, 0xa>(0, v);
    v += dpp_i<kDppRowBcast31, 0xc>(0, v);
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ float wave_total(float f) {
    int v = __float_as_int(f);
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowShr1>(0, v)));
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowShr2>(0, v)));
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowShr4, 0xf, 0xe>(0, v)));
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowShr8, 0xf, 0xc>(0, v)));
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowBcast15, 0xa>(0, v)));
    v = __float_as_int(__int_as_float(v) + __int_as_float(dpp_i<kDppRowBcast31, 0xc>(0, v)));
    return __int_as_float(__builtin_amdgcn_readlane(v, 63));
}

// Maximum over the wave (lanes without a source compare against themselves).
__device__ __forceinline__ float wave_maximum(float f) {
    int v = __float_as_int(f);
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowShr1>(v, v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowShr2>(v, v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowShr4, 0xf, 0xe>(v, v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowShr8, 0xf, 0xc>(v, v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowBcast15, 0xa>(v, v))));
    v = __float_as_int(fmaxf(__int_as_float(v), __int_as_float(dpp_i<kDppRowBcast31, 0xc>(v, v))));
    return __int_as_float(__builtin_amdgcn_readlane(v, 63));
}

// Exchanges inside a quad of lanes (quad_perm): the value of lane ^ 1 / lane ^ 2.
__device__ __forceinline__ float quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
}
// The value of lane 7 - (lane & 7) of the same 8-lane half row (row_half_mirror):
// after a quad reduction, the other quad's result.
__device__ __forceinline__ float half_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));
}

// Sum over each 16-lane row into every lane of the row, by row_ror 8, 4, 2, 1:
// rotating 16 lanes by 8 is lane ^ 8, and each later rotation adds the same
// pairs as the xor butterfly (the partial sums are periodic by then), so the
// result equals a __shfl_xor(8, 4, 2, 1) butterfly bit for bit.
__device__ __forceinline__ float row_sum16(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x122, 0xf, 0xf, false));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x121, 0xf, 0xf, false));
    return v;
}

// f64 total over the wave on the same DPP tree (both 32-bit halves move together).
template <int Ctrl, int RowMask = 0xf, int BankMask = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
    const uint32_t lo = uint32_t(dpp_i<Ctrl, RowMask, BankMask>(0, int(uint32_t(b))));
    const uint32_t hi = uint32_t(dpp_i<Ctrl, RowMask, BankMask>(0, int(uint32_t(b >> 32))));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}
__device__ __forceinline__ double wave_total_f64(double v) {
    v += dpp_f64<kDppRowShr1>(v);
    v += dpp_f64<kDppRowShr2>(v);
    v += dpp_f64<kDppRowShr4, 0xf, 0xe>(v);
    v += dpp_f64<kDppRowShr8, 0xf, 0xc>(v);
    v += dpp_f64<kDppRowBcast15, 0xa>(v);
    v += dpp_f64<kDppRowBcast31, 0xc>(v);
    const unsigned long long b = static_cast<unsigned long long>(__double_as_longlong(v));
    const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b)), 63));
    const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(b >> 32)), 63));
    return __longlong_as_double(static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo));
}

// One reduce-scatter step over the lane pairs (l, l ^ 32): lanes below 32
// return a(l) + a(l + 32), lanes from 32 return b(l - 32) + b(l). gfx950's
// v_permlane32_swap exchanges a's upper 32 lanes with b's lower 32, so the
// two results hold, in every lane, its own kept value and its partner's.
__device__ __forceinline__ float reduce_scatter32(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The same over the pairs (l, l ^ 16) with v_permlane16_swap (odd 16-lane
// rows of a exchanged with even rows of b): lanes with bit 4 clear return
// a(l) + a(l + 16), the others b(l - 16) + b(l).
__device__ __forceinline__ float reduce_scatter16(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// The value of lane l ^ 8 (row_ror 8 inside each 16-lane row).
__device__ __forceinline__ float row_xor8(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));
}

// Quad transpose of bytes: lane q of each group of four holds P_q; returns to
// lane q the dword whose byte j is byte q of P_j (quad_perm rotations).
__device__ __forceinline__ uint32_t quad_byte_transpose(uint32_t p, int q) {
    const uint32_t r1 = uint32_t(__builtin_amdgcn_mov_dpp(int(p), 0x39, 0xf, 0xf, false));  // P_{(q+1)&3}
    const uint32_t r2 = uint32_t(__builtin_amdgcn_mov_dpp(int(p), 0x4e, 0xf, 0xf, false));  // P_{(q+2)&3}
    const uint32_t r3 = uint32_t(__builtin_amdgcn_mov_dpp(int(p), 0x93, 0xf, 0xf, false));  // P_{(q+3)&3}
    const int sh = 8 * q;
    uint32_t d = ((p >> sh) & 0xffu) << sh;
    d |= ((r1 >> sh) & 0xffu) << (8 * ((q + 1) & 3));
    d |= ((r2 >> sh) & 0xffu) << (8 * ((q + 2) & 3));
    d |= ((r3 >> sh) & 0xffu) << (8 * ((q + 3) & 3));
    return d;
}

}  // namespace wv
