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
