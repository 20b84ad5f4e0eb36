// wv_internal.h — shared declarations of the gfx950 Dense MatVec library.
#pragma once

#include <cstddef>
#include <cstdint>

namespace wv {

// quant.Format values (quant/format.go:9-39).
enum Fmt : int {
    FMT_NONE = 0, FMT_Q8_0 = 1, FMT_Q4_0 = 2, FMT_Q4_1 = 3, FMT_Q5_0 = 4, FMT_Q5_1 = 5,
    FMT_Q2_K = 6, FMT_Q3_K = 7, FMT_Q4_K = 8, FMT_Q5_K = 9, FMT_Q6_K = 10,
    FMT_IQ1_S = 11, FMT_IQ2_XXS = 12, FMT_IQ2_XS = 13, FMT_IQ3_XXS = 14, FMT_IQ3_S = 15,
    FMT_IQ4_NL = 16, FMT_IQ4_XS = 17, FMT_TERNARY = 18, FMT_BINARY = 19, FMT_AFFINE = 20,
    FMT_NATIVE_TERNARY = 1019,  // FormatNone + core.DTypeTernary (core/dtype.go:31)
};

// k-quant super-block spec (quant/kquant.go:29-51).
struct KSpec {
    int bits = 0;
    bool has_dmin = false;
    int qmax = 0;
    int mid = 0;
};
inline bool k_spec(int fmt, KSpec& s) {
    switch (fmt) {
    case FMT_Q2_K: s = {2, true, 3, 0}; return true;
    case FMT_Q3_K: s = {3, true, 7, 0}; return true;
    case FMT_Q4_K: s = {4, true, 15, 0}; return true;
    case FMT_Q5_K: s = {5, true, 31, 0}; return true;
    case FMT_Q6_K: s = {6, false, 63, 32}; return true;
    default: return false;
    }
}
// kSuperBytes (quant/kquant.go:53-60): d, dmin, 16 scale bytes, [16 min bytes], codes.
inline int64_t k_super_bytes(const KSpec& s) { return 8 + 16 + (s.has_dmin ? 16 : 0) + (256 * s.bits + 7) / 8; }

// IQ spec (quant/iq.go:42-68).
struct IQSpec {
    int bits = 0;
    int sg = 0;  // weights sharing one scale
    bool nonlinear = false;
    float mid = 0;
};
inline bool iq_spec(int fmt, IQSpec& s) {
    switch (fmt) {
    case FMT_IQ1_S: s = {1, 32, false, 0.5f}; return true;
    case FMT_IQ2_XXS: s = {2, 32, false, 1.5f}; return true;
    case FMT_IQ2_XS: s = {2, 16, false, 1.5f}; return true;
    case FMT_IQ3_XXS: s = {3, 32, false, 3.5f}; return true;
    case FMT_IQ3_S: s = {3, 16, false, 3.5f}; return true;
    case FMT_IQ4_NL: s = {4, 32, true, 0.0f}; return true;
    case FMT_IQ4_XS: s = {4, 16, false, 7.5f}; return true;
    default: return false;
    }
}

// IQ4_NL grid: a data table whose values must equal quant/iq.go:23-40.
constexpr float kIQ4NLGrid[16] = {
    -1.0f, -0.6961928f, -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f,
    -0.091050036f, 0.0f, 0.0795803f, 0.1609302f, 0.2461123f, 0.33791524f,
    0.44070983f, 0.562617f, 0.72295684f, 1.0f};

struct PackSizes {
    int64_t raw = 0, scales = 0, mins = 0, meta = 0;
    int32_t block_weights = 0;
};
bool pack_sizes(int fmt, int64_t rows, int64_t cols, PackSizes& out);
bool pack(int fmt, const float* w, int64_t rows, int64_t cols, uint8_t* raw, float* scales, uint8_t* meta);
void pack_native_ternary(const float* w, int64_t n, uint8_t* codes, float* scale);

// ---- device residency ----

// How a blob sits in HBM.
enum Layout : int {
    LAYOUT_RAW = 0,      // uploaded bytes verbatim; decoded per element (any shape / format)
    LAYOUT_K_PLANAR = 1, // k-quants, cols % 256 == 0: codes plane + (d,dmin) plane + scale/min plane
    LAYOUT_Q8_PLANAR = 2,// Q8_0, cols % 32 == 0: int8 codes plane + f32 scale plane
    LAYOUT_Q4_PLANAR = 3,// Q4_0, cols % 32 == 0: nibble plane + f32 scale plane
    LAYOUT_TERNARY_I8 = 4,// DTypeTernary, cols % 64 == 0: 2-bit codes rows (as uploaded)
};

// Device view of one blob. Pointers are into one hipMalloc'd allocation.
struct DevBlob {
    int fmt = 0;
    int64_t rows = 0, cols = 0;
    int32_t block_weights = 0;
    float tensor_scale = 1.0f;
    int layout = LAYOUT_RAW;
    int device = 0;
    // LAYOUT_RAW
    const uint8_t* raw = nullptr;
    int64_t raw_len = 0;
    const float* scales = nullptr;
    int64_t n_scales = 0;
    int iq_bits = 0, iq_sg = 0;  // Meta[0], Meta[1] for IQ (iq.go:187-190)
    // planar layouts
    const uint8_t* codes = nullptr;   // row-major code plane
    const uint8_t* codes_hi = nullptr;// Q6_K high-2-bit plane
    const float* blk_scale = nullptr; // Q8_0/Q4_0 per-block f32 scales; k-quants (d,dmin) pairs
    const uint32_t* grp = nullptr;    // k-quants: per 32-column chunk (u0,u1,m0,m1) bytes
    void* base = nullptr;             // allocation owner
    size_t device_bytes = 0;
};

// Kernel launchers (gemv.hip). Return a hipError_t as int.
int launch_matvec(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream);
int launch_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch);
size_t matvec_t_scratch_floats(const DevBlob& b, int batch);
int launch_ternary_acc(const DevBlob& b, const float* d_x, int32_t* d_acc, float* d_act_scale, int batch, void* stream);

}  // namespace wv
