// wv_internal.h — shared declarations of the gfx950 Dense MatVec library.
#pragma once

#include <cstddef>
#include <cstdint>

namespace wv {

struct float2_t {
    float x, y;
};

// quant.Format values (quant/format.go:9-39).
enum Fmt : int {
    FMT_NONE = 0, FMT_Q8_0 = 1, FMT_Q4_0 = 2, FMT_Q4_1 = 3, FMT_Q5_0 = 4, FMT_Q5_1 = 5,
    FMT_Q2_K = 6, FMT_Q3_K = 7, FMT_Q4_K = 8, FMT_Q5_K = 9, FMT_Q6_K = 10,
    FMT_IQ1_S = 11, FMT_IQ2_XXS = 12, FMT_IQ2_XS = 13, FMT_IQ3_XXS = 14, FMT_IQ3_S = 15,
    FMT_IQ4_NL = 16, FMT_IQ4_XS = 17, FMT_TERNARY = 18, FMT_BINARY = 19, FMT_AFFINE = 20,
    // FormatNone weights.Store payloads: WV_NATIVE_BASE + core.DType (core/dtype.go:11-52)
    FMT_NATIVE_BASE = 1000,
    FMT_NATIVE_INT8 = 1009, FMT_NATIVE_INT4 = 1014, FMT_NATIVE_INT2 = 1017, FMT_NATIVE_TERNARY = 1019,
    FMT_NATIVE_BINARY = 1020,
};
// The narrow weights.Store DTypes that run Dense's int8 path
// (forwardSIMDNarrowI8 / forwardSIMDInt8, layers/dense/simd.go:130-195, 303-326):
// code bits per weight, or 0.
inline int narrow_bits(int fmt) {
    switch (fmt) {
    case FMT_NATIVE_INT8: return 8;
    case FMT_NATIVE_INT4: return 4;
    case FMT_NATIVE_INT2: case FMT_NATIVE_TERNARY: return 2;
    case FMT_NATIVE_BINARY: return 1;
    default: return 0;
    }
}

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

// An IQ blob goes to the row-interleaved layout when it is linear and keeps its
// format's default code width and scale group (the kernels are built for those).
inline bool iq_rpl_spec(int fmt, int bits, int sg) {
    IQSpec s;
    return iq_spec(fmt, s) && !s.nonlinear && bits == s.bits && sg == s.sg;
}
// Formats whose codes form one matrix-wide LSB-first stream of `bits`-bit
// codes with one f32 scale per `sg` weights: the linear IQ formats,
// TernaryPacked (2 bits, 16 weights; code 3 reads as 1) and BinaryPacked with
// 32- or 128-weight groups (1 bit). Missing Ternary / Binary scales read as 1.
// IQ4_NL (4-bit codes into a float grid, one scale per 32) takes the same
// planes as IQ4_XS's codes with 8 scales per super-block; its kernels look
// the grid up per weight.
struct LinCodes {
    int bits = 0, sg = 0;
    bool remap3 = false;
};
inline bool rpl_lin_spec(int fmt, int block_weights, int iq_bits, int iq_sg, LinCodes& lc) {
    if (iq_rpl_spec(fmt, iq_bits, iq_sg)) {
        lc = {iq_bits, iq_sg, false};
        return true;
    }
    if (fmt == FMT_IQ4_NL && iq_bits == 4 && iq_sg == 32) {
        lc = {4, 32, false};
        return true;
    }
    if (fmt == FMT_TERNARY) {
        lc = {2, 16, true};
        return true;
    }
    if (fmt == FMT_BINARY) {
        lc = {1, block_weights == 128 ? 128 : 32, false};
        return true;
    }
    return false;
}
// AffinePacked group widths the row-interleaved layout takes: groups that
// tile a 256-column super-block (one scale and min per 2^GSH chunks).
inline bool rpl_affine_group(int block_weights) {
    return block_weights == 32 || block_weights == 64 || block_weights == 128 || block_weights == 256;
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
bool pack(int fmt, const float* w, int64_t rows, int64_t cols, uint8_t* raw, float* scales, float* mins,
          uint8_t* meta);
bool pack_native(int fmt, const float* w, int64_t n, uint8_t* codes, float* scale);

// ---- device residency ----

// How a blob sits in HBM.
enum Layout : int {
    LAYOUT_RAW = 0,        // uploaded bytes verbatim; decoded per element (any shape / format)
    LAYOUT_RPL = 1,        // Q4_K/Q6_K/Q8_0/Q4_0 with cols % 256 == 0: row-interleaved planes (gemv_rpl.hip)
    LAYOUT_NARROW = 4,     // weights.Store Int8/Int4/Int2/Ternary/Binary codes, bits permuted per word
                           // (narrow_permute_words, runtime.hip) + Store.Scale
    LAYOUT_F32 = 5,        // FormatNone f32 weights, row-major (quant/none.go, Store FormatNone+Float32)
};

// Device view of a row-interleaved blob. Rows are grouped 64 at a time (one
// wave's lanes); chunk = 32 columns, super-block (sb) = 256 columns.
//   codes [rg][sb][j][lane][CB] (Q4_K) or [j][rg][sb][lane][CB] (the other
//         formats); CB = 8 / 16 / 32 B per lane and chunk; j = chunk in sb
//   hi    high code bits in the codes' order (Q6_K 8 B, Q5_x / Q3_K 4 B)
//   meta  [rg][sb][lane][MB]      MB = 32 B (Q4_K scale/min bytes, Q8_0/Q4_0
//                                  f32 block scales) or 16 B (Q6_K scales)
//   dd    [rg][sb][lane] (d, dmin) f32 pair (k-quants)
//   wrow  [rg*64] f32 power-of-two row factors of the prefill GEMM
// Chunk j of super-block slot si = row group * nsb + super-block sits at chunk
// index si * cs_si + j * cs_j (times 64 lanes). Q4_K keeps a super-block's 8
// chunks of one row group adjacent (cs_si = 8, cs_j = 1: the owning wave
// streams one 8 KiB run); the other formats keep them chunk-step-major
// (cs_si = 1, cs_j = row groups * nsb: every wave reads the same chunk step
// together), which measured faster for their wider chunks.
inline bool rpl_sb_major(int fmt) { return fmt == FMT_Q4_K; }
inline void rpl_strides(int fmt, int64_t rg, int64_t nsb, int64_t& cs_si, int64_t& cs_j) {
    cs_si = rpl_sb_major(fmt) ? 8 : 1;
    cs_j = rpl_sb_major(fmt) ? 1 : rg * nsb;
}

struct RplArgs {
    const uint8_t* codes;
    const uint8_t* hi;
    const uint8_t* meta;
    const float2_t* dd;
    // [rg*64] power-of-two row factors of the prefill GEMM (gemm_row_factor);
    // null on the fused images, which only the GEMV kernels read.
    const float* wrow;
    // K-split partial sums [batch chunk][ksplit][rg*64], in scratch the caller
    // of the launch provides (never stored with the blob: two launches on one
    // blob may run at once).
    float* partial;
    int rows, nsb, rg_count, ksplit;
    int64_t cs_si, cs_j;  // chunk strides of the code planes (rpl_chunk)
    // Output epilogue of the forward kernel: RPL_STORE y = Wx;
    // RPL_ADD y += Wx (residual); RPL_SILU_MUL y = silu(aux) * Wx (SwiGLU up);
    // RPL_SWIGLU on a gate/up row-pair blob (row 2i gate i, row 2i+1 up i):
    // y[i] = silu(gate_i) * up_i, y holding rows/2 values per batch row.
    int mode;
    const float* aux;  // [batch][rows] gate values for RPL_SILU_MUL
    // Fused RMSNorm of x (nrm_gamma != nullptr): x is scaled by
    // inv * gamma, inv = 1/sqrt(sum(x^2)/cols + eps), with sum(x^2) given as
    // nrm_n partial sums per batch row in nrm_ss (written by the producer).
    const float* nrm_gamma;
    const float* nrm_ss;
    int nrm_n;
    double nrm_eps;
    // With RPL_ADD: sums of the updated y^2 over each 16 rows
    // ([batch][rg*4]), the partials the next fused RMSNorm consumes.
    float* ss_out;
};// Chunk index (in lane items / 64) of chunk j of super-block slot si.
constexpr int64_t rpl_chunk(const RplArgs& a, int64_t si, int j) { return si * a.cs_si + j * a.cs_j; }


// Options of one forward launch on the row-interleaved layout.
struct RplExtra {
    int mode = 0;
    const float* aux = nullptr;
    const float* nrm_gamma = nullptr;
    const float* nrm_ss = nullptr;
    int nrm_n = 0;
    double nrm_eps = 0.0;
    float* ss_out = nullptr;
    float* partial = nullptr;  // K-split scratch, rpl_scratch_floats() floats
};
enum RplMode { RPL_STORE = 0, RPL_ADD = 1, RPL_SILU_MUL = 2, RPL_SWIGLU = 3 };

// core.ActivationType values (core/layer.go:88-99).
enum Act : int {
    ACT_LINEAR = -1, ACT_RELU = 0, ACT_SILU = 1, ACT_GELU = 2, ACT_TANH = 3, ACT_SIGMOID = 4, ACT_LEAKY_RELU = 5,
    ACT_RELU2 = 6,
};
inline bool act_valid(int a) { return a >= ACT_LINEAR && a <= ACT_RELU2; }

// Forward epilogue of launch_matvec: applyBiasAct (layers/dense/dense.go:145-167).
struct BiasAct {
    const double* bias = nullptr;  // [rows] f64, or null
    int act = ACT_LINEAR;
    float* post = nullptr;  // [batch][rows]; null: no epilogue (y = W x only)
};

constexpr int kRplTMaxBatch = 16;  // batch rows per MatVecT launch on LAYOUT_RPL
constexpr int kRplFwdBatch = 8;    // batch rows per K-split forward launch on LAYOUT_RPL

// Device view of one blob. Pointers are into one hipMalloc'd allocation that
// holds weights only: every launch that needs scratch takes it as an argument.
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
    const float* mins = nullptr;  // AffinePacked biases (Blob.Mins), one per group of block_weights
    int64_t n_mins = 0;
    int iq_bits = 0, iq_sg = 0;  // Meta[0], Meta[1] for IQ (iq.go:187-190)
    // LAYOUT_NARROW (codes of a weights.Store DType) and LAYOUT_F32 (f32 weights)
    const uint8_t* codes = nullptr;
    // LAYOUT_RPL
    RplArgs rpl{};
    // Some row factor of rpl.wrow lies outside [2^-2, 2^20] (a row whose
    // largest B-operand value is below 2^-8 or above 2^14): the prefill GEMM
    // runs its kernels that apply the factors. Otherwise every row is held
    // well by fp16 as it stands and the kernels without them run.
    bool gemm_row_factors = false;
    void* base = nullptr;   // allocation owner
    size_t device_bytes = 0;  // bytes of the allocation
};

// Kernel launchers (gemv.hip, gemv_rpl.hip, native.hip). Return a hipError_t
// as int. A launcher whose kernels need scratch takes it as `d_scratch` and
// returns hipErrorInvalidValue when it is null; *_scratch_floats() give the
// floats it needs (0: none).
int launch_rpl(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, int mode = RPL_STORE,
               const float* aux = nullptr, float* d_scratch = nullptr);
int launch_rpl_ex(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, const RplExtra& ex);
size_t rpl_scratch_floats(const DevBlob& b, int batch);
size_t matvec_scratch_floats(const DevBlob& b, int batch);
int launch_matvec(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream, float* d_scratch,
                  const BiasAct* ba = nullptr);
size_t matvec_t_scratch_floats(const DevBlob& b, int batch);
int launch_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch);
// Fused row-interleaved images (gemv_rpl.hip), built on the device from
// resident blobs of one format and width: rpl_fuse_rows stacks the parts'
// rows (each part's rows a multiple of 64); rpl_fuse_pairs interleaves two
// equal blobs row by row (row 2i from a, row 2i+1 from b; rows a multiple of
// 32) for RPL_SWIGLU. The result owns a new allocation (out.base).
int rpl_fuse_rows(const DevBlob* parts, int n, DevBlob& out, void* stream);
int rpl_fuse_pairs(const DevBlob& a, const DevBlob& b, DevBlob& out, void* stream);
// Batched prefill GEMM (gemm_rpl.hip): fp16 MFMA on the row-interleaved Q4_K layout.
bool gemm_supported(const DevBlob& b, int M);
size_t gemm_scratch_floats(const DevBlob& b, int M);
int launch_gemm(const DevBlob& b, const float* d_x, float* d_y, int M, void* stream, float* d_scratch);
// The two halves of launch_gemm, for callers that feed one converted X to
// several projections: the fp16 operand order b's plan reads (A fragments for
// k_gemm_rg), the conversion of X (or, with d_u, of silu(X) * U) into xh and
// xscale (gemm_x_floats / gemm_scale_floats of the widest weight), and the
// launch on it (d_part: split-K partials, gemm_scratch_floats' tail).
bool gemm_x_frag(const DevBlob& b, int M);
size_t gemm_x_floats(const DevBlob& b, int M);
size_t gemm_scale_floats(int M);
void gemm_convert_x(const float* d_x, const float* d_u, int cols, int M, bool frag, void* xh, float* xscale,
                    void* stream);
// With d_splits, a K-split GEMM leaves its partials in d_part
// ([*d_splits][M][rows], unsummed; d_y is then not written) and stores the
// split count there (1: the result is in d_y).
int launch_gemm_xh(const DevBlob& b, const void* xh, const float* xscale, float* d_y, int M, void* stream,
                   float* d_part, int* d_splits = nullptr);
// y[i] = the sum over `splits` slices of part ([splits][n]) in split order.
void launch_split_sum(const float* part, float* y, int64_t n, int splits, void* stream);
// The key-split prompt attention's ranges (part: [ks][M][n_heads][hd + 4],
// ks <= 8) merged straight into the fp16 operand of a GEMM over the
// n_heads * hd columns (row-major, or with frag the A-fragment order), with
// its row factors in xscale.
int launch_merge_x_f16r(const float* part, int ks, int n_heads, int hd, int M, bool frag, void* xh, float* xscale,
                        void* stream);
// h (+)= a, then the RMSNorm of M rows of dim (a multiple of 8, at most 16384)
// straight into the fp16 operand of the GEMM plans (row-major, or with frag
// the A-fragment order of gemm_x_frag plans), and into the f32 rows y when y
// is given. a may be a_splits (1 to 4) unsummed K-split slices, a_stride
// floats apart, added in split order.
int launch_norm_x_f16r(float* h, const float* a, int a_splits, int64_t a_stride, const float* gamma, float* y, void* xh,
                       float* xscale, int M, int dim, double eps, bool frag, void* stream);
// MatVecT on LAYOUT_RPL (slice partials in d_scratch when the plan has several slices).
int launch_rpl_matvec_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, float* d_scratch);
size_t rpl_t_scratch_floats(const RplArgs& a, int batch);
// gx[b][c] += sum_k part[(b*nsplit + k)*cols + c], k ascending.
void launch_gemvt_reduce(const float* part, float* gx, int64_t cols, int nsplit, int batch, void* stream);
// The elementwise applyBiasAct epilogue over y[batch][rows] (layouts without a fused one).
int launch_bias_act(const float* d_y, float* d_y_pre, float* d_post, const double* d_bias, int act, int64_t rows,
                    int batch, void* stream);
// weights.Store DTypes on LAYOUT_NARROW / LAYOUT_F32 (native.hip).
int launch_narrow_acc(const DevBlob& b, const float* d_x, int32_t* d_acc, float* d_act_scale, int batch, void* stream);
int launch_native_fwd(const DevBlob& b, const float* d_x, float* d_y, int batch, void* stream);
// weights.Store.MatVec / MatVecT on FormatNone stores: f64 x / y, f64 sums
// over the decoded weights (weights/native.go:1120-1158).
int launch_store_f64(const DevBlob& b, const double* d_x, double* d_y, void* stream);
size_t store_t_scratch_floats(const DevBlob& b);
int launch_store_t_f64(const DevBlob& b, const double* d_gy, double* d_gx, void* stream, double* d_scratch);
// MatVecT (gx += W^T gy, f32) on LAYOUT_NARROW / LAYOUT_F32.
size_t native_t_scratch_floats(const DevBlob& b, int batch);
int launch_native_t(const DevBlob& b, const float* d_gy, float* d_gx, int batch, void* stream, double* d_scratch);

}  // namespace wv
