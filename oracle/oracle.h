/*
 * oracle.h — TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of welvet's CPU algorithms for the Dense MatVec path
 * (reference: github.com/openfluke/welvet, read at /root/reference):
 *   - the packers of quant.Pack and weights' DTypeTernary native pack,
 *   - the decoders of quant.Unpack,
 *   - the scalar quant.MatVec / quant.MatVecT (flat f32 walk),
 *   - the fused SIMD path of layers/dense (Ensure*SIMDCache projections,
 *     simd.Dot*Row kernels with f64 accumulation, row-sharded threads),
 *   - the narrow-DType int8 path (quantizeActsI8 + DotI8Tile) and the
 *     weights.Store packers / decoders of those DTypes.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker / the reported CPU baseline. The HIP
 * product (welvet_amd/) never links or calls it.
 *
 * Format numbers are quant.Format's iota order (quant/format.go:9-39).
 */
#ifndef WELVET_ORACLE_H
#define WELVET_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    OR_NONE = 0, OR_Q8_0, OR_Q4_0, OR_Q4_1, OR_Q5_0, OR_Q5_1,
    OR_Q2_K, OR_Q3_K, OR_Q4_K, OR_Q5_K, OR_Q6_K,
    OR_IQ1_S, OR_IQ2_XXS, OR_IQ2_XS, OR_IQ3_XXS, OR_IQ3_S, OR_IQ4_NL, OR_IQ4_XS,
    OR_TERNARY, OR_BINARY, OR_AFFINE
};

/* Sizes quant.Pack produces for (format, rows, cols): out[0]=raw bytes,
 * out[1]=n scales, out[2]=n mins, out[3]=n meta bytes, out[4]=BlockWeights.
 * Returns 0, or -1 for an unsupported format / bad shape. */
int or_pack_sizes(int fmt, int64_t rows, int64_t cols, int64_t out[5]);

/* quant.Pack (quant/pack.go:4). Buffers sized by or_pack_sizes. */
int or_pack(int fmt, const float *w, int64_t rows, int64_t cols,
            uint8_t *raw, float *scales, float *mins, uint8_t *meta);

/* quant.Unpack (quant/unpack.go:4): dequantize to out[rows*cols]. */
int or_unpack(int fmt, int64_t rows, int64_t cols, int32_t block_weights,
              const uint8_t *raw, int64_t raw_len,
              const float *scales, int64_t n_scales,
              const float *mins, int64_t n_mins,
              const uint8_t *meta, int64_t n_meta, float *out);

/* quant.MatVec (quant/matvec.go:5): y overwritten, flat-order f32 walk
 * (AffinePacked: the per-group form of affine_g64.go:178-267). mins is
 * Blob.Mins (AffinePacked biases; NULL for every other format). */
int or_matvec_scalar(int fmt, int64_t rows, int64_t cols, int32_t block_weights,
                     const uint8_t *raw, int64_t raw_len,
                     const float *scales, int64_t n_scales,
                     const float *mins, int64_t n_mins,
                     const uint8_t *meta, int64_t n_meta,
                     const float *x, float *y);

/* quant.MatVecT (quant/matvec_t.go:5): gx += W^T gy (gx not zeroed). */
int or_matvec_t_scalar(int fmt, int64_t rows, int64_t cols, int32_t block_weights,
                       const uint8_t *raw, int64_t raw_len,
                       const float *scales, int64_t n_scales,
                       const float *mins, int64_t n_mins,
                       const uint8_t *meta, int64_t n_meta,
                       const float *gy, float *gx);

/* Textbook f64 GEMV over an already-dequantized f32 matrix: y[r] = sum_c w*x in
 * f64 (long double accumulation, rounded once to f64). */
void or_gemv_f64(const float *w, int64_t rows, int64_t cols, const float *x, double *y);

/* ---- fused SIMD path (layers/dense ForwardSIMD) = the timed CPU baseline ---- */

/* Builds the Ensure*SIMDCache projection once (timed separately by callers).
 * Returns an opaque handle (NULL on failure). */
void *or_simd_prepare(int fmt, int64_t rows, int64_t cols, int32_t block_weights,
                      const uint8_t *raw, int64_t raw_len,
                      const float *scales, int64_t n_scales,
                      const float *mins, int64_t n_mins,
                      const uint8_t *meta, int64_t n_meta);
void or_simd_free(void *h);
/* y = W x for `batch` rows of x (batch*cols) → y (batch*rows), using
 * nthreads row-shard workers (gemv_parallel.go: serial below 64 rows). */
int or_simd_matvec(void *h, const float *x, float *y, int batch, int nthreads);

/* ---- DTypeTernary (FormatNone, per-tensor absMax scale) int8 path ---- */

/* weights/native.go:249-267 packTernary: codes 4/byte LSB-first. */
void or_pack_native_ternary(const float *w, int64_t n, uint8_t *codes, float *scale);
/* layers/dense/simd.go:526-549 quantizeActsI8; returns the act scale. */
float or_quantize_acts_i8(const float *x, int64_t n, int8_t *xq);
/* layers/dense/simd.go:130-147 forwardSIMDNarrowI8 (serial; expands codes
 * every call as the reference does). acc (rows*batch int32) and act_scale
 * (batch floats) may be NULL. */
int or_ternary_i8_forward(const uint8_t *codes, float scale, int64_t rows, int64_t cols,
                          const float *x, float *y, int32_t *acc, float *act_scale, int batch);

/* ---- narrow weights.Store DTypes (dt = core.DType: 9 Int8, 14 Int4, 17 Int2,
 * 19 Ternary, 20 Binary) ---- */

/* packNative (weights/native.go:88-283): codes (n*bits+7)/8 bytes LSB-first,
 * Store.Scale; returns bits per code (0: not a narrow DType). */
int or_pack_native(int dt, const float *w, int64_t n, uint8_t *codes, float *scale);
/* expandNarrowToI8 (layers/dense/simd.go:149-195). */
int or_expand_narrow_i8(int dt, const uint8_t *codes, int64_t n, int8_t *out);
/* Dense's int8 path for any narrow DType (simd.go:130-147, 303-326). */
int or_narrow_i8_forward(int dt, const uint8_t *codes, float scale, int64_t rows, int64_t cols,
                         const float *x, float *y, int32_t *acc, float *act_scale, int batch);
/* weightAt (weights/decode.go:50-215): the f32 weights weights.Store decodes. */
int or_native_decode(int dt, const uint8_t *codes, float scale, int64_t n, float *out);

/* One-time cost helpers for the baseline report. */
int or_num_cpus(void);

#ifdef __cplusplus
}
#endif
#endif
