/*
 * welvet_hip.h — C ABI of the MI355X (gfx950) Dense MatVec library.
 *
 * Drop-in device backend for welvet's fused dequantize-and-dot path
 * (github.com/openfluke/welvet). Plain C types only: a cgo / ctypes binding
 * passes Go slices / numpy buffers as pointer + length.
 *
 * Conventions
 *   - Every function returns 0 (WV_OK) or a negative WV_E_* code; the message
 *     of the last failure on the calling thread is wv_last_error().
 *   - Formats use quant.Format's numbering (quant/format.go:9-39). The
 *     per-tensor DType packs of weights.Store (FormatNone + DType) use
 *     WV_NATIVE_BASE + core.DType (core/dtype.go:11-52).
 *   - A packed blob is uploaded once into HBM (copied; the caller keeps
 *     ownership of its host buffers, which may be freed after the call) and
 *     referenced by an opaque 64-bit handle afterwards.
 *   - *_dev entry points take device pointers and a hipStream_t passed as
 *     void* (NULL = the library's own stream for the current device); they
 *     enqueue work and return without synchronising. Host-pointer entry
 *     points copy in, compute and copy out synchronously.
 *   - Every entry point except wv_matvec_dev_noalloc is thread-safe (handle
 *     table under a mutex, thread-local error text). A blob holds weights
 *     only: the scratch such a call needs (K-split or slice partials) is one
 *     of a few per-device slots that the call holds until its launches are
 *     enqueued, with the GPU ordering a slot's next user after its last one,
 *     so concurrent calls on one blob, from several threads or on several
 *     streams, never share partials. The slots grow on first use of a larger
 *     shape (hipMalloc) and are kept for the process. wv_matvec_dev_noalloc
 *     is the exception: all its calls on one GPU share one fixed array; calls
 *     on one stream are ordered by it, a call on another stream while the
 *     previous call still runs fails with WV_E_BUSY, and under graph capture
 *     the caller orders the replays (see its declaration). Blob and decoder handles
 *     must not be freed while another thread still calls with them.
 */
#ifndef WELVET_HIP_H
#define WELVET_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define WV_OK 0
#define WV_E_ARG (-1)      /* null pointer / bad argument */
#define WV_E_SHAPE (-2)    /* size mismatch (quant/helpers.go:94-114 wording) */
#define WV_E_FORMAT (-3)   /* format not implemented (quant/errors.go:17-19) */
#define WV_E_OOM (-4)      /* device memory exhausted (webgpu.IsAffineVRAMFull analogue) */
#define WV_E_HIP (-5)      /* HIP runtime error */
#define WV_E_NODEV (-6)    /* no HIP device */
#define WV_E_HANDLE (-7)   /* unknown / freed handle */
#define WV_E_BUSY (-8)     /* wv_matvec_dev_noalloc: its scratch is in use by a call on another stream */

/* ---- formats: quant.Format values (quant/format.go:9-39) ---- */
enum wv_format {
    WV_FMT_NONE = 0,
    WV_FMT_Q8_0 = 1, WV_FMT_Q4_0 = 2, WV_FMT_Q4_1 = 3, WV_FMT_Q5_0 = 4, WV_FMT_Q5_1 = 5,
    WV_FMT_Q2_K = 6, WV_FMT_Q3_K = 7, WV_FMT_Q4_K = 8, WV_FMT_Q5_K = 9, WV_FMT_Q6_K = 10,
    WV_FMT_IQ1_S = 11, WV_FMT_IQ2_XXS = 12, WV_FMT_IQ2_XS = 13, WV_FMT_IQ3_XXS = 14,
    WV_FMT_IQ3_S = 15, WV_FMT_IQ4_NL = 16, WV_FMT_IQ4_XS = 17,
    WV_FMT_TERNARY_PACKED = 18, WV_FMT_BINARY_PACKED = 19, WV_FMT_AFFINE_PACKED = 20
};
/* WV_FMT_NONE blobs hold f32 weights (rows*cols*4 bytes of Raw, quant/none.go:3-21;
 * also a weights.Store FormatNone + DTypeFloat32 master, weights/store.go:19-22).
 * FormatNone stores of a narrow DType: weights.Store{DType, Native, Scale}
 * (weights/store.go:14-32) uploaded as raw = Native, tensor_scale = Scale. */
#define WV_NATIVE_BASE 1000
#define WV_NATIVE_INT8 (WV_NATIVE_BASE + 9)     /* core.DTypeInt8 */
#define WV_NATIVE_INT4 (WV_NATIVE_BASE + 14)    /* core.DTypeInt4 */
#define WV_NATIVE_INT2 (WV_NATIVE_BASE + 17)    /* core.DTypeInt2 */
#define WV_NATIVE_TERNARY (WV_NATIVE_BASE + 19) /* core.DTypeTernary */
#define WV_NATIVE_BINARY (WV_NATIVE_BASE + 20)  /* core.DTypeBinary */

/* core.ActivationType values (core/layer.go:88-99). */
#define WV_ACT_LINEAR (-1)
#define WV_ACT_RELU 0
#define WV_ACT_SILU 1
#define WV_ACT_GELU 2
#define WV_ACT_TANH 3
#define WV_ACT_SIGMOID 4
#define WV_ACT_LEAKY_RELU 5
#define WV_ACT_RELU2 6

/* ---- library ---- */

/* Selects and initialises HIP device `device` for this process.
 * Replaces: webgpu session creation (webgpu/dense.go:23-113). */
int wv_init(int device);

/* Text of the last error on the calling thread ("" if none). */
const char *wv_last_error(void);

/* Library version string. */
const char *wv_version(void);

/* ---- host-side packers: quant.Pack (quant/pack.go:4) ---- */

/* Sizes Pack produces: *raw_len bytes of Blob.Raw, *n_scales / *n_mins floats
 * of Blob.Scales / Blob.Mins, *n_meta bytes of Blob.Meta, *block_weights.
 * Replaces the allocation arithmetic inside quant.Pack* (e.g. q4_0.go:15-16,
 * kquant.go:70-73, iq.go:80-83). */
int wv_pack_sizes(int format, int64_t rows, int64_t cols, size_t *raw_len,
                  size_t *n_scales, size_t *n_mins, size_t *n_meta, int32_t *block_weights);

/* quant.Pack(format, weights, rows, cols) (quant/pack.go:4): row-major f32
 * weights[rows*cols] → caller-sized Raw/Scales/Mins/Meta buffers. */
int wv_pack(int format, const float *weights, int64_t rows, int64_t cols,
            uint8_t *raw, float *scales, float *mins, uint8_t *meta);

/* weights.Store packing of a narrow DType (SetDType -> packNative,
 * weights/native.go:88-97 Int8, 180-194 packInt4, 218-230 packInt2,
 * 249-269 packTernary, 271-283 packBinary): format is WV_NATIVE_INT8 / INT4 /
 * INT2 / TERNARY / BINARY; codes receive (n*bits+7)/8 bytes (LSB-first) and
 * *scale the Store.Scale. */
int wv_pack_native(int format, const float *weights, int64_t n, uint8_t *codes, float *scale);

/* ---- resident blobs ---- */

/* Uploads a packed quant.Blob (quant/format.go:110-131) into HBM once.
 * Replaces the per-call CreateBufferInit uploads of the WebGPU path
 * (webgpu/dense.go:570-617) and the lazily built host SIMD caches
 * (quant.EnsureFusedSIMDCache, quant/qx_simd.go:150). For the WV_NATIVE_*
 * DTypes raw = Store.Native codes and tensor_scale = Store.Scale; for
 * WV_FMT_NONE raw = the f32 weights. */
int wv_blob_upload(int format, int64_t rows, int64_t cols, int32_t block_weights,
                   const uint8_t *raw, size_t raw_len,
                   const float *scales, size_t n_scales,
                   const float *mins, size_t n_mins,
                   const uint8_t *meta, size_t n_meta,
                   float tensor_scale, uint64_t *handle);

/* wv_blob_upload with upload options (0 = wv_blob_upload).
 * WV_UPLOAD_REFERENCE_LAYOUT keeps the device copy in the reference's byte
 * order (Raw, Mins, Scales as quant.Blob holds them, quant/format.go:110-131)
 * instead of the row-interleaved layout that the formats with 256-column rows
 * take by default; every format has kernels on that layout. It serves tests
 * and comparisons of the two layouts: their results agree within the f32
 * tolerance. Unknown flag bits are WV_E_ARG. */
#define WV_UPLOAD_REFERENCE_LAYOUT 1u
int wv_blob_upload_flags(int format, int64_t rows, int64_t cols, int32_t block_weights,
                         const uint8_t *raw, size_t raw_len,
                         const float *scales, size_t n_scales,
                         const float *mins, size_t n_mins,
                         const uint8_t *meta, size_t n_meta,
                         float tensor_scale, uint32_t flags, uint64_t *handle);

/* Uploads a packed blob straight from its ENTITY wire bytes, replacing
 * entity.DecodePackedBlob (model/entity/packed.go:37-76; the same layout as
 * weights.DecodePackedWire, weights/packed_wire.go:57-110) plus the host SIMD
 * cache build: wire = u32 ns | u32 nm | u32 nr | f32 scales[ns] |
 * f32 mins[nm] | raw[nr], little-endian, no padding. The wire carries no
 * Meta or BlockWeights: IQ formats take their default bit width and scale
 * group, BinaryPacked infers g128 from the scale count
 * (InferBinaryBlockWeights, quant/binary_g128.go:79-94) and AffinePacked its
 * group (InferAffineBlockWeights, quant/affine_g64.go:99-122). Errors match
 * the reference's wording: "packed wire too short", "packed wire truncated
 * (need N, have M)". FormatNone payloads (raw f32) are not packed blobs. */
int wv_blob_upload_wire(int format, int64_t rows, int64_t cols, const uint8_t *wire, size_t wire_len,
                        uint64_t *handle);

/* Releases the device copy (host_release.go:15 analogue for the device side). */
int wv_blob_free(uint64_t handle);

/* Shape / residency of a blob: any out-pointer may be NULL. */
int wv_blob_info(uint64_t handle, int *format, int64_t *rows, int64_t *cols,
                 size_t *device_bytes, int *layout);

/* A cap on the device memory that uploaded blobs may hold on each GPU, in
 * bytes (0, the default: no cap). The reference keeps its resident weight
 * caches under a soft cap and answers an upload past it with "weight VRAM
 * budget full" (webgpu/affine_cache.go:111-123, binary_cache.go, f32_cache.go),
 * the one error its Dense layer falls back to the host on
 * (IsAffineVRAMFull, affine_cache.go:73-83; layers/dense/webgpu.go:598-601).
 * Here an upload that would take a device's blobs past the cap fails with
 * WV_E_OOM "wv_blob_upload: weight VRAM budget full (...)" before anything is
 * allocated, and wv_blob_free returns its bytes to the budget. Lowering the
 * cap frees nothing. Copies the decoder makes for its fused projections are
 * not counted. */
int wv_set_weight_budget(uint64_t bytes);

/* Device bytes held by uploaded blobs on the current device (the figure the
 * budget is checked against), and the cap (0: none). Either pointer may be
 * NULL. Reference: AffineWeightCacheBytes (webgpu/affine_cache.go:60-68). */
int wv_weight_bytes(uint64_t *resident, uint64_t *budget);

/* ---- forward: quant.MatVec / dense.MatVecPackedBlob / dense.Forward ---- */

/* y[batch*rows] = W x[batch*cols] for each of `batch` rows (y overwritten).
 * Host pointers; synchronous. The batched form behind Dense's forward
 * (layers/dense/simd.go:23-77 packed branch, forwardSIMDBlockFused
 * simd_block.go:17-39) and dense.MatVecPackedBlob (simd.go:571-614); the
 * single-vector quant.MatVec contract is wv_quant_matvec. On the WV_NATIVE_*
 * DTypes it is Dense's int8 path (forwardSIMDNarrowI8 / forwardSIMDInt8,
 * simd.go:130-195, 303-326): activations absmax-quantized to int8
 * (quantizeActsI8, simd.go:526-549), exact int32 accumulators,
 * y = f32(acc) * actScale * scale. On WV_FMT_NONE it is forwardSIMDMasterF32
 * (simd.go:201-214): f32 weights, f64 sums. */
int wv_matvec(uint64_t handle, const float *x, float *y, int32_t batch);

/* Device-pointer form of wv_matvec, enqueued on `stream`. */
int wv_matvec_dev(uint64_t handle, const float *d_x, float *d_y, int32_t batch, void *stream);

/* wv_matvec_dev that allocates nothing. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Kernels that need scratch (the K-split partials of large-K shapes) use one
 * fixed 4 MiB device array per GPU, held until the process ends, instead of a
 * per-call allocation; a shape whose partials (up to 8 batch rows x the K
 * split x the rows padded to 64) exceed 2^20 floats fails with WV_E_SHAPE
 * before anything is enqueued. Every call on a GPU shares that GPU's array,
 * so calls that overlap on one GPU would race: calls on one stream are
 * ordered by it, and a call on another stream while the previous call's
 * work has not finished fails with WV_E_BUSY, nothing enqueued. Under HIP
 * graph capture that check is off and callers must order the replays
 * themselves. Results equal wv_matvec_dev's. */
int wv_matvec_dev_noalloc(uint64_t handle, const float *d_x, float *d_y, int32_t batch, void *stream);

/* quant.MatVec (quant/matvec.go:5-35) for one vector, with its argument check
 * checkBlobYX (quant/helpers.go:94-103): len_x >= cols and len_y >= rows, else
 * WV_E_SHAPE "MatVec: size mismatch rows=R cols=C len(x)=X len(y)=Y"; x past
 * cols is not read and y past rows is not written. Host pointers; synchronous.
 * WV_NATIVE_* blobs are not quant blobs (WV_E_FORMAT). */
int wv_quant_matvec(uint64_t handle, const float *x, size_t len_x, float *y, size_t len_y);

/* dense.MatVecPackedBlob (layers/dense/simd.go:570-614), the LM head's and
 * standalone projections' entry, one vector: len_x >= cols and len_y >= rows,
 * else WV_E_SHAPE "dense: packed matvec shape"; an unknown handle is
 * WV_E_HANDLE "dense: nil packed blob". Its format switch covers the packed
 * formats only: a WV_FMT_NONE blob (and a WV_NATIVE_* Store, a FormatNone
 * blob there) is WV_E_FORMAT "dense: MatVecPackedBlob unsupported none".
 * Otherwise as wv_quant_matvec: x past cols is not read, y past rows is not
 * written. Host pointers; synchronous. */
int wv_matvec_packed_blob(uint64_t handle, const float *x, size_t len_x, float *y, size_t len_y);

/* dense.Forward for a linear map with bias and activation (layers/dense/
 * dense.go:100-112 -> ForwardSIMD simd.go:23-77, applyBiasAct dense.go:145-167):
 * pre[batch*rows] = W x (+ bias), post = act(pre). bias: f64[rows] or NULL
 * (weights.Store.Bias); act: a WV_ACT_* value. With a bias, pre holds
 * f32(f64(Wx) + bias); post = f32(act(f64(pre))). post may be NULL only when
 * act is WV_ACT_LINEAR and bias is NULL (linearNoBias: post is pre). Every
 * blob kind, including the WV_NATIVE_* DTypes and WV_FMT_NONE. */
int wv_dense_forward(uint64_t handle, const float *x, float *pre, float *post, int32_t batch,
                     const double *bias, int32_t act);

/* Device-pointer form of wv_dense_forward (d_bias a device pointer), enqueued on `stream`. */
int wv_dense_forward_dev(uint64_t handle, const float *d_x, float *d_pre, float *d_post, int32_t batch,
                         const double *d_bias, int32_t act, void *stream);

/* dense.Forward for a block of token rows (a prefill), through the batched
 * prefill GEMM: forwardSIMDBlockFused (layers/dense/simd_block.go:17-39),
 * which runs the block's rows as independent GEMVs, with applyBiasAct
 * (dense.go:145-167) after it. pre = W x as wv_matmul_dev computes it (fp16
 * MFMA, within 2e-3 normwise, wherever wv_matmul_dev takes the GEMM: a
 * row-interleaved blob and batch > 8, or Q4_K at any batch), then bias and
 * act as in wv_dense_forward; every other case is wv_dense_forward itself.
 * Arguments, errors and the post rule as wv_dense_forward. */
int wv_dense_forward_block(uint64_t handle, const float *x, float *pre, float *post, int32_t batch,
                           const double *bias, int32_t act);

/* Device-pointer form of wv_dense_forward_block, enqueued on `stream`. */
int wv_dense_forward_block_dev(uint64_t handle, const float *d_x, float *d_pre, float *d_post, int32_t batch,
                               const double *d_bias, int32_t act, void *stream);

/* WV_NATIVE_* DTypes only: the exact int32 accumulators (batch*rows) and the
 * per-batch-row activation scales (batch) of the int8 path, device pointers. */
int wv_native_acc_dev(uint64_t handle, const float *d_x, int32_t *d_acc, float *d_act_scale,
                      int32_t batch, void *stream);

/* weights.Store.MatVec with f64 activations (weights/store.go:133-145,
 * 162-180): packed blobs run quant.MatVec on f32(x) and widen y (its check and
 * wording); WV_FMT_NONE and WV_NATIVE_* stores run matVecNativeF64
 * (weights/native.go:1120-1137): y = sum_c f64(w_rc) * x_c in f64 over the
 * decoded weights (weightAt, weights/decode.go:50-215), WV_E_SHAPE
 * "weights: matvecF64 shape" if len_x < cols or len_y < rows. y entries past
 * rows are set to 0, as MatVec's zeroed result buffer. Host pointers. */
int wv_store_matvec(uint64_t handle, const double *x, size_t len_x, double *y, size_t len_y);

/* ---- batched prefill: M token rows through the same Dense layer ---- */

/* Y[M*rows] = X[M*cols] W^T for a block of M token rows (Y overwritten).
 * Replaces forwardSIMDBlockFused (layers/dense/simd_block.go:17-39) and the
 * batch loop of forwardSIMDQ4_0 (layers/dense/simd.go:294-299), which run M
 * independent GEMVs. Row-interleaved blobs use fp16 MFMA with f32
 * accumulation (results within 2e-3 normwise of the f64 reference, not the
 * 1e-5 of wv_matvec; each token row and each weight row is scaled by a power
 * of two into fp16's range and back, so outlier or tiny activations and
 * weights keep that bar): Q4_K at every m, the other row-interleaved formats
 * (wv_blob_info layout "row-interleaved") from m = 9. Every other
 * case runs the batched GEMV kernels of wv_matvec_dev. Device pointers,
 * enqueued on `stream`. */
int wv_matmul_dev(uint64_t handle, const float *d_x, float *d_y, int32_t m, void *stream);

/* Host-pointer form of wv_matmul_dev; synchronous. */
int wv_matmul(uint64_t handle, const float *x, float *y, int32_t m);

/* ---- backward: quant.MatVecT ---- */

/* gx[batch*cols] += W^T gy[batch*rows] (gx NOT zeroed, quant/matvec_t.go:3-5).
 * Host pointers; synchronous. The batched form of quant.MatVecT
 * (quant/matvec_t.go:5) as backwardSIMDPacked calls it (layers/dense/
 * simd_quant.go:103-126); on WV_NATIVE_* and WV_FMT_NONE blobs the input
 * gradient of BackwardSIMD (simd.go:412-504): f64 sums of gy * w added to gx. */
int wv_matvec_t(uint64_t handle, const float *gy, float *gx, int32_t batch);

/* Device-pointer form of wv_matvec_t. */
int wv_matvec_t_dev(uint64_t handle, const float *d_gy, float *d_gx, int32_t batch, void *stream);

/* quant.MatVecT (quant/matvec_t.go:5-35) for one vector, with checkBlobGYGX
 * (quant/helpers.go:105-114): len_gy >= rows and len_gx >= cols, else WV_E_SHAPE
 * "MatVecT: size mismatch rows=R cols=C len(gy)=G len(gx)=X"; gx[:cols] += W^T gy[:rows]. */
int wv_quant_matvec_t(uint64_t handle, const float *gy, size_t len_gy, float *gx, size_t len_gx);

/* weights.Store.MatVecT with f64 activations (weights/store.go:147-160,
 * 182-206): packed blobs run quant.MatVecT on f32 copies of gy and gx (every
 * gx entry comes back through f32); WV_FMT_NONE and WV_NATIVE_* stores run
 * matVecTNativeF64 (weights/native.go:1139-1158): gx[c] += sum_r w_rc * gy_r
 * in f64, rows with gy_r == 0 skipped; WV_E_SHAPE "weights: matvecTF64 shape". */
int wv_store_matvec_t(uint64_t handle, const double *gy, size_t len_gy, double *gx, size_t len_gx);

/* ---- device decode step (greedy), for a decoder whose projections are resident blobs ---- */

/* Dimensions of a decoder (model/transformer config; layers/mha/config.go,
 * layers/swiglu/config.go, layers/rmsnorm/config.go). head_dim 64 or 128,
 * n_heads a multiple of n_kv_heads with at most 8 query heads per KV head. */
typedef struct wv_decoder_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
    double rope_theta, rms_eps;
} wv_decoder_config;

/* Creates a decoder: activations, f32 KV caches (head-major [n_kv_heads][max_seq][head_dim])
 * per layer (zeroed) and its own stream on the current device. */
int wv_decoder_create(const wv_decoder_config *cfg, uint64_t *decoder);

/* Layer `layer`'s projections as resident blobs {Q, K, V, O, gate, up, down}
 * (shapes as in mha.Layer Q/K/V/O and swiglu.Layer Gate/Up/Down, rows = out)
 * and its two RMSNorm gammas (host, hidden floats each). The blobs must stay
 * allocated while the decoder uses them. Replaces the per-layer sequence of
 * model/transformer/forward.go:55-77. */
int wv_decoder_set_layer(uint64_t decoder, int32_t layer, const uint64_t *blobs, const float *attn_norm,
                         const float *ffn_norm);

/* LM head blob (vocab x hidden), final RMSNorm gamma (NULL = no final norm,
 * forward.go:80-86) and the f32 embedding table (vocab x hidden, host). */
int wv_decoder_set_output(uint64_t decoder, uint64_t lm_head, const float *final_norm, const float *embedding);

/* Writes KV-cache rows first_pos .. first_pos+n_pos-1 of `layer` (host k, v:
 * n_pos rows of n_kv_heads*head_dim floats), as the prompt's prefill would. */
int wv_decoder_set_kv(uint64_t decoder, int32_t layer, int32_t first_pos, int32_t n_pos, const float *k,
                      const float *v);

/* Non-zero: capture the whole step once into a HIP graph and replay it. */
int wv_decoder_use_graph(uint64_t decoder, int32_t enable);

/* Runs n_steps greedy decode steps from input `token` at position `pos`:
 * each step is ForwardTokens for one new token (forward.go:26-90: RMSNorm,
 * Q/K/V, RoPE, KV append, GQA causal attention, O + residual, RMSNorm, SwiGLU
 * + residual, final norm, LM head) followed by argmax, whose token feeds the
 * next step. advance_pos != 0 moves the position on by one per step (real
 * generation); 0 recomputes position `pos` each step. tokens_out (host,
 * n_steps, may be NULL) receives the generated tokens, last_logits (host,
 * vocab, may be NULL) the last step's logits. Synchronous. */
int wv_decoder_generate(uint64_t decoder, int32_t token, int32_t pos, int32_t n_steps, int32_t advance_pos,
                        int32_t *tokens_out, float *last_logits);

/* ForwardTokens over a prompt (model/transformer/forward.go:26-90 with the
 * whole token block, as mha.Forward runs it with its KV cache,
 * layers/mha/cpu.go:163-215): the n_tokens ids (host) at positions
 * pos0 .. pos0+n_tokens-1 go through every layer as one block: RMSNorm of each
 * row, Q/K/V of the block (the batched prefill GEMM where the blob has one,
 * fp16 MFMA within 2e-3; the batched GEMVs otherwise), RoPE and the K/V rows
 * appended to the cache at their positions, causal GQA attention of each row
 * over the cache up to its own position (layers/mha/attn.go:40-118), O +
 * residual, RMSNorm, SwiGLU + residual; then the final norm, LM head and
 * argmax of the last row. *next_token (may be NULL) receives that argmax and
 * last_logits (host, vocab floats, may be NULL) the last row's logits.
 * wv_decoder_generate(*next_token, pos0 + n_tokens, ...) then continues the
 * sequence with no host copy of the cache. Errors: WV_E_ARG "empty ids",
 * WV_E_SHAPE when pos0 + n_tokens exceeds max_seq. Synchronous. */
int wv_decoder_prefill(uint64_t decoder, const int32_t *tokens, int32_t n_tokens, int32_t pos0,
                       int32_t *next_token, float *last_logits);

/* Releases the decoder (not the blobs it references). */
int wv_decoder_free(uint64_t decoder);

/* ---- streams ---- */

/* Blocks until all work the library enqueued on `stream` (NULL = its own) is done. */
int wv_sync(void *stream);

#ifdef __cplusplus
}
#endif
#endif /* WELVET_HIP_H */
