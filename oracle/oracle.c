/*
 * oracle.c — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * CPU restatement of welvet's Dense MatVec path. Each function cites the
 * reference file:line it follows. Built with -O2 -ffp-contract=off (no FMA
 * contraction, no fast-math) so that f32 expressions round after every
 * operation as Go's float32 arithmetic does on amd64.
 *
 * Parity pins for this file live in tests/test_oracle_*.py: closed-form
 * known-answer blocks, invariants, brute force on tiny inputs and an
 * independent numpy restatement (oracle/np_ref.py).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>
#include <immintrin.h>

/* ------------------------------------------------------------------ */
/* helpers (quant/helpers.go)                                          */
/* ------------------------------------------------------------------ */

/* putF32/getF32 little-endian (quant/helpers.go:8-19). x86-64 is LE. */
static void put_f32(uint8_t *b, float v) { memcpy(b, &v, 4); }
static float get_f32(const uint8_t *b) { float v; memcpy(&v, b, 4); return v; }
static uint32_t get_u32(const uint8_t *b) { uint32_t v; memcpy(&v, b, 4); return v; }
static void put_u32(uint8_t *b, uint32_t v) { memcpy(b, &v, 4); }

/* roundToInt = int(math.Round(v)), half away from zero (helpers.go:151-153). */
static long round_to_int(double v) { return (long)round(v); }
static long clamp_l(long v, long lo, long hi) { return v < lo ? lo : (v > hi ? hi : v); }
static float abs32(float v) { return v < 0 ? -v : v; }

/* absMean in f32, sequential (helpers.go:49-58). */
static float abs_mean(const float *w, int64_t s, int64_t e) {
    if (e <= s) return 0;
    float sum = 0;
    for (int64_t i = s; i < e; i++) sum += abs32(w[i]);
    return sum / (float)(e - s);
}
/* maxAbsRange (helpers.go:60-69). */
static float max_abs_range(const float *w, int64_t s, int64_t e) {
    float m = 0;
    for (int64_t i = s; i < e; i++) { float a = abs32(w[i]); if (a > m) m = a; }
    return m;
}
/* minMaxRange (helpers.go:71-85). */
static void min_max_range(const float *w, int64_t s, int64_t e, float *mn, float *mx) {
    if (s >= e) { *mn = 0; *mx = 0; return; }
    float a = w[s], b = w[s];
    for (int64_t i = s + 1; i < e; i++) { if (w[i] < a) a = w[i]; if (w[i] > b) b = w[i]; }
    *mn = a; *mx = b;
}

/* bitWriter / bitReader: LSB-first within bytes, bytes ascending
 * (helpers.go:116-149). The reader returns 0 bits past the buffer end. */
typedef struct { uint8_t *buf; int64_t len; int64_t pos; } bitw_t;
static void bw_write(bitw_t *bw, uint32_t val, int nbits) {
    for (int i = 0; i < nbits; i++) {
        if ((val >> i) & 1u) bw->buf[bw->pos >> 3] |= (uint8_t)(1u << (bw->pos & 7));
        bw->pos++;
    }
}
typedef struct { const uint8_t *buf; int64_t len; int64_t pos; } bitr_t;
static uint32_t br_read(bitr_t *br, int nbits) {
    uint32_t v = 0;
    for (int i = 0; i < nbits; i++) {
        if ((br->pos >> 3) < br->len && ((br->buf[br->pos >> 3] >> (br->pos & 7)) & 1u)) v |= 1u << i;
        br->pos++;
    }
    return v;
}

/* ------------------------------------------------------------------ */
/* format specs                                                        */
/* ------------------------------------------------------------------ */

/* kSpecFor (quant/kquant.go:36-51). */
typedef struct { int bits, has_dmin, qmax, mid; } kspec_t;
static int kspec_for(int fmt, kspec_t *s) {
    switch (fmt) {
    case OR_Q2_K: *s = (kspec_t){2, 1, 3, 0}; return 1;
    case OR_Q3_K: *s = (kspec_t){3, 1, 7, 0}; return 1;
    case OR_Q4_K: *s = (kspec_t){4, 1, 15, 0}; return 1;
    case OR_Q5_K: *s = (kspec_t){5, 1, 31, 0}; return 1;
    case OR_Q6_K: *s = (kspec_t){6, 0, 63, 32}; return 1;
    default: return 0;
    }
}
/* kSuperBytes (kquant.go:53-60). */
static int64_t ksuper_bytes(const kspec_t *s) {
    int64_t n = 8 + 16;
    if (s->has_dmin) n += 16;
    return n + (256 * s->bits + 7) / 8;
}

/* iqSpecFor (quant/iq.go:49-68). */
typedef struct { int bits, sg, nonlinear; float mid; } iqspec_t;
static int iqspec_for(int fmt, iqspec_t *s) {
    switch (fmt) {
    case OR_IQ1_S: *s = (iqspec_t){1, 32, 0, 0.5f}; return 1;
    case OR_IQ2_XXS: *s = (iqspec_t){2, 32, 0, 1.5f}; return 1;
    case OR_IQ2_XS: *s = (iqspec_t){2, 16, 0, 1.5f}; return 1;
    case OR_IQ3_XXS: *s = (iqspec_t){3, 32, 0, 3.5f}; return 1;
    case OR_IQ3_S: *s = (iqspec_t){3, 16, 0, 3.5f}; return 1;
    case OR_IQ4_NL: *s = (iqspec_t){4, 32, 1, 0.0f}; return 1;
    case OR_IQ4_XS: *s = (iqspec_t){4, 16, 0, 7.5f}; return 1;
    default: return 0;
    }
}
/* iq4nlGrid (quant/iq.go:23-40). A data table: the values must be identical. */
static const float IQ4NL_GRID[16] = {
    -1.0f, -0.6961928f, -0.52507305f, -0.3949175f, -0.28444138f, -0.18477343f,
    -0.091050036f, 0.0f, 0.0795803f, 0.1609302f, 0.2461123f, 0.33791524f,
    0.44070983f, 0.562617f, 0.72295684f, 1.0f};

int or_pack_sizes(int fmt, int64_t rows, int64_t cols, int64_t out[5]) {
    if (rows <= 0 || cols <= 0) return -1;
    int64_t n = rows * cols;
    memset(out, 0, 5 * sizeof(int64_t));
    kspec_t ks; iqspec_t is;
    switch (fmt) {
    case OR_Q4_0: out[0] = (n + 31) / 32 * 20; out[4] = 32; return 0;
    case OR_Q8_0: out[0] = (n + 31) / 32 * 36; out[4] = 32; return 0;
    case OR_Q4_1: out[0] = (n + 31) / 32 * 24; out[4] = 32; return 0;
    case OR_Q5_0: out[0] = (n + 31) / 32 * 24; out[4] = 32; return 0;
    case OR_Q5_1: out[0] = (n + 31) / 32 * 28; out[4] = 32; return 0;
    case OR_TERNARY: out[0] = (n + 15) / 16 * 4; out[1] = (n + 15) / 16; out[4] = 16; return 0;
    case OR_BINARY: out[0] = (n + 31) / 32 * 4; out[1] = (n + 31) / 32; out[4] = 32; return 0;
    case OR_AFFINE: /* PackAffine4 (affine_pack.go:15-41): 4-bit codes, group 64 along cols */
        if (cols % 64) return -1;
        out[0] = n / 2; out[1] = out[2] = n / 64; out[3] = 1; out[4] = 64;
        return 0;
    default: break;
    }
    if (kspec_for(fmt, &ks)) { out[0] = (n + 255) / 256 * ksuper_bytes(&ks); out[4] = 256; return 0; }
    if (iqspec_for(fmt, &is)) {
        int64_t padn = (n + is.sg - 1) / is.sg * is.sg;
        out[0] = (padn * is.bits + 7) / 8; out[1] = padn / is.sg; out[3] = 2; out[4] = 32;
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------ */
/* packers                                                             */
/* ------------------------------------------------------------------ */

/* quantNibble (quant/q4_0.go:142-154): f32 divide, f64 round, clamp [-8,7]. */
static int quant_nibble(const float *w, int64_t i, int64_t n, float scale) {
    if (i >= n) return 0;
    long q = round_to_int((double)(w[i] / scale));
    if (q > 7) q = 7;
    if (q < -8) q = -8;
    return (int)q;
}

/* PackQ4_0 (quant/q4_0.go:10-45). */
static void pack_q4_0(const float *w, int64_t n, uint8_t *raw) {
    int64_t blocks = (n + 31) / 32;
    for (int64_t bi = 0; bi < blocks; bi++) {
        int64_t s = bi * 32, e = s + 32 < n ? s + 32 : n;
        float scale = max_abs_range(w, s, e) / 7;
        if (scale == 0) scale = 1;
        uint8_t *o = raw + bi * 20;
        put_f32(o, scale);
        for (int j = 0; j < 16; j++) {
            int q1 = quant_nibble(w, s + 2 * j, n, scale), q2 = quant_nibble(w, s + 2 * j + 1, n, scale);
            o[4 + j] = (uint8_t)((q1 & 0xF) | ((q2 & 0xF) << 4));
        }
    }
}

/* PackQ8_0 (quant/q8_0.go:8-44): q = round(f64(w)/f64(scale)) clamp ±127. */
static void pack_q8_0(const float *w, int64_t n, uint8_t *raw) {
    int64_t blocks = (n + 31) / 32;
    for (int64_t bi = 0; bi < blocks; bi++) {
        int64_t s = bi * 32, e = s + 32 < n ? s + 32 : n;
        float scale = max_abs_range(w, s, e) / 127;
        if (scale == 0) scale = 1;
        uint8_t *o = raw + bi * 36;
        put_f32(o, scale);
        for (int j = 0; j < 32; j++) {
            int64_t i = s + j;
            long q = 0;
            if (i < n) q = clamp_l(round_to_int((double)w[i] / (double)scale), -127, 127);
            o[4 + j] = (uint8_t)(int8_t)q;
        }
    }
}

/* packQ4_1 (quant/q4_1.go:8-49): q = round(f64(f32((w-mn)/scale))) in [0,15]. */
static void pack_q4_1(const float *w, int64_t n, uint8_t *raw) {
    int64_t blocks = (n + 31) / 32;
    for (int64_t bi = 0; bi < blocks; bi++) {
        int64_t s = bi * 32, e = s + 32 < n ? s + 32 : n;
        float mn, mx; min_max_range(w, s, e, &mn, &mx);
        float scale = (mx - mn) / 15;
        if (scale == 0) scale = 1;
        uint8_t *o = raw + bi * 24;
        put_f32(o, scale); put_f32(o + 4, mn);
        for (int j = 0; j < 16; j++) {
            uint8_t nib[2];
            for (int k = 0; k < 2; k++) {
                int64_t i = s + 2 * j + k;
                long q = 0;
                if (i < n) { float t = (w[i] - mn) / scale; q = clamp_l(round_to_int((double)t), 0, 15); }
                nib[k] = (uint8_t)q;
            }
            o[8 + j] = (uint8_t)(nib[0] | (nib[1] << 4));
        }
    }
}

/* packQ5_0 (quant/q5_0.go:8-45): 5-bit LSB-first stream of q+16. */
static void pack_q5_0(const float *w, int64_t n, uint8_t *raw) {
    int64_t blocks = (n + 31) / 32;
    for (int64_t bi = 0; bi < blocks; bi++) {
        int64_t s = bi * 32, e = s + 32 < n ? s + 32 : n;
        float scale = max_abs_range(w, s, e) / 15;
        if (scale == 0) scale = 1;
        uint8_t *o = raw + bi * 24;
        put_f32(o, scale);
        bitw_t bw = {o + 4, 20, 0};
        for (int j = 0; j < 32; j++) {
            int64_t i = s + j;
            long q = 16;
            if (i < n) q = clamp_l(round_to_int((double)w[i] / (double)scale) + 16, 0, 31);
            bw_write(&bw, (uint32_t)q, 5);
        }
    }
}

/* packQ5_1 (quant/q5_1.go:8-47). */
static void pack_q5_1(const float *w, int64_t n, uint8_t *raw) {
    int64_t blocks = (n + 31) / 32;
    for (int64_t bi = 0; bi < blocks; bi++) {
        int64_t s = bi * 32, e = s + 32 < n ? s + 32 : n;
        float mn, mx; min_max_range(w, s, e, &mn, &mx);
        float scale = (mx - mn) / 31;
        if (scale == 0) scale = 1;
        uint8_t *o = raw + bi * 28;
        put_f32(o, scale); put_f32(o + 4, mn);
        bitw_t bw = {o + 8, 20, 0};
        for (int j = 0; j < 32; j++) {
            int64_t i = s + j;
            long q = 0;
            if (i < n) { float t = (w[i] - mn) / scale; q = clamp_l(round_to_int((double)t), 0, 31); }
            bw_write(&bw, (uint32_t)q, 5);
        }
    }
}

/* packK (quant/kquant.go:62-176). */
static void pack_k(const kspec_t *sp, const float *w, int64_t n, uint8_t *raw) {
    int64_t sbs = (n + 255) / 256, sbb = ksuper_bytes(sp);
    for (int64_t si = 0; si < sbs; si++) {
        int64_t base = si * 256;
        uint8_t *o = raw + si * sbb;
        float gscale[16], gmin[16];
        uint32_t qs[256];
        for (int g = 0; g < 16; g++) {
            int64_t gs = base + g * 16, ge = gs + 16;
            gscale[g] = 0; gmin[g] = 0;
            if (gs >= n) { gscale[g] = 1; continue; }  /* kquant.go:86-89: qs stay 0 */
            if (ge > n) ge = n;
            if (sp->has_dmin) {
                float mn, mx; min_max_range(w, gs, ge, &mn, &mx);
                float sc = (mx - mn) / (float)sp->qmax;
                if (sc == 0) sc = 1;
                gmin[g] = mn; gscale[g] = sc;
                for (int j = 0; j < 16; j++) {
                    int64_t i = gs + j;
                    long q = 0;
                    if (i < n) { float t = (w[i] - mn) / sc; q = clamp_l(round_to_int((double)t), 0, sp->qmax); }
                    qs[g * 16 + j] = (uint32_t)q;
                }
            } else {
                float amax = max_abs_range(w, gs, ge);
                float sc = amax / (float)sp->mid;
                if (sc == 0) sc = 1;
                gscale[g] = sc;
                for (int j = 0; j < 16; j++) {
                    int64_t i = gs + j;
                    long q = sp->mid;
                    if (i < n) q = clamp_l(round_to_int((double)w[i] / (double)sc) + sp->mid, 0, sp->qmax);
                    qs[g * 16 + j] = (uint32_t)q;
                }
            }
        }
        /* groups past n keep qs = 0 for every spec (the Go array is zeroed). */
        for (int g = 0; g < 16; g++)
            if (base + g * 16 >= n) for (int j = 0; j < 16; j++) qs[g * 16 + j] = 0;
        float d = 0, dmin = 0;
        for (int g = 0; g < 16; g++) {
            if (gscale[g] > d) d = gscale[g];
            if (sp->has_dmin) { float a = abs32(gmin[g]); if (a > dmin) dmin = a; }
        }
        if (d == 0) d = 1;
        if (sp->has_dmin && dmin == 0) dmin = 1;
        memset(o, 0, (size_t)sbb);
        put_f32(o, d); put_f32(o + 4, dmin);
        for (int g = 0; g < 16; g++)
            o[8 + g] = (uint8_t)clamp_l(round_to_int((double)gscale[g] / (double)d * 255), 0, 255);
        int64_t qoff = 8 + 16;
        if (sp->has_dmin) {
            for (int g = 0; g < 16; g++) {
                long u = 0;
                if (dmin > 0) u = clamp_l(round_to_int((double)gmin[g] / (double)dmin * 127), -127, 127);
                o[qoff + g] = (uint8_t)(int8_t)u;
            }
            qoff += 16;
        }
        bitw_t bw = {o + qoff, sbb - qoff, 0};
        for (int i = 0; i < 256; i++) bw_write(&bw, qs[i], sp->bits);
    }
}

/* packIQ (quant/iq.go:70-167). */
static void pack_iq(const iqspec_t *sp, const float *w, int64_t n, uint8_t *raw, float *scales, uint8_t *meta) {
    int64_t padn = (n + sp->sg - 1) / sp->sg * sp->sg, nsc = padn / sp->sg;
    int qmax = (1 << sp->bits) - 1;
    bitw_t bw = {raw, (padn * sp->bits + 7) / 8, 0};
    for (int64_t s = 0; s < nsc; s++) {
        int64_t st = s * sp->sg, en = st + sp->sg;
        if (en > n) en = n;
        if (st >= n) {
            scales[s] = 1;
            for (int j = 0; j < sp->sg; j++) bw_write(&bw, 0, sp->bits);
            continue;
        }
        if (sp->nonlinear) {
            float scale = max_abs_range(w, st, en);
            if (scale == 0) scale = 1;
            scales[s] = scale;
            for (int j = 0; j < sp->sg; j++) {
                int64_t i = st + j;
                int best = 0; float best_err = 1e30f;
                if (i < n) {
                    float target = w[i] / scale;
                    for (int c = 0; c < 16; c++) {
                        float e = abs32(IQ4NL_GRID[c] - target);
                        if (e < best_err) { best_err = e; best = c; }
                    }
                }
                bw_write(&bw, (uint32_t)best, 4);
            }
            continue;
        }
        float amax = max_abs_range(w, st, en);
        float scale;
        if (sp->bits == 1) scale = amax;
        else {
            float denom = (float)qmax - sp->mid;
            if (denom < 1) denom = 1;
            scale = amax / denom;
        }
        if (scale == 0) scale = 1;
        scales[s] = scale;
        for (int j = 0; j < sp->sg; j++) {
            int64_t i = st + j;
            long q = 0;
            if (i < n) {
                if (sp->bits == 1) q = w[i] >= 0 ? 1 : 0;
                else q = clamp_l(round_to_int((double)w[i] / (double)scale + (double)sp->mid), 0, qmax);
            }
            bw_write(&bw, (uint32_t)q, sp->bits);
        }
    }
    meta[0] = (uint8_t)sp->bits; meta[1] = (uint8_t)sp->sg;
}

/* packTernary (quant/ternary.go:11-51): per-16 absMean scale, 2-bit codes. */
static void pack_ternary(const float *w, int64_t n, uint8_t *raw, float *scales) {
    int64_t ng = (n + 15) / 16;
    for (int64_t g = 0; g < ng; g++) {
        int64_t s = g * 16, e = s + 16 < n ? s + 16 : n;
        float scale = abs_mean(w, s, e);
        if (scale == 0) scale = 1;
        scales[g] = scale;
        uint32_t word = 0;
        for (int j = 0; j < 16; j++) {
            int64_t i = s + j;
            uint32_t code = 1;
            if (i < n) { long q = clamp_l(round_to_int((double)(w[i] / scale)), -1, 1); code = (uint32_t)(q + 1); }
            word |= (code & 3u) << (j * 2);
        }
        put_u32(raw + g * 4, word);
    }
}

/* packBinary (quant/binary.go:11-47): per-32 absMean scale, bit = w >= 0. */
static void pack_binary(const float *w, int64_t n, uint8_t *raw, float *scales) {
    int64_t ng = (n + 31) / 32;
    for (int64_t g = 0; g < ng; g++) {
        int64_t s = g * 32, e = s + 32 < n ? s + 32 : n;
        float scale = abs_mean(w, s, e);
        if (scale == 0) scale = 1;
        scales[g] = scale;
        uint32_t word = 0;
        for (int j = 0; j < 32; j++) { int64_t i = s + j; if (i < n && w[i] >= 0) word |= 1u << j; }
        put_u32(raw + g * 4, word);
    }
}

/* PackAffine4 (affine_pack.go:15-86) with group g: per group min/max in f32,
 * s = (max - min)/15 (s == 0, NaN or Inf → s = 1, min = 0), code =
 * round(f64(f32((v - min) * f32(1/s)))) half away, clamped to [0, 15], eight
 * codes per little-endian u32 LSB-first; scales = s, mins = min, meta = {4}
 * (BlobFromMLXAffine4, affine_g64.go:22-78). */
static void pack_affine(const float *w, int64_t rows, int64_t cols, int g, uint8_t *raw, float *scales, float *mins,
                        uint8_t *meta) {
    const float levels = 15.0f;
    int64_t gpr = cols / g;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t gi = 0; gi < gpr; gi++) {
            const float *v = w + r * cols + gi * g;
            float mn = v[0], mx = v[0];
            for (int j = 1; j < g; j++) {
                if (v[j] < mn) mn = v[j];
                if (v[j] > mx) mx = v[j];
            }
            float sc = (mx - mn) / levels;
            if (sc == 0 || isnan(sc) || isinf(sc)) { sc = 1; mn = 0; }
            scales[r * gpr + gi] = sc;
            mins[r * gpr + gi] = mn;
            float inv = 1 / sc;
            for (int wi = 0; wi < g / 8; wi++) {
                uint32_t word = 0;
                for (int j = 0; j < 8; j++) {
                    float t = (v[wi * 8 + j] - mn) * inv;
                    long code = clamp_l(round_to_int((double)t), 0, 15);
                    word |= (uint32_t)code << (4 * j);
                }
                put_u32(raw + ((r * cols + gi * g) / 8 + wi) * 4, word);
            }
        }
    }
    meta[0] = 4;
}

int or_pack(int fmt, const float *w, int64_t rows, int64_t cols,
            uint8_t *raw, float *scales, float *mins, uint8_t *meta) {
    int64_t sz[5];
    if (or_pack_sizes(fmt, rows, cols, sz) != 0) return -1;
    int64_t n = rows * cols;
    memset(raw, 0, (size_t)sz[0]);
    kspec_t ks; iqspec_t is;
    switch (fmt) {
    case OR_Q4_0: pack_q4_0(w, n, raw); return 0;
    case OR_Q8_0: pack_q8_0(w, n, raw); return 0;
    case OR_Q4_1: pack_q4_1(w, n, raw); return 0;
    case OR_Q5_0: pack_q5_0(w, n, raw); return 0;
    case OR_Q5_1: pack_q5_1(w, n, raw); return 0;
    case OR_TERNARY: pack_ternary(w, n, raw, scales); return 0;
    case OR_BINARY: pack_binary(w, n, raw, scales); return 0;
    case OR_AFFINE: pack_affine(w, rows, cols, 64, raw, scales, mins, meta); return 0;
    default: break;
    }
    if (kspec_for(fmt, &ks)) { pack_k(&ks, w, n, raw); return 0; }
    if (iqspec_for(fmt, &is)) { pack_iq(&is, w, n, raw, scales, meta); return 0; }
    return -1;
}

/* ------------------------------------------------------------------ */
/* decoders: one callback per (flat index, weight) in the reference's  */
/* walk order, shared by Unpack / MatVec / MatVecT                     */
/* ------------------------------------------------------------------ */

typedef struct {
    int fmt; int64_t rows, cols; int32_t bw;
    const uint8_t *raw; int64_t raw_len;
    const float *scales; int64_t ns;
    const float *mins; int64_t nm;
    const uint8_t *meta; int64_t nmeta;
} blob_t;

typedef void (*visit_fn)(void *ctx, int64_t i, float w);

/* decodeKWeight (quant/kquant.go:178-188). */
static float decode_k_weight(float d, float dmin, uint8_t su, uint8_t mu, uint32_t q, const kspec_t *sp) {
    float sc = d * (float)su / 255;
    if (sc == 0) sc = d / 255;
    if (sp->has_dmin) {
        float mn = dmin * (float)(int8_t)mu / 127;
        return mn + (float)q * sc;
    }
    return sc * (float)((int)q - sp->mid);
}

/* iqDequant (quant/iq.go:169-180). */
static float iq_dequant(const iqspec_t *sp, float scale, uint32_t q) {
    if (sp->nonlinear) return scale * IQ4NL_GRID[q & 15];
    if (sp->bits == 1) return (q & 1) ? scale : -scale;
    return scale * ((float)q - sp->mid);
}

static int is_g128(const blob_t *b) { return b->fmt == OR_BINARY && b->bw == 128; }

static int walk(const blob_t *b, visit_fn fn, void *ctx) {
    int64_t n = b->rows * b->cols;
    kspec_t ks; iqspec_t is;
    switch (b->fmt) {
    case OR_Q4_0: { /* matVecQ4_0 (q4_0.go:81-111) */
        int64_t blocks = b->raw_len / 20;
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = b->raw + bi * 20;
            float scale = get_f32(o);
            for (int j = 0; j < 16; j++) {
                int q1 = o[4 + j] & 0xF, q2 = o[4 + j] >> 4;
                if (q1 > 7) q1 -= 16;
                if (q2 > 7) q2 -= 16;
                int64_t i = bi * 32 + 2 * j;
                if (i < n) fn(ctx, i, (float)q1 * scale);
                if (i + 1 < n) fn(ctx, i + 1, (float)q2 * scale);
            }
        }
        return 0;
    }
    case OR_Q8_0: { /* matVecQ8_0 (q8_0.go:68-87) */
        int64_t blocks = b->raw_len / 36;
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = b->raw + bi * 36;
            float scale = get_f32(o);
            for (int j = 0; j < 32; j++) {
                int64_t i = bi * 32 + j;
                if (i >= n) break;
                fn(ctx, i, (float)(int8_t)o[4 + j] * scale);
            }
        }
        return 0;
    }
    case OR_Q4_1: { /* matVecQ4_1 (q4_1.go:78-102): w = mn + q*scale */
        int64_t blocks = b->raw_len / 24;
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = b->raw + bi * 24;
            float scale = get_f32(o), mn = get_f32(o + 4);
            for (int j = 0; j < 16; j++)
                for (int k = 0; k < 2; k++) {
                    int64_t i = bi * 32 + 2 * j + k;
                    if (i >= n) break;
                    int q = (o[8 + j] >> (4 * k)) & 0xF;
                    fn(ctx, i, mn + (float)q * scale);
                }
        }
        return 0;
    }
    case OR_Q5_0: { /* matVecQ5_0 (q5_0.go:68-89) */
        int64_t blocks = b->raw_len / 24;
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = b->raw + bi * 24;
            float scale = get_f32(o);
            bitr_t br = {o + 4, 20, 0};
            for (int j = 0; j < 32; j++) {
                int q = (int)br_read(&br, 5) - 16;
                int64_t i = bi * 32 + j;
                if (i < n) fn(ctx, i, (float)q * scale);
            }
        }
        return 0;
    }
    case OR_Q5_1: { /* matVecQ5_1 (q5_1.go:72-94) */
        int64_t blocks = b->raw_len / 28;
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = b->raw + bi * 28;
            float scale = get_f32(o), mn = get_f32(o + 4);
            bitr_t br = {o + 8, 20, 0};
            for (int j = 0; j < 32; j++) {
                int q = (int)br_read(&br, 5);
                int64_t i = bi * 32 + j;
                if (i < n) fn(ctx, i, mn + (float)q * scale);
            }
        }
        return 0;
    }
    case OR_TERNARY: { /* forEachTernary (ternary.go:64-82) */
        int64_t ng = b->raw_len / 4;
        for (int64_t g = 0; g < ng; g++) {
            uint32_t word = get_u32(b->raw + g * 4);
            float scale = g < b->ns ? b->scales[g] : 1.0f;
            for (int j = 0; j < 16; j++) {
                int64_t i = g * 16 + j;
                if (i >= n) break;
                uint32_t c = (word >> (2 * j)) & 3u;
                fn(ctx, i, c == 0 ? -scale : (c == 2 ? scale : 0.0f));
            }
        }
        return 0;
    }
    case OR_BINARY: {
        if (is_g128(b)) { /* forEachBinaryG128 (binary_g128.go:107-139) */
            int64_t gpr = b->cols / 128, wpr = b->cols / 32;
            for (int64_t r = 0; r < b->rows; r++)
                for (int64_t g = 0; g < gpr; g++) {
                    int64_t si = r * gpr + g;
                    float scale = si < b->ns ? b->scales[si] : 1.0f;
                    for (int wi = 0; wi < 4; wi++) {
                        int64_t woff = (r * wpr + g * 4 + wi) * 4;
                        if (woff + 4 > b->raw_len) return 0;
                        uint32_t word = get_u32(b->raw + woff);
                        int64_t base = r * b->cols + g * 128 + wi * 32;
                        for (int j = 0; j < 32; j++) {
                            int64_t i = base + j;
                            if (i >= n) return 0;
                            fn(ctx, i, ((word >> j) & 1u) ? scale : -scale);
                        }
                    }
                }
            return 0;
        }
        /* forEachBinary (binary.go:49-75) */
        int64_t ng = b->raw_len / 4;
        for (int64_t g = 0; g < ng; g++) {
            uint32_t word = get_u32(b->raw + g * 4);
            float scale = g < b->ns ? b->scales[g] : 1.0f;
            for (int j = 0; j < 32; j++) {
                int64_t i = g * 32 + j;
                if (i >= n) break;
                fn(ctx, i, ((word >> j) & 1u) ? scale : -scale);
            }
        }
        return 0;
    }
    default: break;
    }
    if (kspec_for(b->fmt, &ks)) { /* forEachK (kquant.go:190-228) */
        int64_t sbb = ksuper_bytes(&ks), sbs = b->raw_len / sbb;
        for (int64_t si = 0; si < sbs; si++) {
            const uint8_t *o = b->raw + si * sbb;
            float d = get_f32(o), dmin = get_f32(o + 4);
            const uint8_t *sc = o + 8;
            const uint8_t *mins = ks.has_dmin ? o + 24 : NULL;
            int64_t qoff = ks.has_dmin ? 40 : 24;
            bitr_t br = {o + qoff, sbb - qoff, 0};
            for (int g = 0; g < 16; g++) {
                uint8_t mu = mins ? mins[g] : 0;
                for (int j = 0; j < 16; j++) {
                    int64_t i = si * 256 + g * 16 + j;
                    uint32_t q = br_read(&br, ks.bits);
                    if (i >= n) continue;
                    fn(ctx, i, decode_k_weight(d, dmin, sc[g], mu, q, &ks));
                }
            }
        }
        return 0;
    }
    if (b->fmt == OR_AFFINE) { /* decodeRowAffine (affine_g64.go:124-161): w = f32(s*code) + beta */
        int bits = b->nmeta > 0 && b->meta[0] > 0 ? b->meta[0] : 4;
        int g = b->bw > 0 ? b->bw : 64, cpw = 32 / bits;
        if (bits != 4 || b->cols % g || g % cpw) return -1;
        int64_t wpr = b->cols / cpw, gpr = b->cols / g;
        uint32_t mask = (1u << bits) - 1;
        for (int64_t r = 0; r < b->rows; r++)
            for (int64_t gi = 0; gi < gpr; gi++) {
                int64_t si = r * gpr + gi;
                float sc = si < b->ns ? b->scales[si] : 1, beta = si < b->nm ? b->mins[si] : 0;
                for (int wi = 0; wi < g / cpw; wi++) {
                    uint32_t word = get_u32(b->raw + (r * wpr + gi * (g / cpw) + wi) * 4);
                    for (int j = 0; j < cpw; j++) {
                        float code = (float)((word >> (j * bits)) & mask);
                        fn(ctx, r * b->cols + gi * g + wi * cpw + j, sc * code + beta);
                    }
                }
            }
        return 0;
    }
    if (iqspec_for(b->fmt, &is)) { /* forEachIQ (iq.go:182-207) */
        if (b->nmeta >= 2) { is.bits = b->meta[0]; is.sg = b->meta[1]; }
        bitr_t br = {b->raw, b->raw_len, 0};
        for (int64_t s = 0; s < b->ns; s++) {
            float scale = b->scales[s];
            for (int j = 0; j < is.sg; j++) {
                uint32_t q = br_read(&br, is.bits);
                int64_t i = s * is.sg + j;
                if (i >= n) continue;
                fn(ctx, i, iq_dequant(&is, scale, q));
            }
        }
        return 0;
    }
    return -1;
}

static void visit_store(void *ctx, int64_t i, float w) { ((float *)ctx)[i] = w; }

typedef struct { const blob_t *b; const float *x; float *y; } mv_ctx;
static void visit_mv(void *ctx, int64_t i, float w) {
    mv_ctx *c = (mv_ctx *)ctx;
    c->y[i / c->b->cols] += w * c->x[i % c->b->cols];
}
static void visit_mvt(void *ctx, int64_t i, float w) {
    mv_ctx *c = (mv_ctx *)ctx;
    c->y[i % c->b->cols] += w * c->x[i / c->b->cols];
}

int or_unpack(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t *raw, int64_t raw_len,
              const float *scales, int64_t ns, const float *mins, int64_t nm, const uint8_t *meta, int64_t nmeta,
              float *out) {
    blob_t b = {fmt, rows, cols, bw, raw, raw_len, scales, ns, mins, nm, meta, nmeta};
    memset(out, 0, (size_t)(rows * cols) * sizeof(float));
    return walk(&b, visit_store, out);
}

/* matVecBinaryG128 (binary_g128.go:159-239): exact-float ±s form,
 * acc += s*(2*sum1 - sumAll) with sumAll per 32-word via 4 partial sums. */
static float g128_sum32(const float *x) {
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    for (int i = 0; i < 32; i += 4) { s0 += x[i]; s1 += x[i + 1]; s2 += x[i + 2]; s3 += x[i + 3]; }
    return s0 + s1 + s2 + s3;
}
static void matvec_g128(const blob_t *b, const float *x, float *y) {
    int64_t gpr = b->cols / 128, wpr = b->cols / 32;
    float *sum_all = (float *)malloc((size_t)wpr * sizeof(float));
    for (int64_t w = 0; w < wpr; w++) sum_all[w] = g128_sum32(x + w * 32);
    for (int64_t r = 0; r < b->rows; r++) {
        float acc = 0;
        for (int64_t g = 0; g < gpr; g++) {
            float scale = b->scales[r * gpr + g];
            for (int wi = 0; wi < 4; wi++) {
                uint32_t word = get_u32(b->raw + (r * wpr + g * 4 + wi) * 4);
                const float *xs = x + g * 128 + wi * 32;
                float sum1 = 0;
                for (int j = 0; j < 32; j++) sum1 += xs[j] * (float)((word >> j) & 1u);
                acc += scale * (2 * sum1 - sum_all[g * 4 + wi]);
            }
        }
        y[r] = acc;
    }
    free(sum_all);
}

/* matVecAffine (affine_g64.go:178-267): f32 sumX per group (sequential),
 * per group f32 codeDot = sum code*x, acc += s*codeDot + beta*sumX[g]. */
static int matvec_affine(const blob_t *b, const float *x, float *y) {
    int bits = b->nmeta > 0 && b->meta[0] > 0 ? b->meta[0] : 4;
    int g = b->bw > 0 ? b->bw : 64, cpw = 32 / bits;
    if (bits != 4 || b->cols % g || g % cpw) return -1;
    int64_t wpr = b->cols / cpw, gpr = b->cols / g;
    uint32_t mask = (1u << bits) - 1;
    float *sum_x = (float *)malloc((size_t)gpr * sizeof(float));
    for (int64_t gi = 0; gi < gpr; gi++) {
        float s = 0;
        for (int j = 0; j < g; j++) s += x[gi * g + j];
        sum_x[gi] = s;
    }
    for (int64_t r = 0; r < b->rows; r++) {
        float acc = 0;
        for (int64_t gi = 0; gi < gpr; gi++) {
            float sc = b->scales[r * gpr + gi], beta = b->mins[r * gpr + gi], code_dot = 0;
            for (int wi = 0; wi < g / cpw; wi++) {
                uint32_t word = get_u32(b->raw + (r * wpr + gi * (g / cpw) + wi) * 4);
                const float *xb = x + gi * g + wi * cpw;
                for (int j = 0; j < cpw; j++) code_dot += (float)((word >> (j * bits)) & mask) * xb[j];
            }
            acc += sc * code_dot + beta * sum_x[gi];
        }
        y[r] = acc;
    }
    free(sum_x);
    return 0;
}

/* matVecTAffine (affine_g64.go:269-286): rows with gy == 0 are skipped,
 * otherwise gx[j] += w[r][j] * gy[r] over the decoded row. */
typedef struct { const blob_t *b; const float *gy; float *gx; } mvt_aff_ctx;
static void visit_mvt_affine(void *ctx, int64_t i, float w) {
    mvt_aff_ctx *c = (mvt_aff_ctx *)ctx;
    float g = c->gy[i / c->b->cols];
    if (g != 0) c->gx[i % c->b->cols] += w * g;
}

int or_matvec_scalar(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t *raw, int64_t raw_len,
                     const float *scales, int64_t ns, const float *mins, int64_t nm, const uint8_t *meta,
                     int64_t nmeta, const float *x, float *y) {
    blob_t b = {fmt, rows, cols, bw, raw, raw_len, scales, ns, mins, nm, meta, nmeta};
    if (is_g128(&b)) { matvec_g128(&b, x, y); return 0; }
    if (fmt == OR_AFFINE) return matvec_affine(&b, x, y);
    for (int64_t r = 0; r < rows; r++) y[r] = 0;
    mv_ctx c = {&b, x, y};
    return walk(&b, visit_mv, &c);
}

int or_matvec_t_scalar(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t *raw, int64_t raw_len,
                       const float *scales, int64_t ns, const float *mins, int64_t nm, const uint8_t *meta,
                       int64_t nmeta, const float *gy, float *gx) {
    blob_t b = {fmt, rows, cols, bw, raw, raw_len, scales, ns, mins, nm, meta, nmeta};
    if (fmt == OR_AFFINE) {
        mvt_aff_ctx c = {&b, gy, gx};
        return walk(&b, visit_mvt_affine, &c);
    }
    mv_ctx c = {&b, gy, gx};
    return walk(&b, visit_mvt, &c);
}

void or_gemv_f64(const float *w, int64_t rows, int64_t cols, const float *x, double *y) {
    for (int64_t r = 0; r < rows; r++) {
        long double s = 0;
        const float *wr = w + r * cols;
        for (int64_t c = 0; c < cols; c++) s += (long double)wr[c] * (long double)x[c];
        y[r] = (double)s;
    }
}

/* ------------------------------------------------------------------ */
/* fused SIMD path (CPU baseline)                                      */
/* ------------------------------------------------------------------ */

typedef struct {
    int fmt; int64_t rows, cols;
    /* projections (Ensure*SIMDCache) */
    float *scales;      /* per block / group */
    float *mins;        /* per block / group (asymmetric) */
    int8_t *qs;         /* Int8QS, one per weight */
    uint32_t *q4;       /* Q4Packed words (Q4_0 / Q4_1) */
    float *f32;         /* F32Cache (Ternary/Binary g32) */
    int has_dmin, mid, sg, iq_kind; float iq_mid;
    blob_t g128;        /* BinaryG128 keeps the packed form */
    uint8_t *g128_raw; float *g128_scales;
} simd_t;

/* DotQ4_0 block (dot_q4_amd64.s:24-102 semantics): f64 sum of x*q over a
 * 32-block times the block scale. AVX2: nibbles → int32 → f64 FMAs. */
static inline double q4_block_dot_avx2(const float *x, const uint32_t *pk, float scale) {
    __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd();
    for (int w = 0; w < 4; w++) {
        uint32_t word = pk[w];
        int32_t q[8];
        for (int k = 0; k < 8; k++) { int v = (word >> (4 * k)) & 0xF; q[k] = v > 7 ? v - 16 : v; }
        __m256i qi = _mm256_loadu_si256((const __m256i *)q);
        __m128i qlo = _mm256_castsi256_si128(qi), qhi = _mm256_extracti128_si256(qi, 1);
        __m256d ql = _mm256_cvtepi32_pd(qlo), qh = _mm256_cvtepi32_pd(qhi);
        __m256d xl = _mm256_cvtps_pd(_mm_loadu_ps(x + 8 * w)), xh = _mm256_cvtps_pd(_mm_loadu_ps(x + 8 * w + 4));
        a0 = _mm256_fmadd_pd(xl, ql, a0);
        a1 = _mm256_fmadd_pd(xh, qh, a1);
    }
    __m256d s = _mm256_add_pd(a0, a1);
    __m128d h = _mm_add_pd(_mm256_castpd256_pd128(s), _mm256_extractf128_pd(s, 1));
    double r = _mm_cvtsd_f64(_mm_add_sd(h, _mm_unpackhi_pd(h, h)));
    return r * (double)scale;
}

/* q8BlockDot32Avx2 semantics (dot_qx_amd64.s:11-61): f64 Σ x*q times scale. */
static inline double q8_block_dot_avx2(const float *x, const int8_t *q, float scale) {
    __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd();
    for (int k = 0; k < 32; k += 8) {
        __m128i qb = _mm_loadl_epi64((const __m128i *)(q + k));
        __m256i qi = _mm256_cvtepi8_epi32(qb);
        __m256d ql = _mm256_cvtepi32_pd(_mm256_castsi256_si128(qi)), qh = _mm256_cvtepi32_pd(_mm256_extracti128_si256(qi, 1));
        __m256d xl = _mm256_cvtps_pd(_mm_loadu_ps(x + k)), xh = _mm256_cvtps_pd(_mm_loadu_ps(x + k + 4));
        a0 = _mm256_fmadd_pd(xl, ql, a0);
        a1 = _mm256_fmadd_pd(xh, qh, a1);
    }
    __m256d s = _mm256_add_pd(a0, a1);
    __m128d h = _mm_add_pd(_mm256_castpd256_pd128(s), _mm256_extractf128_pd(s, 1));
    return _mm_cvtsd_f64(_mm_add_sd(h, _mm_unpackhi_pd(h, h))) * (double)scale;
}

/* q41BlockDot32Avx2 semantics (dot_qx_amd64.s:65-141): scale*Σx*q + min*Σx. */
static inline double q41_block_dot_avx2(const float *x, const uint32_t *pk, float scale, float mn) {
    __m256d aq = _mm256_setzero_pd(), ax = _mm256_setzero_pd();
    for (int w = 0; w < 4; w++) {
        uint32_t word = pk[w];
        int32_t q[8];
        for (int k = 0; k < 8; k++) q[k] = (word >> (4 * k)) & 0xF;
        __m256i qi = _mm256_loadu_si256((const __m256i *)q);
        __m256d ql = _mm256_cvtepi32_pd(_mm256_castsi256_si128(qi)), qh = _mm256_cvtepi32_pd(_mm256_extracti128_si256(qi, 1));
        __m256d xl = _mm256_cvtps_pd(_mm_loadu_ps(x + 8 * w)), xh = _mm256_cvtps_pd(_mm_loadu_ps(x + 8 * w + 4));
        aq = _mm256_fmadd_pd(xl, ql, aq); aq = _mm256_fmadd_pd(xh, qh, aq);
        ax = _mm256_add_pd(ax, xl); ax = _mm256_add_pd(ax, xh);
    }
    double t[4], u[4];
    _mm256_storeu_pd(t, aq); _mm256_storeu_pd(u, ax);
    return ((t[0] + t[2]) + (t[1] + t[3])) * (double)scale + ((u[0] + u[2]) + (u[1] + u[3])) * (double)mn;
}

/* dotF32AccF64Avx2 semantics (avx2_amd64.s:14-79): f32·f32 with f64 accumulation. */
static double dot_tile_f64(const float *x, const float *w, int64_t n) {
    __m256d a0 = _mm256_setzero_pd(), a1 = _mm256_setzero_pd();
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        a0 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(x + i)), _mm256_cvtps_pd(_mm_loadu_ps(w + i)), a0);
        a1 = _mm256_fmadd_pd(_mm256_cvtps_pd(_mm_loadu_ps(x + i + 4)), _mm256_cvtps_pd(_mm_loadu_ps(w + i + 4)), a1);
    }
    __m256d s = _mm256_add_pd(a0, a1);
    __m128d h = _mm_add_pd(_mm256_castpd256_pd128(s), _mm256_extractf128_pd(s, 1));
    double r = _mm_cvtsd_f64(_mm_add_sd(h, _mm_unpackhi_pd(h, h)));
    for (; i < n; i++) r += (double)x[i] * (double)w[i];
    return r;
}

/* DotKRow (simd/dot_k.go:25-74), pure Go in the reference: scalar f64. */
static double dot_k_row(const float *in, const float *scales, const float *mins, const int8_t *qs,
                        int64_t basew, int64_t n, int has_dmin, int mid) {
    double sum = 0;
    int64_t i = 0;
    if (basew % 16 == 0) {
        for (; i + 16 <= n; i += 16) {
            int64_t g = (basew + i) / 16, off = basew + i;
            double sc = scales[g];
            if (has_dmin) {
                double mn = mins[g], accq = 0, sumx = 0;
                for (int j = 0; j < 16; j++) { double xi = in[i + j]; accq += xi * (double)(uint8_t)qs[off + j]; sumx += xi; }
                sum += accq * sc + mn * sumx;
            } else {
                double acc = 0;
                for (int j = 0; j < 16; j++) acc += (double)in[i + j] * (double)((int)(uint8_t)qs[off + j] - mid);
                sum += acc * sc;
            }
        }
    }
    for (; i < n; i++) {
        int64_t g = (basew + i) / 16;
        int q = (uint8_t)qs[basew + i];
        if (has_dmin) sum += (double)in[i] * ((double)mins[g] + (double)q * (double)scales[g]);
        else sum += (double)in[i] * (double)scales[g] * (double)(q - mid);
    }
    return sum;
}

/* DotIQRow (simd/dot_k.go:78-136): scalar f64. */
static double dot_iq_row(const float *in, const float *scales, const int8_t *qs, int64_t basew, int64_t n,
                         int sg, float mid, int kind) {
    double sum = 0;
    int64_t i = 0;
    if (basew % sg == 0) {
        for (; i + sg <= n; i += sg) {
            double sc = scales[(basew + i) / sg], acc = 0;
            int64_t off = basew + i;
            for (int j = 0; j < sg; j++) {
                uint8_t q = (uint8_t)qs[off + j];
                double code = kind == 1 ? ((q & 1) ? 1.0 : -1.0) : kind == 2 ? (double)IQ4NL_GRID[q & 15] : ((double)q - (double)mid);
                acc += (double)in[i + j] * code;
            }
            sum += acc * sc;
        }
    }
    for (; i < n; i++) {
        double sc = scales[(basew + i) / sg];
        uint8_t q = (uint8_t)qs[basew + i];
        double code = kind == 1 ? ((q & 1) ? 1.0 : -1.0) : kind == 2 ? (double)IQ4NL_GRID[q & 15] : ((double)q - (double)mid);
        sum += (double)in[i] * code * sc;
    }
    return sum;
}

/* DotQ5_1Row (simd/dot_qx.go:134-166): scalar f64. */
static double dot_q5_1_row(const float *in, const float *scales, const float *mins, const int8_t *qs,
                           int64_t basew, int64_t n) {
    double sum = 0;
    int64_t i = 0;
    if (basew % 32 == 0) {
        for (; i + 32 <= n; i += 32) {
            int64_t blk = (basew + i) / 32, off = basew + i;
            double sc = scales[blk], mn = mins[blk], accq = 0, sumx = 0;
            for (int j = 0; j < 32; j++) { double xi = in[i + j]; accq += xi * (double)(uint8_t)qs[off + j]; sumx += xi; }
            sum += accq * sc + mn * sumx;
        }
    }
    for (; i < n; i++) {
        int64_t blk = (basew + i) / 32;
        sum += (double)in[i] * ((double)mins[blk] + (double)(uint8_t)qs[basew + i] * (double)scales[blk]);
    }
    return sum;
}

static double q4_0_row_tail(const float *in, const float *scales, const uint32_t *pk, int64_t basew, int64_t i0, int64_t n) {
    double sum = 0;
    for (int64_t i = i0; i < n; i++) {
        int64_t gi = basew + i;
        int q = (pk[gi / 8] >> ((gi % 8) * 4)) & 0xF;
        if (q > 7) q -= 16;
        sum += (double)in[i] * (double)q * (double)scales[gi / 32];
    }
    return sum;
}

/* DotAffineRow (simd/dot_k.go:140-165): per group f64 accQ = sum x*code,
 * sum += accQ*s + beta*f64(sumX[g]) with the f32 group sums of AffineSumX. */
static double dot_affine_row(const float *in, const float *scales, const float *mins, const float *sum_x,
                             const int8_t *qs, int64_t basew, int64_t n, int g, int64_t scale_base) {
    double sum = 0;
    for (int64_t gi = 0; gi < n / g; gi++) {
        double sc = scales[scale_base + gi], beta = mins[scale_base + gi], accq = 0;
        for (int j = 0; j < g; j++) accq += (double)in[gi * g + j] * (double)(uint8_t)qs[basew + gi * g + j];
        sum += accq * sc + beta * (double)sum_x[gi];
    }
    return sum;
}

/* One output row of the fused path for any projected format (sum_x: the
 * AffineSumX group sums of x, for AffinePacked). */
static float simd_row(const simd_t *s, const float *x, int64_t o, const float *sum_x) {
    int64_t in = s->cols, basew = o * in;
    switch (s->fmt) {
    case OR_Q4_0: { /* dotQ4_0RowSimd (dot_q4_amd64.go:8-22) */
        double sum = 0; int64_t i = 0;
        if (basew % 32 == 0) for (; i + 32 <= in; i += 32) sum += q4_block_dot_avx2(x + i, s->q4 + (basew + i) / 8, s->scales[(basew + i) / 32]);
        if (i < in) sum += q4_0_row_tail(x, s->scales, s->q4, basew, i, in);
        return (float)sum;
    }
    case OR_Q8_0: case OR_Q5_0: { /* dotQ8_0RowSimd (dot_qx_amd64.go:11-25) */
        double sum = 0; int64_t i = 0;
        if (basew % 32 == 0) for (; i + 32 <= in; i += 32) sum += q8_block_dot_avx2(x + i, s->qs + basew + i, s->scales[(basew + i) / 32]);
        for (; i < in; i++) sum += (double)x[i] * (double)s->qs[basew + i] * (double)s->scales[(basew + i) / 32];
        return (float)sum;
    }
    case OR_Q4_1: {
        double sum = 0; int64_t i = 0;
        if (basew % 32 == 0) for (; i + 32 <= in; i += 32) sum += q41_block_dot_avx2(x + i, s->q4 + (basew + i) / 8, s->scales[(basew + i) / 32], s->mins[(basew + i) / 32]);
        for (; i < in; i++) {
            int64_t gi = basew + i, blk = gi / 32;
            double q = (double)((s->q4[gi / 8] >> ((gi % 8) * 4)) & 0xF);
            sum += (double)x[i] * ((double)s->mins[blk] + q * (double)s->scales[blk]);
        }
        return (float)sum;
    }
    case OR_Q5_1: return (float)dot_q5_1_row(x, s->scales, s->mins, s->qs, basew, in);
    case OR_AFFINE: return (float)dot_affine_row(x, s->scales, s->mins, sum_x, s->qs, basew, in, s->sg, o * (in / s->sg));
    case OR_TERNARY: return (float)dot_tile_f64(x, s->f32 + basew, in);
    case OR_BINARY: return (float)dot_tile_f64(x, s->f32 + basew, in);
    default: break;
    }
    kspec_t ks;
    if (kspec_for(s->fmt, &ks)) return (float)dot_k_row(x, s->scales, s->mins, s->qs, basew, in, s->has_dmin, s->mid);
    return (float)dot_iq_row(x, s->scales, s->qs, basew, in, s->sg, s->iq_mid, s->iq_kind);
}

void *or_simd_prepare(int fmt, int64_t rows, int64_t cols, int32_t bw, const uint8_t *raw, int64_t raw_len,
                      const float *scales, int64_t ns, const float *mins, int64_t nm, const uint8_t *meta,
                      int64_t nmeta) {
    simd_t *s = (simd_t *)calloc(1, sizeof(simd_t));
    s->fmt = fmt; s->rows = rows; s->cols = cols;
    int64_t n = rows * cols;
    kspec_t ks; iqspec_t is;
    blob_t b = {fmt, rows, cols, bw, raw, raw_len, scales, ns, mins, nm, meta, nmeta};
    if (fmt == OR_AFFINE) { /* EnsureAffineSIMDCache (k_iq_simd.go:187-240): codes to Int8QS */
        int g = bw > 0 ? bw : 64;
        int bits = nmeta > 0 && meta[0] > 0 ? meta[0] : 4;
        int64_t gpr = cols / g;
        if (bits != 4 || cols % g || ns < rows * gpr || nm < rows * gpr || raw_len < n / 2) { free(s); return NULL; }
        s->qs = (int8_t *)malloc((size_t)n);
        for (int64_t i = 0; i < n; i++) s->qs[i] = (int8_t)((raw[i / 2] >> (4 * (i & 1))) & 15);
        s->scales = (float *)malloc((size_t)ns * 4);
        s->mins = (float *)malloc((size_t)nm * 4);
        memcpy(s->scales, scales, (size_t)ns * 4);
        memcpy(s->mins, mins, (size_t)nm * 4);
        s->sg = g;
        return s;
    }
    if (fmt == OR_Q4_0 || fmt == OR_Q4_1) { /* EnsureQ4SIMDCache / EnsureQ41SIMDCache (q4_simd.go:7-35, qx_simd.go:34-65) */
        int bb = fmt == OR_Q4_0 ? 20 : 24, qo = fmt == OR_Q4_0 ? 4 : 8;
        int64_t blocks = (n + 31) / 32;
        s->scales = (float *)malloc((size_t)blocks * 4);
        s->mins = (float *)malloc((size_t)blocks * 4);
        s->q4 = (uint32_t *)malloc((size_t)blocks * 16);
        for (int64_t bi = 0; bi < blocks; bi++) {
            s->scales[bi] = get_f32(raw + bi * bb);
            s->mins[bi] = fmt == OR_Q4_1 ? get_f32(raw + bi * bb + 4) : 0;
            for (int k = 0; k < 4; k++) s->q4[bi * 4 + k] = get_u32(raw + bi * bb + qo + 4 * k);
        }
        return s;
    }
    if (fmt == OR_Q8_0 || fmt == OR_Q5_0 || fmt == OR_Q5_1) { /* qx_simd.go:6-31, 68-147 */
        int bb = fmt == OR_Q8_0 ? 36 : (fmt == OR_Q5_0 ? 24 : 28);
        int64_t blocks = (n + 31) / 32;
        s->scales = (float *)malloc((size_t)blocks * 4);
        s->mins = (float *)malloc((size_t)blocks * 4);
        s->qs = (int8_t *)malloc((size_t)blocks * 32);
        for (int64_t bi = 0; bi < blocks; bi++) {
            const uint8_t *o = raw + bi * bb;
            s->scales[bi] = get_f32(o);
            s->mins[bi] = fmt == OR_Q5_1 ? get_f32(o + 4) : 0;
            if (fmt == OR_Q8_0) { for (int j = 0; j < 32; j++) s->qs[bi * 32 + j] = (int8_t)o[4 + j]; continue; }
            bitr_t br = {o + (fmt == OR_Q5_0 ? 4 : 8), 20, 0};
            for (int j = 0; j < 32; j++) {
                int q = (int)br_read(&br, 5);
                s->qs[bi * 32 + j] = (int8_t)(fmt == OR_Q5_0 ? q - 16 : q);
            }
        }
        return s;
    }
    if (kspec_for(fmt, &ks)) { /* EnsureKSIMDCache (k_iq_simd.go:17-87) */
        int64_t sbb = ksuper_bytes(&ks), sbs = raw_len / sbb;
        s->scales = (float *)malloc((size_t)sbs * 16 * 4);
        s->mins = (float *)calloc((size_t)sbs * 16, 4);
        s->qs = (int8_t *)malloc((size_t)sbs * 256);
        for (int64_t si = 0; si < sbs; si++) {
            const uint8_t *o = raw + si * sbb;
            float d = get_f32(o), dmin = get_f32(o + 4);
            int64_t qoff = ks.has_dmin ? 40 : 24;
            bitr_t br = {o + qoff, sbb - qoff, 0};
            for (int g = 0; g < 16; g++) {
                float sc = d * (float)o[8 + g] / 255;
                if (sc == 0) sc = d / 255;
                s->scales[si * 16 + g] = sc;
                if (ks.has_dmin) s->mins[si * 16 + g] = dmin * (float)(int8_t)o[24 + g] / 127;
                for (int j = 0; j < 16; j++) s->qs[si * 256 + g * 16 + j] = (int8_t)br_read(&br, ks.bits);
            }
        }
        s->has_dmin = ks.has_dmin; s->mid = ks.mid;
        return s;
    }
    if (iqspec_for(fmt, &is)) { /* EnsureIQSIMDCache (k_iq_simd.go:108-154) */
        if (nmeta >= 2) { is.bits = meta[0]; is.sg = meta[1]; }
        int64_t padn = (n + is.sg - 1) / is.sg * is.sg;
        s->qs = (int8_t *)malloc((size_t)padn);
        bitr_t br = {raw, raw_len, 0};
        for (int64_t i = 0; i < padn; i++) s->qs[i] = (int8_t)br_read(&br, is.bits);
        s->scales = (float *)malloc((size_t)ns * 4);
        memcpy(s->scales, scales, (size_t)ns * 4);
        s->sg = is.sg; s->iq_mid = is.mid;
        s->iq_kind = is.bits == 1 ? 1 : (is.nonlinear ? 2 : 0);
        return s;
    }
    if (fmt == OR_TERNARY || (fmt == OR_BINARY && bw != 128)) { /* EnsureFloatCache (qx_simd.go:181-201) */
        s->f32 = (float *)malloc((size_t)n * 4);
        or_unpack(fmt, rows, cols, bw, raw, raw_len, scales, ns, mins, nm, meta, nmeta, s->f32);
        return s;
    }
    if (fmt == OR_BINARY && bw == 128) { /* native packed G128 (no inflate) */
        s->g128_raw = (uint8_t *)malloc((size_t)raw_len);
        memcpy(s->g128_raw, raw, (size_t)raw_len);
        s->g128_scales = (float *)malloc((size_t)ns * 4);
        memcpy(s->g128_scales, scales, (size_t)ns * 4);
        s->g128 = b; s->g128.raw = s->g128_raw; s->g128.scales = s->g128_scales;
        return s;
    }
    free(s);
    return NULL;
}

void or_simd_free(void *h) {
    simd_t *s = (simd_t *)h;
    if (!s) return;
    free(s->scales); free(s->mins); free(s->qs); free(s->q4); free(s->f32);
    free(s->g128_raw); free(s->g128_scales);
    free(s);
}

typedef struct { const simd_t *s; const float *x; float *y; int64_t lo, hi; } job_t;
static void *simd_worker(void *arg) {
    job_t *j = (job_t *)arg;
    const simd_t *s = j->s;
    int64_t o = j->lo;
    if (s->fmt == OR_Q4_0 || s->fmt == OR_Q8_0 || s->fmt == OR_Q5_0 || s->fmt == OR_Q4_1) {
        /* Rows4 (dot_q4_amd64.go:25-38, dot_qx_amd64.go:27-71): 4 rows share the x block. */
        if (s->cols % 32 == 0) {
            for (; o + 3 < j->hi; o += 4) {
                double acc[4] = {0, 0, 0, 0};
                for (int64_t i = 0; i < s->cols; i += 32)
                    for (int r = 0; r < 4; r++) {
                        int64_t bw = (o + r) * s->cols + i;
                        if (s->fmt == OR_Q4_0) acc[r] += q4_block_dot_avx2(j->x + i, s->q4 + bw / 8, s->scales[bw / 32]);
                        else if (s->fmt == OR_Q4_1) acc[r] += q41_block_dot_avx2(j->x + i, s->q4 + bw / 8, s->scales[bw / 32], s->mins[bw / 32]);
                        else acc[r] += q8_block_dot_avx2(j->x + i, s->qs + bw, s->scales[bw / 32]);
                    }
                for (int r = 0; r < 4; r++) j->y[o + r] = (float)acc[r];
            }
        }
    }
    float *sum_x = NULL;
    if (s->fmt == OR_AFFINE) { /* gemvAffineRowsF32 (gemv_parallel.go:331-339): AffineSumX per worker */
        int64_t gpr = s->cols / s->sg;
        sum_x = (float *)malloc((size_t)gpr * sizeof(float));
        for (int64_t gi = 0; gi < gpr; gi++) {
            float t = 0;
            for (int k = 0; k < s->sg; k++) t += j->x[gi * s->sg + k];
            sum_x[gi] = t;
        }
    }
    for (; o < j->hi; o++) j->y[o] = simd_row(s, j->x, o, sum_x);
    free(sum_x);
    return NULL;
}

int or_simd_matvec(void *h, const float *x, float *y, int batch, int nthreads) {
    simd_t *s = (simd_t *)h;
    if (!s) return -1;
    for (int bt = 0; bt < batch; bt++) {
        const float *xb = x + (int64_t)bt * s->cols;
        float *yb = y + (int64_t)bt * s->rows;
        if (s->g128_raw) { matvec_g128(&s->g128, xb, yb); continue; }
        int64_t out = s->rows;
        if (out < 64 || nthreads < 2) { job_t j = {s, xb, yb, 0, out}; simd_worker(&j); continue; }
        int w = nthreads > out ? (int)out : nthreads;
        int64_t chunk = (out + w - 1) / w;
        pthread_t th[512]; job_t jobs[512];
        int nt = 0;
        for (int k = 0; k < w && k < 512; k++) {
            int64_t lo = k * chunk, hi = lo + chunk < out ? lo + chunk : out;
            if (lo >= hi) break;
            jobs[nt] = (job_t){s, xb, yb, lo, hi};
            pthread_create(&th[nt], NULL, simd_worker, &jobs[nt]);
            nt++;
        }
        for (int k = 0; k < nt; k++) pthread_join(th[k], NULL);
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* DTypeTernary int8 path                                              */
/* ------------------------------------------------------------------ */

/* absMax (weights/native.go:1160-1169). */
void or_pack_native_ternary(const float *w, int64_t n, uint8_t *codes, float *scale_out) {
    float scale = 0;
    for (int64_t i = 0; i < n; i++) { float a = (float)fabs((double)w[i]); if (a > scale) scale = a; }
    if (scale == 0) scale = 1;
    memset(codes, 0, (size_t)((n + 3) / 4));
    for (int64_t i = 0; i < n; i++) {
        float r = w[i] / scale;
        int code = r > 0.5f ? 2 : (r < -0.5f ? 0 : 1);
        codes[i / 4] |= (uint8_t)(code << ((i % 4) * 2));
    }
    *scale_out = scale;
}

float or_quantize_acts_i8(const float *x, int64_t n, int8_t *xq) {
    float maxabs = 0;
    for (int64_t i = 0; i < n; i++) { float a = (float)fabs((double)x[i]); if (a > maxabs) maxabs = a; }
    float scale = maxabs / 127;
    if (scale == 0) scale = 1;
    for (int64_t i = 0; i < n; i++) {
        long q = (long)round((double)(x[i] / scale));
        if (q > 127) q = 127;
        if (q < -128) q = -128;
        xq[i] = (int8_t)q;
    }
    return scale;
}

/* dotI8AccI32Avx2 semantics (dot_i8_amd64.s:4-56): exact int32 Σ a*b. */
static int32_t dot_i8(const int8_t *a, const int8_t *b, int64_t n) {
    __m256i acc = _mm256_setzero_si256();
    int64_t i = 0;
    for (; i + 16 <= n; i += 16) {
        __m256i va = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a + i)));
        __m256i vb = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(b + i)));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(va, vb));
    }
    int32_t t[8];
    _mm256_storeu_si256((__m256i *)t, acc);
    int32_t s = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
    for (; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

int or_ternary_i8_forward(const uint8_t *codes, float scale, int64_t rows, int64_t cols,
                          const float *x, float *y, int32_t *acc, float *act_scale, int batch) {
    int64_t n = rows * cols;
    if (scale == 0) scale = 1;
    /* expandNarrowToI8 (layers/dense/simd.go:149-195), redone every call. */
    int8_t *wi8 = (int8_t *)malloc((size_t)n);
    for (int64_t i = 0; i < n; i++) wi8[i] = (int8_t)(((codes[i / 4] >> ((i % 4) * 2)) & 3) - 1);
    int8_t *xq = (int8_t *)malloc((size_t)cols);
    for (int bt = 0; bt < batch; bt++) {
        float as = or_quantize_acts_i8(x + (int64_t)bt * cols, cols, xq);
        if (act_scale) act_scale[bt] = as;
        for (int64_t o = 0; o < rows; o++) {
            int32_t a = dot_i8(xq, wi8 + o * cols, cols);
            if (acc) acc[(int64_t)bt * rows + o] = a;
            y[(int64_t)bt * rows + o] = (float)a * as * scale;  /* simd.go:142, left to right */
        }
    }
    free(xq); free(wi8);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Narrow weights.Store DTypes: Int8 (9), Int4 (14), Int2 (17),         */
/* Ternary (19), Binary (20) — core.DType values (core/dtype.go:23-34). */
/* ------------------------------------------------------------------ */

static int narrow_bits_of(int dt) {
    switch (dt) {
    case 9: return 8;
    case 14: return 4;
    case 17: case 19: return 2;
    case 20: return 1;
    default: return 0;
    }
}

/* clampI(math.Round(float64(f32)), lo, hi) (weights/native.go:1184-1192). */
static int round_clamp(float v, double lo, double hi) {
    double r = round((double)v);
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int)r;
}

/* packNative for the narrow DTypes: Int8 (weights/native.go:88-97),
 * packInt4 (:180-194), packInt2 (:218-230), packTernary (:249-269),
 * packBinary (:271-283). Returns the bits per code, 0 for other DTypes. */
int or_pack_native(int dt, const float *w, int64_t n, uint8_t *codes, float *scale_out) {
    const int bits = narrow_bits_of(dt);
    if (!bits || n <= 0) return 0;
    float amax = 0;
    for (int64_t i = 0; i < n; i++) { float a = (float)fabs((double)w[i]); if (a > amax) amax = a; }
    float scale = dt == 9 ? amax / 127 : (dt == 14 ? amax / 7 : amax);
    if (scale == 0) scale = 1;
    memset(codes, 0, (size_t)((n * bits + 7) / 8));
    for (int64_t i = 0; i < n; i++) {
        unsigned code;
        switch (dt) {
        case 9: code = (uint8_t)(int8_t)round_clamp(w[i] / scale, -128, 127); break;
        case 14: code = (unsigned)round_clamp(w[i] / scale, -8, 7) & 0xF; break;
        case 17: code = (unsigned)(round_clamp(w[i] / scale, -2, 1) + 2) & 3; break;
        case 19: { float r = w[i] / scale; code = r > 0.5f ? 2 : (r < -0.5f ? 0 : 1); break; }
        default: code = w[i] >= 0 ? 1 : 0; break;
        }
        const int64_t bit = i * bits;
        codes[bit >> 3] |= (uint8_t)(code << (bit & 7));
    }
    *scale_out = scale;
    return bits;
}

/* expandNarrowToI8 (layers/dense/simd.go:149-195); Int8 bytes as they are
 * (nativeInt8Weights, simd.go:506-511). */
int or_expand_narrow_i8(int dt, const uint8_t *codes, int64_t n, int8_t *out) {
    for (int64_t i = 0; i < n; i++) {
        int v;
        switch (dt) {
        case 9: v = (int8_t)codes[i]; break;
        case 14: { int q = (i % 2 == 0) ? (codes[i / 2] & 0xF) : (codes[i / 2] >> 4); v = q > 7 ? q - 16 : q; break; }
        case 17: v = ((codes[i / 4] >> ((i % 4) * 2)) & 3) - 2; break;
        case 19: v = ((codes[i / 4] >> ((i % 4) * 2)) & 3) - 1; break;
        case 20: v = (codes[i / 8] & (1 << (i % 8))) ? 1 : -1; break;
        default: return -1;
        }
        out[i] = (int8_t)v;
    }
    return 0;
}

/* forwardSIMDNarrowI8 / forwardSIMDInt8 (layers/dense/simd.go:130-147,
 * 303-326): expand (every call, as the reference), quantizeActsI8, DotI8Tile
 * per row, y = f32(acc) * actScale * scale. acc / act_scale may be NULL. */
int or_narrow_i8_forward(int dt, const uint8_t *codes, float scale, int64_t rows, int64_t cols,
                         const float *x, float *y, int32_t *acc, float *act_scale, int batch) {
    int64_t n = rows * cols;
    if (scale == 0) scale = 1;
    int8_t *wi8 = (int8_t *)malloc((size_t)n);
    if (or_expand_narrow_i8(dt, codes, n, wi8)) { free(wi8); return -1; }
    int8_t *xq = (int8_t *)malloc((size_t)cols);
    for (int bt = 0; bt < batch; bt++) {
        float as = or_quantize_acts_i8(x + (int64_t)bt * cols, cols, xq);
        if (act_scale) act_scale[bt] = as;
        for (int64_t o = 0; o < rows; o++) {
            int32_t a = dot_i8(xq, wi8 + o * cols, cols);
            if (acc) acc[(int64_t)bt * rows + o] = a;
            y[(int64_t)bt * rows + o] = (float)a * as * scale;
        }
    }
    free(xq); free(wi8);
    return 0;
}

/* weightAt (weights/decode.go:50-215) for the narrow DTypes: f32(q) * scale;
 * Ternary codes 0 / 2 -> -scale / +scale, 1 and 3 -> 0; Binary +-scale. */
int or_native_decode(int dt, const uint8_t *codes, float scale, int64_t n, float *out) {
    if (scale == 0) scale = 1;
    for (int64_t i = 0; i < n; i++) {
        switch (dt) {
        case 19: {
            int c = (codes[i / 4] >> ((i % 4) * 2)) & 3;
            out[i] = c == 0 ? -scale : (c == 2 ? scale : 0.0f);
            break;
        }
        case 20: out[i] = (codes[i / 8] & (1 << (i % 8))) ? scale : -scale; break;
        case 9: case 14: case 17: {
            int8_t q;
            if (dt == 9) q = (int8_t)codes[i];
            else if (dt == 14) { int v = (i % 2 == 0) ? (codes[i / 2] & 0xF) : (codes[i / 2] >> 4); q = (int8_t)(v > 7 ? v - 16 : v); }
            else q = (int8_t)(((codes[i / 4] >> ((i % 4) * 2)) & 3) - 2);
            out[i] = (float)q * scale;
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

int or_num_cpus(void) { return (int)sysconf(_SC_NPROCESSORS_ONLN); }
