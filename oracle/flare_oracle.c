/*
 * flare_oracle.c -- CPU restatement of flarellm's x86_64 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see flare_oracle.h).  Citations are
 * path:line into the reference checkout.  Build with -ffp-contract=off and
 * without -ffast-math: the reference (Rust) never contracts a*b+c.
 */
#include "flare_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Row-parallel threading (OpenMP).  Default 1 thread: the reference's
 * quantized x86 path is single-threaded.  Rows, heads and tensor blocks are
 * independent, and every row keeps its sequential order of operations, so the
 * results do not depend on the thread count. */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int or_get_threads(void) { return g_threads; }
/* Summation order of the float reductions (row sums of the matvecs, sums of
 * squares, f32 dots).  0 = the reference's sequential order (default).
 * 1 = pairwise (recursive halving): an equally valid order, used only to
 * measure how far two correct implementations that sum in different orders
 * drift apart on a model -- the yardstick for the GPU's tree-order kernels.
 * Not part of the restatement. */
static int g_order = 0;
void or_set_order(int order) { g_order = order ? 1 : 0; }

static float pairwise(const float *t, size_t n) {
    if (n <= 2) return n == 0 ? 0.0f : (n == 1 ? t[0] : t[0] + t[1]);
    size_t h = n / 2;
    return pairwise(t, h) + pairwise(t + h, n - h);
}

#define OR_PAR _Pragma("omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)")

#define Q8_BLK 32
#define Q8_BYTES 34
#define Q4K_VALS 256
#define Q4K_BYTES 144
#define Q6K_BYTES 210

static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Rust `f32 as i8`: saturating, NaN -> 0. */
static int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}
/* Rust f32::max / f32::min (IEEE maxNum/minNum). */
static float rmax(float a, float b) { return fmaxf(a, b); }

/* flare-core/src/model.rs:5302-5329 (f16_to_f32_inline); identical results to
 * flare-loader/src/quantize.rs:505-537 (f16_to_f32). */
float or_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, mant = bits & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return bits_f32(sign << 31);
        uint32_t e = exp, m = mant;
        while ((m & 0x400u) == 0) { m <<= 1; e -= 1u; }
        m &= 0x3FFu;
        return bits_f32((sign << 31) | ((113u + e) << 23) | (m << 13));
    }
    if (exp == 0x1F) return bits_f32((sign << 31) | (0xFFu << 23) | (mant << 13));
    return bits_f32((sign << 31) | ((exp + 112u) << 23) | (mant << 13));
}

/* IEEE binary32 -> binary16, round to nearest even.  The reference's f16 KV
 * store uses half::f16::from_f32 (flare-gpu/src/kv_cache.rs:132-133, crate
 * half 2.7.1, not vendored); this is the IEEE conversion that crate documents.
 * Pinned against numpy.float16 in the tests. */
uint16_t or_f32_to_f16_rne(float f) {
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0));
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_m = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

/* flare-loader/src/quantize.rs:189-197 */
void or_dequant_q8_0_block(const uint8_t *blk, float out[32]) {
    float scale = or_f16_to_f32(rd16(blk));
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)blk[2 + i] * scale;
}

/* flare-core/src/model.rs:8709-8719 (unpack_q4k_scales); same packing as
 * flare-loader/src/quantize.rs:400-406. */
void or_unpack_q4k_scales(const uint8_t *s, uint8_t sc[8], uint8_t mn[8]) {
    for (int i = 0; i < 4; i++) {
        sc[i] = s[i] & 0x3F;
        mn[i] = s[i + 4] & 0x3F;
        sc[i + 4] = (uint8_t)((s[i] >> 6) | ((s[i + 8] & 0x0F) << 2));
        mn[i + 4] = (uint8_t)((s[i + 4] >> 6) | ((s[i + 8] >> 4) << 2));
    }
}

/* flare-loader/src/quantize.rs:386-423 (flare nibble layout: low nibble of
 * qs[j] is weight j, high nibble is weight j+128). */
void or_dequant_q4k_block(const uint8_t *blk, float out[256]) {
    float d = or_f16_to_f32(rd16(blk));
    float dmin = or_f16_to_f32(rd16(blk + 2));
    uint8_t sc[8], mn[8];
    or_unpack_q4k_scales(blk + 4, sc, mn);
    const uint8_t *qs = blk + 16;
    for (int j = 0; j < 128; j++) {
        int b = j / 32;
        float lo = (float)(qs[j] & 0x0F), hi = (float)((qs[j] >> 4) & 0x0F);
        out[j] = d * (float)sc[b] * lo - dmin * (float)mn[b];
        out[j + 128] = d * (float)sc[b + 4] * hi - dmin * (float)mn[b + 4];
    }
}

/* flare-loader/src/quantize.rs:343-384 (llama.cpp Q6_K layout). */
void or_dequant_q6k_block(const uint8_t *blk, float out[256]) {
    const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
    float d = or_f16_to_f32(rd16(blk + 208));
    for (int half = 0; half < 2; half++) {
        int ql_off = half * 64, qh_off = half * 32, sc_off = half * 8, y_off = half * 128;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[ql_off + l] & 0xF) | ((qh[qh_off + l] & 3) << 4)) - 32;
            int q2 = (int)((ql[ql_off + l + 32] & 0xF) | (((qh[qh_off + l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[ql_off + l] >> 4) | (((qh[qh_off + l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[ql_off + l + 32] >> 4) | (((qh[qh_off + l] >> 6) & 3) << 4)) - 32;
            float sc1 = (float)(int8_t)scales[sc_off + is];
            float sc2 = (float)(int8_t)scales[sc_off + is + 2];
            float sc3 = (float)(int8_t)scales[sc_off + is + 4];
            float sc4 = (float)(int8_t)scales[sc_off + is + 6];
            out[y_off + l] = d * sc1 * (float)q1;
            out[y_off + l + 32] = d * sc2 * (float)q2;
            out[y_off + l + 64] = d * sc3 * (float)q3;
            out[y_off + l + 96] = d * sc4 * (float)q4;
        }
    }
}

/* flare-loader/src/gguf.rs:717-880 (dequantize_tensor), for the formats on the
 * hot path. `bpr` counts blocks of the format per row. */
int or_dequant_tensor(const uint8_t *data, int format, size_t rows, size_t bpr, float *out) {
    size_t nb = rows * bpr;
    switch (format) {
    case OR_F32: memcpy(out, data, nb * sizeof(float)); return 0;
    case OR_Q8_0: {
        OR_PAR
        for (size_t b = 0; b < nb; b++) or_dequant_q8_0_block(data + b * Q8_BYTES, out + b * 32);
        return 0;
    }
    case OR_Q4K: {
        OR_PAR
        for (size_t b = 0; b < nb; b++) or_dequant_q4k_block(data + b * Q4K_BYTES, out + b * 256);
        return 0;
    }
    case OR_Q6K: {
        OR_PAR
        for (size_t b = 0; b < nb; b++) or_dequant_q6k_block(data + b * Q6K_BYTES, out + b * 256);
        return 0;
    }
    }
    return -1;
}

/* flare-core/src/model.rs:5534-5571, x86 branch 5557-5570. */
void or_quantize_input_q8_0(const float *x, size_t n, float *scales, int8_t *q) {
    size_t blocks = n / Q8_BLK;
    for (size_t b = 0; b < blocks; b++) {
        const float *blk = x + b * Q8_BLK;
        float amax = 0.0f;
        for (int j = 0; j < Q8_BLK; j++) amax = rmax(amax, fabsf(blk[j]));
        float d = amax / 127.0f;
        float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
        scales[b] = d;
        for (int j = 0; j < Q8_BLK; j++) q[b * Q8_BLK + j] = sat_i8(roundf(blk[j] * id));
    }
}

/* x.iter().map(|v| v * v).sum() (model.rs:5615, 7466): a sequential f32 fold
 * (pairwise when g_order == 1). */
static float sum_squares(const float *x, size_t n) {
    if (g_order) {
        float *t = (float *)malloc(n * sizeof(float));
        for (size_t i = 0; i < n; i++) t[i] = x[i] * x[i];
        float s = pairwise(t, n);
        free(t);
        return s;
    }
    float sum_sq = 0.0f;
    for (size_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
    return sum_sq;
}

/* flare-core/src/model.rs:5610-5640 (rmsnorm_quantize_q8_0_scalar). Note the
 * product order (x*w)*inv_rms, unlike rmsnorm_scalar_into. */
void or_rmsnorm_quantize_q8_0(const float *x, const float *w, size_t n, float eps,
                              float *scales, int8_t *q) {
    float sum_sq = sum_squares(x, n);
    float rms = sqrtf(sum_sq / (float)n + eps);
    float inv_rms = 1.0f / rms;
    size_t blocks = n / Q8_BLK;
    for (size_t b = 0; b < blocks; b++) {
        size_t s = b * Q8_BLK;
        float normed[32], amax = 0.0f;
        for (int j = 0; j < Q8_BLK; j++) {
            float v = x[s + j] * w[s + j] * inv_rms;
            normed[j] = v;
            amax = rmax(amax, fabsf(v));
        }
        float scale = amax / 127.0f;
        scales[b] = scale;
        float inv_scale = (scale != 0.0f) ? 127.0f / amax : 0.0f;
        for (int j = 0; j < Q8_BLK; j++) q[s + j] = sat_i8(roundf(normed[j] * inv_scale));
    }
}

/* flare-core/src/model.rs:7469-7477 (rmsnorm_scalar_into): (x*inv_rms)*w. */
void or_rmsnorm(const float *x, const float *w, size_t n, float eps, float *out) {
    float sum_sq = sum_squares(x, n);
    float rms = sqrtf(sum_sq / (float)n + eps);
    float inv_rms = 1.0f / rms;
    for (size_t i = 0; i < n; i++) out[i] = (x[i] * inv_rms) * w[i];
}

/* Integer part of model.rs:8082-8099: s0+s1+s2+s3 over one 32-block. */
static int32_t q8_block_idot(const uint8_t *wq, const int8_t *xq) {
    int32_t s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    for (int j = 0; j < 32; j += 4) {
        s0 += (int32_t)(int8_t)wq[j] * (int32_t)xq[j];
        s1 += (int32_t)(int8_t)wq[j + 1] * (int32_t)xq[j + 1];
        s2 += (int32_t)(int8_t)wq[j + 2] * (int32_t)xq[j + 2];
        s3 += (int32_t)(int8_t)wq[j + 3] * (int32_t)xq[j + 3];
    }
    return s0 + s1 + s2 + s3;
}

void or_block_dots_q8_0(const uint8_t *w, const int8_t *xq, size_t rows, size_t bpr,
                        int32_t *dots) {
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++)
            dots[r * bpr + b] = q8_block_idot(w + (r * bpr + b) * Q8_BYTES + 2, xq + b * Q8_BLK);
}

/* flare-core/src/model.rs:8067-8102 (one row). */
static float q8_row_dot(const uint8_t *row, const float *xs, const int8_t *xq, size_t bpr) {
    float sum = 0.0f;
    for (size_t b = 0; b < bpr; b++) {
        const uint8_t *blk = row + b * Q8_BYTES;
        float w_scale = or_f16_to_f32(rd16(blk));
        float combined = w_scale * xs[b];
        sum += combined * (float)q8_block_idot(blk + 2, xq + b * Q8_BLK);
    }
    return sum;
}

/* The same per-block terms, summed pairwise (g_order == 1). */
static float q8_row_dot_pw(const uint8_t *row, const float *xs, const int8_t *xq, size_t bpr) {
    float *t = (float *)malloc(bpr * sizeof(float));
    for (size_t b = 0; b < bpr; b++) {
        const uint8_t *blk = row + b * Q8_BYTES;
        float combined = or_f16_to_f32(rd16(blk)) * xs[b];
        t[b] = combined * (float)q8_block_idot(blk + 2, xq + b * Q8_BLK);
    }
    float s = pairwise(t, bpr);
    free(t);
    return s;
}

void or_matvec_q8_0_preq(const uint8_t *w, const float *xs, const int8_t *xq, size_t rows,
                         size_t bpr, float *out) {
    OR_PAR
    for (size_t r = 0; r < rows; r++)
        out[r] = g_order ? q8_row_dot_pw(w + r * bpr * Q8_BYTES, xs, xq, bpr)
                         : q8_row_dot(w + r * bpr * Q8_BYTES, xs, xq, bpr);
}

/* Strict '>' over the row scores keeps the first maximum (model.rs:8550,
 * 8652, 8682).  Scores are formed row-parallel, then scanned in row order. */
static void first_max(const float *scores, size_t rows, int64_t *idx, float *val) {
    int64_t bi = 0;
    float bv = -INFINITY;
    for (size_t r = 0; r < rows; r++)
        if (scores[r] > bv) { bv = scores[r]; bi = (int64_t)r; }
    *idx = bi;
    *val = bv;
}

/* flare-core/src/model.rs:8518-8556: strict '>' keeps the first maximum. */
void or_matvec_argmax_q8_0_preq(const uint8_t *w, const float *xs, const int8_t *xq,
                                size_t rows, size_t bpr, int64_t *idx, float *val) {
    float *sc = (float *)malloc(rows * sizeof(float));
    or_matvec_q8_0_preq(w, xs, xq, rows, bpr, sc);
    first_max(sc, rows, idx, val);
    free(sc);
}

/* Integer parts of model.rs:8997-9014 for one superblock. */
static void q4k_sub_idots(const uint8_t *qs, const int8_t *xq_blk /* 256 */, int sub,
                          int32_t *dot_lo, int32_t *dot_hi, int32_t *qs_lo, int32_t *qs_hi) {
    int32_t dl = 0, dh = 0, sl = 0, sh = 0;
    const int8_t *in_lo = xq_blk + sub * 32, *in_hi = xq_blk + (sub + 4) * 32;
    for (int k = 0; k < 32; k++) {
        uint8_t byte = qs[sub * 32 + k];
        int32_t lo = byte & 0x0F, hi = byte >> 4;
        dl += lo * (int32_t)in_lo[k];
        dh += hi * (int32_t)in_hi[k];
        sl += in_lo[k];
        sh += in_hi[k];
    }
    *dot_lo = dl; *dot_hi = dh; *qs_lo = sl; *qs_hi = sh;
}

void or_block_dots_q4k(const uint8_t *w, const int8_t *xq, size_t rows, size_t bpr,
                       int32_t *dots) {
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *blk = w + (r * bpr + b) * Q4K_BYTES;
            for (int sub = 0; sub < 4; sub++) {
                int32_t dl, dh, sl, sh;
                q4k_sub_idots(blk + 16, xq + b * 256, sub, &dl, &dh, &sl, &sh);
                dots[(r * bpr + b) * 8 + 2 * sub] = dl;
                dots[(r * bpr + b) * 8 + 2 * sub + 1] = dh;
            }
        }
}

/* flare-core/src/model.rs:8969-9025 (dot_q4k_q8_0_scalar). */
static float q4k_row_dot(const uint8_t *row, const float *xs, const int8_t *xq, size_t bpr) {
    float sum = 0.0f;
    for (size_t b = 0; b < bpr; b++) {
        const uint8_t *blk = row + b * Q4K_BYTES;
        float d = or_f16_to_f32(rd16(blk)), dmin = or_f16_to_f32(rd16(blk + 2));
        uint8_t sc[8], mn[8];
        or_unpack_q4k_scales(blk + 4, sc, mn);
        size_t is_base = b * 8;
        for (int sub = 0; sub < 4; sub++) {
            int32_t dl, dh, sl, sh;
            q4k_sub_idots(blk + 16, xq + b * 256, sub, &dl, &dh, &sl, &sh);
            float s_lo = xs[is_base + sub], s_hi = xs[is_base + sub + 4];
            float d_sc_lo = d * (float)sc[sub];
            float dmin_mn_lo = dmin * (float)mn[sub];
            float d_sc_hi = d * (float)sc[sub + 4];
            float dmin_mn_hi = dmin * (float)mn[sub + 4];
            sum += s_lo * (d_sc_lo * (float)dl - dmin_mn_lo * (float)sl);
            sum += s_hi * (d_sc_hi * (float)dh - dmin_mn_hi * (float)sh);
        }
    }
    return sum;
}

/* The same per-sub-block terms, summed pairwise (g_order == 1). */
static float q4k_row_dot_pw(const uint8_t *row, const float *xs, const int8_t *xq, size_t bpr) {
    float *t = (float *)malloc(bpr * 8 * sizeof(float));
    size_t nt = 0;
    for (size_t b = 0; b < bpr; b++) {
        const uint8_t *blk = row + b * Q4K_BYTES;
        float d = or_f16_to_f32(rd16(blk)), dmin = or_f16_to_f32(rd16(blk + 2));
        uint8_t sc[8], mn[8];
        or_unpack_q4k_scales(blk + 4, sc, mn);
        size_t is_base = b * 8;
        for (int sub = 0; sub < 4; sub++) {
            int32_t dl, dh, sl, sh;
            q4k_sub_idots(blk + 16, xq + b * 256, sub, &dl, &dh, &sl, &sh);
            float s_lo = xs[is_base + sub], s_hi = xs[is_base + sub + 4];
            float d_sc_lo = d * (float)sc[sub];
            float dmin_mn_lo = dmin * (float)mn[sub];
            float d_sc_hi = d * (float)sc[sub + 4];
            float dmin_mn_hi = dmin * (float)mn[sub + 4];
            t[nt++] = s_lo * (d_sc_lo * (float)dl - dmin_mn_lo * (float)sl);
            t[nt++] = s_hi * (d_sc_hi * (float)dh - dmin_mn_hi * (float)sh);
        }
    }
    float s = pairwise(t, nt);
    free(t);
    return s;
}

/* flare-core/src/model.rs:9672-9779, x86 branch 9768-9778. */
void or_matvec_q4k_q8(const uint8_t *w, const float *xs, const int8_t *xq, size_t rows,
                      size_t cols, float *out) {
    size_t bpr = cols / Q4K_VALS;
    OR_PAR
    for (size_t r = 0; r < rows; r++)
        out[r] = g_order ? q4k_row_dot_pw(w + r * bpr * Q4K_BYTES, xs, xq, bpr)
                         : q4k_row_dot(w + r * bpr * Q4K_BYTES, xs, xq, bpr);
}

/* flare-core/src/model.rs:8569-8659, x86 branch 8644-8658. */
void or_matvec_argmax_q4k_q8_preq(const uint8_t *w, const float *xs, const int8_t *xq,
                                  size_t rows, size_t cols, int64_t *idx, float *val) {
    float *sc = (float *)malloc(rows * sizeof(float));
    or_matvec_q4k_q8(w, xs, xq, rows, cols, sc);
    first_max(sc, rows, idx, val);
    free(sc);
}

/* sum += row[j] * vec[j] in column order (model.rs:8679-8681); pairwise when
 * g_order == 1. */
static float f32_dot(const float *row, const float *vec, size_t n) {
    if (g_order) {
        float *t = (float *)malloc(n * sizeof(float));
        for (size_t j = 0; j < n; j++) t[j] = row[j] * vec[j];
        float s = pairwise(t, n);
        free(t);
        return s;
    }
    float s = 0.0f;
    for (size_t j = 0; j < n; j++) s += row[j] * vec[j];
    return s;
}

/* flare-core/src/model.rs:8668-8689 (matvec_argmax_f32): sequential f32. */
void or_matvec_argmax_f32(const float *mat, const float *vec, size_t rows, size_t cols,
                          int64_t *idx, float *val) {
    float *sc = (float *)malloc(rows * sizeof(float));
    OR_PAR
    for (size_t r = 0; r < rows; r++) {
        sc[r] = f32_dot(mat + r * cols, vec, cols);
    }
    first_max(sc, rows, idx, val);
    free(sc);
}

/* Plain sequential f32 matvec (model.rs:5286-5292 matvec_scalar_row order);
 * the reference's AVX2 variant (5098-5149) reorders the sum, so outputs of the
 * non-greedy logits path are compared with a tolerance. */
void or_matvec_f32(const float *mat, const float *vec, size_t rows, size_t cols, float *out) {
    OR_PAR
    for (size_t r = 0; r < rows; r++) out[r] = f32_dot(mat + r * cols, vec, cols);
}

/* flare-core/src/model.rs:7190-7212 (RopeTable::new) and 7299-7313
 * (apply_rope): identical per-(pos, d) formula, so table and inline agree. */
void or_rope_row(size_t head_dim, size_t pos, float theta, float *c, float *s) {
    size_t half = head_dim / 2;
    for (size_t d = 0; d < half; d++) {
        float freq = 1.0f / powf(theta, 2.0f * (float)d / (float)head_dim);
        float angle = (float)pos * freq;
        s[d] = sinf(angle);
        c[d] = cosf(angle);
    }
}

/* flare-core/src/model.rs:7283-7296 (rotate-half pairs (i, i+half)). */
void or_apply_rope(float *data, size_t num_heads, size_t head_dim, size_t pos, float theta) {
    size_t half = head_dim / 2;
    float *c = (float *)malloc(half * sizeof(float)), *s = (float *)malloc(half * sizeof(float));
    or_rope_row(head_dim, pos, theta, c, s);
    for (size_t h = 0; h < num_heads; h++) {
        float *p = data + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            float x0 = p[i], x1 = p[i + half];
            p[i] = x0 * c[i] - x1 * s[i];
            p[i + half] = x0 * s[i] + x1 * c[i];
        }
    }
    free(c);
    free(s);
}

/* flare-core/src/model.rs:9788-9795 */
void or_silu_mul(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* flare-core/src/model.rs:9849-9905 + 9914-9966 (online softmax, scalar). */
void or_gqa_attention(const float *q, const float *k_cache, const float *v_cache,
                      size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t seq_len,
                      float *out) {
    size_t heads_per_kv = num_heads / num_kv_heads;
    size_t kv_stride = num_kv_heads * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    OR_PAR
    for (size_t h = 0; h < num_heads; h++) {
        size_t kvh = h / heads_per_kv;
        const float *qh = q + h * head_dim;
        float *o = out + h * head_dim;
        for (size_t d = 0; d < head_dim; d++) o[d] = 0.0f;
        float max_score = -INFINITY, sum_exp = 0.0f;
        for (size_t t = 0; t < seq_len; t++) {
            const float *k = k_cache + t * kv_stride + kvh * head_dim;
            const float *v = v_cache + t * kv_stride + kvh * head_dim;
            float dot = 0.0f;
            for (size_t d = 0; d < head_dim; d++) dot += qh[d] * k[d];
            float score = dot * scale;
            float new_max = rmax(max_score, score);
            float old_scale = expf(max_score - new_max);
            float new_weight = expf(score - new_max);
            sum_exp = sum_exp * old_scale + new_weight;
            for (size_t d = 0; d < head_dim; d++) o[d] = o[d] * old_scale + new_weight * v[d];
            max_score = new_max;
        }
        if (sum_exp > 0.0f) {
            float inv = 1.0f / sum_exp;
            for (size_t d = 0; d < head_dim; d++) o[d] *= inv;
        }
    }
}

/* flare-core/src/kv_cache.rs:332-371 (quantize_to_packed). */
void or_kivi_quantize_to_packed(const float *v, size_t n, uint8_t *packed, float *scale_out,
                                float *min_out) {
    float mn = INFINITY, mx = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (v[i] < mn) mn = v[i];
        if (v[i] > mx) mx = v[i];
    }
    float range = mx - mn;
    const float EPS = 1.1920929e-7f; /* f32::EPSILON */
    float scale = fabsf(range) < EPS ? 0.0f : range / 3.0f;
    float inv = fabsf(scale) < EPS ? 0.0f : 3.0f / range;
    size_t nbytes = (n + 3) / 4;
    memset(packed, 0, nbytes);
    for (size_t i = 0; i < n; i++) {
        uint8_t qv = 0;
        if (!(fabsf(scale) < EPS)) {
            float r = roundf((v[i] - mn) * inv);
            r = r < 0.0f ? 0.0f : (r > 3.0f ? 3.0f : r);
            qv = (uint8_t)r;
        }
        packed[i / 4] |= (uint8_t)(qv << ((i % 4) * 2));
    }
    *scale_out = scale;
    *min_out = mn;
}

/* ---- KV forms of the long-context attention benchmark ------------------- */
/* No reference implementation exists (README.md:70 lists a Q8 KV cache; the
 * KIVI variant of the benchmark differs from QuantizedKvCache): the
 * arithmetic follows quantize_input_q8_0_into (model.rs:5557-5570, via
 * or_quantize_input_q8_0) and quantize_to_packed (kv_cache.rs:332-371, via
 * or_kivi_quantize_to_packed); stored scales are binary16 (RNE). */
#define KIVI_GROUP 32
#define KIVI_RESIDUAL 128

size_t or_kivi32_qlen(size_t T) {
    if (T <= KIVI_RESIDUAL + 1) return 0;
    return KIVI_GROUP * ((T - 1 - KIVI_RESIDUAL) / KIVI_GROUP);
}

static float h16(float x) { return or_f16_to_f32(or_f32_to_f16_rne(x)); }

/* quantize n values (gathered with stride) and write back their binary16-
 * scale dequantization code * scale + min (kv_cache.rs:384-392 order) */
static void kivi_group_roundtrip(float *v, size_t n, size_t stride) {
    float buf[KIVI_GROUP];
    uint8_t packed[KIVI_GROUP / 4];
    float scale, mn;
    for (size_t i = 0; i < n; i++) buf[i] = v[i * stride];
    or_kivi_quantize_to_packed(buf, n, packed, &scale, &mn);
    float sh = h16(scale), mh = h16(mn);
    for (size_t i = 0; i < n; i++) {
        float code = (float)((packed[i / 4] >> ((i % 4) * 2)) & 3);
        v[i * stride] = code * sh + mh;
    }
}

void or_kv_view(int kv_mode, const float *K, const float *V, size_t T, size_t nkv, size_t D,
                float *Kout, float *Vout) {
    size_t kvd = nkv * D, n = T * kvd;
    if (kv_mode == OR_KV_Q8) {
        float sc[1];
        int8_t q[32];
        for (size_t b = 0; b < n / 32; b++) {
            for (int w = 0; w < 2; w++) {
                const float *src = (w ? V : K) + 32 * b;
                float *dst = (w ? Vout : Kout) + 32 * b;
                or_quantize_input_q8_0(src, 32, sc, q);
                float d = h16(sc[0]);
                for (int i = 0; i < 32; i++) dst[i] = (float)q[i] * d;
            }
        }
        return;
    }
    for (size_t i = 0; i < n; i++) {
        Kout[i] = kv_mode == OR_KV_F32 ? K[i] : h16(K[i]);
        Vout[i] = kv_mode == OR_KV_F32 ? V[i] : h16(V[i]);
    }
    if (kv_mode != OR_KV_KIVI32) return;
    size_t Q = or_kivi32_qlen(T);
    for (size_t g = 0; g < Q / KIVI_GROUP; g++) {
        size_t t0 = g * KIVI_GROUP;
        for (size_t ch = 0; ch < kvd; ch++) /* K: per channel over the 32 tokens */
            kivi_group_roundtrip(Kout + t0 * kvd + ch, KIVI_GROUP, kvd);
        for (size_t t = t0; t < t0 + KIVI_GROUP; t++) /* V: per token over 32 channels */
            for (size_t cg = 0; cg < kvd / KIVI_GROUP; cg++)
                kivi_group_roundtrip(Vout + t * kvd + cg * KIVI_GROUP, KIVI_GROUP, 1);
    }
}

/* ======================================================================= */
/* Whole-model greedy decode: flare-core/src/model.rs:1872-1942            */
/* (forward_greedy) and 1955-2561 (forward_layers), x86 flags:             */
/* use_quant_for_dim / should_use_q8_for_size are always true (5362-5396). */
/* ======================================================================= */

typedef struct {
    /* kv_cache.rs:35-58; RESIDUAL_WINDOW = 32 (kv_cache.rs:15) */
    uint8_t **kp, **vp;
    float **ks, **kmin, **vs, **vmin, **rk, **rv;
    size_t res_len;
} kivi_t;

struct or_model {
    or_config c;
    or_layer *layers;
    float *embed_f32;    /* token_embedding dequantized (weights.rs load path) */
    float *out_f32;      /* output_weight as f32 (tied: embedding) or NULL */
    const uint8_t *out_raw;
    const float *out_norm;
    float **kc, **vc;    /* KvCache f32 ring per layer (kv_cache.rs:431-546) */
    size_t position, length;
    kivi_t kv2;
    /* forward buffers */
    float *x, *q, *k, *v, *attn, *proj, *normed, *gate, *up, *hid, *ffn, *final_normed;
    float *xs;
    int8_t *xq;
    float *kdq, *vdq;
};

static size_t fmt_bpr(int fmt, size_t cols) {
    return (fmt == OR_Q8_0) ? cols / 32 : (fmt == OR_F32 ? cols : cols / 256);
}

or_model *or_model_create(const or_config *cfg, const or_layer *layers,
                          const uint8_t *embedding, const uint8_t *output_weight,
                          const float *output_norm) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->c = *cfg;
    size_t H = cfg->hidden, L = cfg->layers, V = cfg->vocab;
    size_t qd = (size_t)cfg->heads * cfg->head_dim, kvd = (size_t)cfg->kv_heads * cfg->head_dim;
    size_t F = cfg->inter, S = cfg->max_seq;
    m->layers = (or_layer *)malloc(L * sizeof(or_layer));
    memcpy(m->layers, layers, L * sizeof(or_layer));
    m->embed_f32 = (float *)malloc(V * H * sizeof(float));
    or_dequant_tensor(embedding, cfg->embed_format, V, fmt_bpr(cfg->embed_format, H), m->embed_f32);
    if (cfg->output_format < 0) {
        m->out_f32 = m->embed_f32; /* weights.rs:50-51: output falls back to token_embd */
    } else if (cfg->output_format == OR_Q8_0 || cfg->output_format == OR_Q4K) {
        m->out_raw = output_weight; /* raw_output_weight: fused quantized argmax */
    } else {
        m->out_f32 = (float *)malloc(V * H * sizeof(float));
        or_dequant_tensor(output_weight, cfg->output_format, V, fmt_bpr(cfg->output_format, H),
                          m->out_f32);
    }
    m->out_norm = output_norm;
    m->kc = (float **)calloc(L, sizeof(float *));
    m->vc = (float **)calloc(L, sizeof(float *));
    for (size_t l = 0; l < L; l++) {
        m->kc[l] = (float *)calloc(S * kvd, sizeof(float));
        m->vc[l] = (float *)calloc(S * kvd, sizeof(float));
    }
    if (cfg->kv_mode == OR_KV_KIVI2) {
        kivi_t *k = &m->kv2;
        size_t ppt = (kvd + 3) / 4;
        k->res_len = S < 32 ? S : 32;
        k->kp = (uint8_t **)calloc(L, sizeof(void *));
        k->vp = (uint8_t **)calloc(L, sizeof(void *));
        k->ks = (float **)calloc(L, sizeof(void *));
        k->kmin = (float **)calloc(L, sizeof(void *));
        k->vs = (float **)calloc(L, sizeof(void *));
        k->vmin = (float **)calloc(L, sizeof(void *));
        k->rk = (float **)calloc(L, sizeof(void *));
        k->rv = (float **)calloc(L, sizeof(void *));
        for (size_t l = 0; l < L; l++) {
            k->kp[l] = (uint8_t *)calloc(S * ppt, 1);
            k->vp[l] = (uint8_t *)calloc(S * ppt, 1);
            k->ks[l] = (float *)calloc(kvd, sizeof(float));
            k->kmin[l] = (float *)calloc(kvd, sizeof(float));
            k->vs[l] = (float *)calloc(S, sizeof(float));
            k->vmin[l] = (float *)calloc(S, sizeof(float));
            k->rk[l] = (float *)calloc(k->res_len * kvd, sizeof(float));
            k->rv[l] = (float *)calloc(k->res_len * kvd, sizeof(float));
        }
    }
    if (cfg->kv_mode == OR_KV_KIVI2 || cfg->kv_mode == OR_KV_Q8 || cfg->kv_mode == OR_KV_KIVI32) {
        m->kdq = (float *)calloc(S * kvd, sizeof(float));
        m->vdq = (float *)calloc(S * kvd, sizeof(float));
    }
    size_t big = F > H ? F : H;
    if (qd > big) big = qd;
    m->x = (float *)calloc(H, 4);
    m->q = (float *)calloc(qd, 4);
    m->k = (float *)calloc(kvd, 4);
    m->v = (float *)calloc(kvd, 4);
    m->attn = (float *)calloc(qd, 4);
    m->proj = (float *)calloc(H, 4);
    m->normed = (float *)calloc(H, 4);
    m->gate = (float *)calloc(F, 4);
    m->up = (float *)calloc(F, 4);
    m->hid = (float *)calloc(F, 4);
    m->ffn = (float *)calloc(H, 4);
    m->final_normed = (float *)calloc(H, 4);
    m->xs = (float *)calloc(big / 32 + 1, 4);
    m->xq = (int8_t *)calloc(big, 1);
    return m;
}

void or_model_destroy(or_model *m) {
    if (!m) return;
    size_t L = m->c.layers;
    for (size_t l = 0; l < L; l++) { free(m->kc[l]); free(m->vc[l]); }
    free(m->kc); free(m->vc);
    if (m->c.kv_mode == OR_KV_KIVI2) {
        kivi_t *k = &m->kv2;
        for (size_t l = 0; l < L; l++) {
            free(k->kp[l]); free(k->vp[l]); free(k->ks[l]); free(k->kmin[l]);
            free(k->vs[l]); free(k->vmin[l]); free(k->rk[l]); free(k->rv[l]);
        }
        free(k->kp); free(k->vp); free(k->ks); free(k->kmin);
        free(k->vs); free(k->vmin); free(k->rk); free(k->rv);
    }
    free(m->kdq); free(m->vdq);
    if (m->out_f32 && m->out_f32 != m->embed_f32) free(m->out_f32);
    free(m->embed_f32);
    free(m->layers);
    free(m->x); free(m->q); free(m->k); free(m->v); free(m->attn); free(m->proj);
    free(m->normed); free(m->gate); free(m->up); free(m->hid); free(m->ffn);
    free(m->final_normed); free(m->xs); free(m->xq);
    free(m);
}

/* KvCache::clear (kv_cache.rs:534-545) and QuantizedKvCache::clear (285-310). */
void or_model_reset(or_model *m) {
    size_t kvd = (size_t)m->c.kv_heads * m->c.head_dim, S = m->c.max_seq;
    m->position = 0;
    m->length = 0;
    for (int l = 0; l < m->c.layers; l++) {
        memset(m->kc[l], 0, S * kvd * 4);
        memset(m->vc[l], 0, S * kvd * 4);
        if (m->c.kv_mode == OR_KV_KIVI2) {
            kivi_t *k = &m->kv2;
            size_t ppt = (kvd + 3) / 4;
            memset(k->kp[l], 0, S * ppt);
            memset(k->vp[l], 0, S * ppt);
            memset(k->ks[l], 0, kvd * 4);
            memset(k->kmin[l], 0, kvd * 4);
            memset(k->vs[l], 0, S * 4);
            memset(k->vmin[l], 0, S * 4);
            memset(k->rk[l], 0, k->res_len * kvd * 4);
            memset(k->rv[l], 0, k->res_len * kvd * 4);
        }
    }
}

/* QuantizedKvCache::write (kv_cache.rs:121-162) incl. update_per_channel_stats
 * (kv_cache.rs:399-420). */
static void kivi_write(or_model *m, int l, const float *key, const float *val) {
    kivi_t *k = &m->kv2;
    size_t kvd = (size_t)m->c.kv_heads * m->c.head_dim, ppt = (kvd + 3) / 4;
    size_t pos = m->position, off = pos * ppt;
    float s, mn;
    or_kivi_quantize_to_packed(key, kvd, k->kp[l] + off, &s, &mn);
    const float EPS = 1.1920929e-7f;
    if (m->length == 0) {
        for (size_t i = 0; i < kvd; i++) { k->kmin[l][i] = key[i]; k->ks[l][i] = 0.0f; }
    } else {
        for (size_t i = 0; i < kvd; i++) {
            float old_min = k->kmin[l][i];
            float old_max = old_min + k->ks[l][i] * 3.0f;
            float new_min = fminf(old_min, key[i]);
            float new_max = fmaxf(old_max, key[i]);
            float range = new_max - new_min;
            k->kmin[l][i] = new_min;
            k->ks[l][i] = fabsf(range) < EPS ? 0.0f : range / 3.0f;
        }
    }
    or_kivi_quantize_to_packed(val, kvd, k->vp[l] + off, &s, &mn);
    k->vs[l][pos] = s;
    k->vmin[l][pos] = mn;
    size_t res_off = (pos % k->res_len) * kvd;
    memcpy(k->rk[l] + res_off, key, kvd * 4);
    memcpy(k->rv[l] + res_off, val, kvd * 4);
}

/* QuantizedKvCache::dequant_keys / dequant_values (kv_cache.rs:189-250). */
static void kivi_dequant(const or_model *m, int l, float *kout, float *vout) {
    const kivi_t *k = &m->kv2;
    size_t kvd = (size_t)m->c.kv_heads * m->c.head_dim, ppt = (kvd + 3) / 4;
    size_t n = m->length, S = m->c.max_seq;
    memset(kout, 0, S * kvd * 4);
    memset(vout, 0, S * kvd * 4);
    for (size_t t = 0; t < n; t++) {
        size_t ring = (n < S) ? t : (m->position + t) % S;
        int in_res = (n <= k->res_len) ? 1 : (t >= n - k->res_len);
        float *ko = kout + ring * kvd, *vo = vout + ring * kvd;
        if (in_res) {
            size_t ro = (ring % k->res_len) * kvd;
            memcpy(ko, k->rk[l] + ro, kvd * 4);
            memcpy(vo, k->rv[l] + ro, kvd * 4);
        } else {
            const uint8_t *kp = k->kp[l] + ring * ppt, *vp = k->vp[l] + ring * ppt;
            for (size_t i = 0; i < kvd; i++) {
                float qk = (float)((kp[i / 4] >> ((i % 4) * 2)) & 3);
                ko[i] = qk * k->ks[l][i] + k->kmin[l][i];
                float qv = (float)((vp[i / 4] >> ((i % 4) * 2)) & 3);
                vo[i] = qv * k->vs[l][ring] + k->vmin[l][ring];
            }
        }
    }
}

static void matvec_layer(const or_model *m, const uint8_t *w, size_t rows, size_t cols,
                         const float *xs, const int8_t *xq, float *out) {
    if (m->c.layer_format == OR_Q8_0)
        or_matvec_q8_0_preq(w, xs, xq, rows, cols / 32, out);
    else
        or_matvec_q4k_q8(w, xs, xq, rows, cols, out);
}

static void forward_layers(or_model *m, uint32_t token, size_t pos) {
    const or_config *c = &m->c;
    size_t H = c->hidden, hd = c->head_dim, nh = c->heads, nkv = c->kv_heads;
    size_t qd = nh * hd, kvd = nkv * hd, F = c->inter;
    int q8 = c->layer_format == OR_Q8_0;
    memcpy(m->x, m->embed_f32 + (size_t)token * H, H * 4); /* model.rs:1964-1966 */
    for (int l = 0; l < c->layers; l++) {
        const or_layer *ly = &m->layers[l];
        /* attention block: model.rs:2016-2095 */
        if (q8) {
            or_rmsnorm_quantize_q8_0(m->x, ly->attn_norm, H, c->eps, m->xs, m->xq);
        } else {
            or_rmsnorm(m->x, ly->attn_norm, H, c->eps, m->normed);
            or_quantize_input_q8_0(m->normed, H, m->xs, m->xq);
        }
        matvec_layer(m, ly->wq, qd, H, m->xs, m->xq, m->q);
        matvec_layer(m, ly->wk, kvd, H, m->xs, m->xq, m->k);
        matvec_layer(m, ly->wv, kvd, H, m->xs, m->xq, m->v);
        /* model.rs:2169-2184 */
        or_apply_rope(m->q, nh, hd, pos, c->theta);
        or_apply_rope(m->k, nkv, hd, pos, c->theta);
        /* model.rs:2187-2206: kv_cache.write at the ring position.  In F16
         * mode the stored K/V are rounded through binary16, which models the
         * reference's f16 GPU KV cache (flare-gpu/src/kv_cache.rs:120-159). */
        float *kd = m->kc[l] + m->position * kvd, *vd = m->vc[l] + m->position * kvd;
        for (size_t i = 0; i < kvd; i++) {
            if (c->kv_mode == OR_KV_F16) {
                kd[i] = or_f16_to_f32(or_f32_to_f16_rne(m->k[i]));
                vd[i] = or_f16_to_f32(or_f32_to_f16_rne(m->v[i]));
            } else {
                kd[i] = m->k[i];
                vd[i] = m->v[i];
            }
        }
        if (c->kv_mode == OR_KV_KIVI2) kivi_write(m, l, m->k, m->v);
        size_t seq_len = m->length + 1; /* model.rs:2209 */
        if (c->kv_mode == OR_KV_KIVI2) {
            kivi_dequant(m, l, m->kdq, m->vdq);
            or_gqa_attention(m->q, m->kdq, m->vdq, nh, nkv, hd, seq_len, m->attn);
        } else if (c->kv_mode == OR_KV_Q8 || c->kv_mode == OR_KV_KIVI32) {
            /* rows 0..seq_len-1 as written (no ring wrap: seq_len <= max_seq) */
            or_kv_view(c->kv_mode, m->kc[l], m->vc[l], seq_len, nkv, hd, m->kdq, m->vdq);
            or_gqa_attention(m->q, m->kdq, m->vdq, nh, nkv, hd, seq_len, m->attn);
        } else {
            or_gqa_attention(m->q, m->kc[l], m->vc[l], nh, nkv, hd, seq_len, m->attn);
        }
        /* wo: model.rs:2250-2291 */
        or_quantize_input_q8_0(m->attn, qd, m->xs, m->xq);
        matvec_layer(m, ly->wo, H, qd, m->xs, m->xq, m->proj);
        for (size_t i = 0; i < H; i++) m->x[i] += m->proj[i]; /* 2305-2311 */
        /* FFN: model.rs:2376-2416 */
        if (q8) {
            or_rmsnorm_quantize_q8_0(m->x, ly->ffn_norm, H, c->eps, m->xs, m->xq);
        } else {
            or_rmsnorm(m->x, ly->ffn_norm, H, c->eps, m->normed);
            or_quantize_input_q8_0(m->normed, H, m->xs, m->xq);
        }
        matvec_layer(m, ly->w_gate, F, H, m->xs, m->xq, m->gate);
        matvec_layer(m, ly->w_up, F, H, m->xs, m->xq, m->up);
        or_silu_mul(m->gate, m->up, F, m->hid); /* 2455-2461 */
        or_quantize_input_q8_0(m->hid, F, m->xs, m->xq); /* 2480-2522 */
        matvec_layer(m, ly->w_down, H, F, m->xs, m->xq, m->ffn);
        for (size_t i = 0; i < H; i++) m->x[i] += m->ffn[i]; /* 2537-2543 */
    }
    /* KvCache::advance (kv_cache.rs:484-489), model.rs:2547 */
    m->position = (m->position + 1) % (size_t)c->max_seq;
    if (m->length < (size_t)c->max_seq) m->length++;
    or_rmsnorm(m->x, m->out_norm, H, c->eps, m->final_normed); /* 2553-2558 */
}

int64_t or_forward_greedy(or_model *m, uint32_t token, size_t pos, float *val) {
    const or_config *c = &m->c;
    size_t H = c->hidden, V = c->vocab;
    forward_layers(m, token, pos);
    int64_t idx;
    float v;
    /* model.rs:1898-1932 */
    if (m->out_raw && c->output_format == OR_Q4K && c->layer_format == OR_Q4K) {
        or_quantize_input_q8_0(m->final_normed, H, m->xs, m->xq);
        or_matvec_argmax_q4k_q8_preq(m->out_raw, m->xs, m->xq, V, H, &idx, &v);
    } else if (m->out_raw && c->output_format == OR_Q8_0 && c->layer_format == OR_Q8_0) {
        or_quantize_input_q8_0(m->final_normed, H, m->xs, m->xq);
        or_matvec_argmax_q8_0_preq(m->out_raw, m->xs, m->xq, V, H / 32, &idx, &v);
    } else {
        const float *w = m->out_f32;
        float *tmp = NULL;
        if (!w) { /* quantized output without the matching fused path */
            tmp = (float *)malloc(V * H * 4);
            or_dequant_tensor(m->out_raw, c->output_format, V, fmt_bpr(c->output_format, H), tmp);
            w = tmp;
        }
        or_matvec_argmax_f32(w, m->final_normed, V, H, &idx, &v);
        free(tmp);
    }
    if (val) *val = v;
    return idx;
}

void or_forward_logits(or_model *m, uint32_t token, size_t pos, float *logits) {
    const or_config *c = &m->c;
    size_t H = c->hidden, V = c->vocab;
    forward_layers(m, token, pos);
    if (m->out_raw && c->output_format == OR_Q8_0) {
        or_quantize_input_q8_0(m->final_normed, H, m->xs, m->xq);
        or_matvec_q8_0_preq(m->out_raw, m->xs, m->xq, V, H / 32, logits);
    } else if (m->out_raw && c->output_format == OR_Q4K) {
        or_quantize_input_q8_0(m->final_normed, H, m->xs, m->xq);
        or_matvec_q4k_q8(m->out_raw, m->xs, m->xq, V, H, logits);
    } else {
        or_matvec_f32(m->out_f32, m->final_normed, V, H, logits);
    }
}

const float *or_model_final_normed(const or_model *m) { return m->final_normed; }

/* Generator::step greedy path (generate.rs:186-206) with the prompt fed one
 * token at a time through forward_greedy. */
void or_generate_greedy(or_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                        uint32_t *out) {
    uint32_t tok = 0;
    size_t pos = 0;
    for (size_t i = 0; i < n_prompt; i++, pos++) tok = (uint32_t)or_forward_greedy(m, prompt[i], pos, NULL);
    for (size_t i = 0; i < n_gen; i++) {
        out[i] = tok;
        if (i + 1 < n_gen) tok = (uint32_t)or_forward_greedy(m, tok, pos++, NULL);
    }
}


/* ========================================================================
 * Sampling: flare-core/src/sampling.rs
 * ======================================================================== */

typedef struct {
    float p;
    uint32_t idx;
} or_cand;

/* descending probability; ties by ascending index (the reference's
 * sort_unstable_by leaves equal probabilities in an unspecified order) */
static int or_cand_cmp(const void *a, const void *b) {
    const or_cand *x = (const or_cand *)a, *y = (const or_cand *)b;
    if (x->p > y->p) return -1;
    if (x->p < y->p) return 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

/* sample_greedy (sampling.rs:101-111) */
static uint32_t or_sample_greedy(const float *v, size_t n) {
    uint32_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (v[i] > bv) {
            bv = v[i];
            best = (uint32_t)i;
        }
    return best;
}

/* The walk shared by the three samplers over a descending candidate list:
 * total = sequential sum, threshold = u * total, first prefix >= threshold
 * (sampling.rs:170-180, 206-216, 257-267). */
static uint32_t or_walk(const or_cand *c, size_t L, float u) {
    float total = 0.0f;
    for (size_t i = 0; i < L; i++) total += c[i].p;
    const float thr = u * total;
    float acc = 0.0f;
    for (size_t i = 0; i < L; i++) {
        acc += c[i].p;
        if (acc >= thr) return c[i].idx;
    }
    return c[L - 1].idx;
}

int64_t or_sample(const float *logits, size_t n, float temperature, float top_p, int top_k,
                  float repeat_penalty, float min_p, const uint32_t *prev, size_t n_prev,
                  float rng_val) {
    if (n == 0) return -1;
    float *v = (float *)malloc(n * sizeof(float));
    or_cand *c = (or_cand *)malloc(n * sizeof(or_cand));
    memcpy(v, logits, n * sizeof(float));
    /* apply_repeat_penalty (sampling.rs:83-96) */
    if (repeat_penalty != 1.0f)
        for (size_t j = 0; j < n_prev; j++) {
            const size_t t = prev[j];
            if (t < n) v[t] = v[t] > 0.0f ? v[t] / repeat_penalty : v[t] * repeat_penalty;
        }
    /* apply_temperature (sampling.rs:73-81) */
    if (temperature != 0.0f && temperature != 1.0f) {
        const float inv = 1.0f / temperature;
        for (size_t i = 0; i < n; i++) v[i] *= inv;
    }
    int64_t out;
    if (temperature == 0.0f) {
        out = or_sample_greedy(v, n);
        goto done;
    }
    {
        /* softmax pieces: max fold, exps, sequential sum (sampling.rs:115-119, 132-135) */
        float mx = -INFINITY;
        for (size_t i = 0; i < n; i++) mx = fmaxf(mx, v[i]);
        float sum = 0.0f;
        for (size_t i = 0; i < n; i++) {
            v[i] = expf(v[i] - mx);
            sum += v[i];
        }
        const int mode = top_p < 1.0f ? 1 : (min_p > 0.0f ? 2 : (top_k > 0 ? 3 : 1));
        const float tp = top_p < 1.0f ? top_p : 1.0f;
        if (mode == 2) {
            /* sample_min_p (sampling.rs:228-268): softmax() divides */
            float pmax = 0.0f;
            for (size_t i = 0; i < n; i++) {
                v[i] = v[i] / sum;
                pmax = fmaxf(pmax, v[i]);
            }
            const float thr = min_p * pmax;
            size_t L = 0;
            for (size_t i = 0; i < n; i++)
                if (v[i] >= thr) {
                    c[L].p = v[i];
                    c[L].idx = (uint32_t)i;
                    L++;
                }
            if (L == 0) {
                /* sample_greedy(logits): the penalized, scaled logits */
                memcpy(v, logits, n * sizeof(float));
                out = -2;
                goto fallback;
            }
            qsort(c, L, sizeof(or_cand), or_cand_cmp);
            out = or_walk(c, L, rng_val);
            goto done;
        }
        const float inv_sum = 1.0f / sum;
        for (size_t i = 0; i < n; i++) {
            c[i].p = v[i] * inv_sum;
            c[i].idx = (uint32_t)i;
        }
        /* the K largest (select_nth_unstable_by + truncate), ordered */
        qsort(c, n, sizeof(or_cand), or_cand_cmp);
        if (mode == 1) {
            /* sample_top_p (sampling.rs:131-181): INITIAL_K = 512, cumulative cut */
            const size_t K = n < 512 ? n : 512;
            size_t cutoff = K;
            float cum = 0.0f;
            for (size_t i = 0; i < K; i++) {
                cum += c[i].p;
                if (cum >= tp) {
                    cutoff = i + 1;
                    break;
                }
            }
            out = or_walk(c, cutoff, rng_val);
        } else {
            /* sample_top_k (sampling.rs:186-217) */
            size_t K = (size_t)top_k < n ? (size_t)top_k : n;
            if (K < 1) K = 1;
            out = or_walk(c, K, rng_val);
        }
        goto done;
    }
fallback:
    /* min-p with no candidate: greedy over the transformed logits */
    if (repeat_penalty != 1.0f)
        for (size_t j = 0; j < n_prev; j++) {
            const size_t t = prev[j];
            if (t < n) v[t] = v[t] > 0.0f ? v[t] / repeat_penalty : v[t] * repeat_penalty;
        }
    {
        const float inv = 1.0f / temperature;
        if (temperature != 1.0f)
            for (size_t i = 0; i < n; i++) v[i] *= inv;
    }
    out = or_sample_greedy(v, n);
done:
    free(v);
    free(c);
    return out;
}
