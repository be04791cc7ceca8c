/*
 * oracle.c -- CPU restatement of unltd-inference's quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle the GPU results are compared with,
 * never the product): see oracle.h.
 * Each function cites the reference function it restates. Arithmetic follows
 * the reference operation by operation; the build disables FP contraction so
 * that every a*b+c stays two roundings, as in the reference (kernels.rs:9,
 * quants.rs:345).
 *
 * One deliberate difference: the reference allocates a Vec of products per
 * row and one Vec per level of the pairwise tree (quants.rs:140,
 * kernels.rs:28-40). Here the same tree is evaluated in caller-provided
 * scratch; the summation order, and therefore every bit of the result, is
 * unchanged.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* a1: f16 -> f32, quants.rs:44-72                                          */
/* ---------------------------------------------------------------------- */
float or_f16_to_f32(uint16_t h16) {
    uint32_t h = h16;
    uint32_t sign = (h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t frac = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (frac == 0) {
            bits = sign;
        } else {
            uint32_t e = 113u, m = frac; /* subnormal: renormalise */
            while ((m & 0x400) == 0) {
                m <<= 1;
                e -= 1;
            }
            bits = sign | (e << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 0x1F) {
        bits = frac == 0 ? (sign | 0x7F800000u) : (sign | 0x7FC00000u);
    } else {
        bits = sign | ((exp + 112) << 23) | (frac << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t f16_at(const uint8_t *p) {
    return (uint16_t)(p[0] | (p[1] << 8));
}

/* ---------------------------------------------------------------------- */
/* a2: scale_min_k4, quants.rs:92-102                                       */
/* ---------------------------------------------------------------------- */
void or_scale_min_k4(const uint8_t *s, int g, uint8_t *sc, uint8_t *m) {
    if (g < 4) {
        *sc = s[g] & 63;
        *m = s[g + 4] & 63;
    } else {
        *sc = (uint8_t)((s[g + 4] & 0xF) | ((s[g - 4] >> 6) << 4));
        *m = (uint8_t)((s[g + 4] >> 4) | ((s[g] >> 6) << 4));
    }
}

/* ---------------------------------------------------------------------- */
/* a6: pairwise_sum_f64, kernels.rs:27-42                                   */
/* Level by level: next[i] = lvl[2i] + lvl[2i+1]; an odd tail is carried    */
/* unpaired to the next level. Empty sum = 0.0.                             */
/* ---------------------------------------------------------------------- */
double or_pairwise_sum_f64(const double *vals, size_t n, double *scratch) {
    if (n == 0) return 0.0;
    if (scratch != vals) memcpy(scratch, vals, n * sizeof(double));
    size_t len = n;
    while (len > 1) {
        size_t o = 0, i = 0;
        for (; i + 1 < len; i += 2) scratch[o++] = scratch[i] + scratch[i + 1];
        if (i < len) scratch[o++] = scratch[i];
        len = o;
    }
    return scratch[0];
}

/* a6: dot_f32, quants.rs:106-114 */
static double dot_f32_buf(const float *x, const float *w, size_t n,
                          double *prods) {
    for (size_t i = 0; i < n; i++) prods[i] = (double)x[i] * (double)w[i];
    return or_pairwise_sum_f64(prods, n, prods);
}

/* a7: dot_q4_k, quants.rs:132-156 (element map :146-151) */
static double dot_q4_k_buf(const float *x, const uint8_t *w, size_t n,
                           double *prods) {
    size_t nb = n / OR_QK_K;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q4_K;
        double d = (double)or_f16_to_f32(f16_at(blk));
        double dmin = (double)or_f16_to_f32(f16_at(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int e = 0; e < OR_QK_K; e++) {
            int g = e / 32;
            uint8_t sc, m;
            or_scale_min_k4(scales, g, &sc, &m);
            uint8_t byte = qs[32 * (g / 2) + (e % 32)];
            uint8_t nib = (g % 2 == 0) ? (byte & 0xF) : (byte >> 4);
            double wv = (d * (double)sc) * (double)nib - (dmin * (double)m);
            prods[b * OR_QK_K + e] = (double)x[b * OR_QK_K + e] * wv;
        }
    }
    return or_pairwise_sum_f64(prods, n, prods);
}

/* a8: dot_q6_k, quants.rs:171-200 (element map :185-195) */
static double dot_q6_k_buf(const float *x, const uint8_t *w, size_t n,
                           double *prods) {
    size_t nb = n / OR_QK_K;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q6_K;
        const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
        double d = (double)or_f16_to_f32(f16_at(blk + 208));
        for (int e = 0; e < OR_QK_K; e++) {
            uint8_t byte = ql[64 * (e / 128) + (e % 64)];
            uint8_t nib = ((e / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
            int hi2 = (qh[(e % 32) + 32 * (e / 128)] >> (2 * ((e % 128) / 32))) & 3;
            int q = ((int)nib | (hi2 << 4)) - 32;
            int8_t sc = (int8_t)scales[e / 16];
            double wv = d * ((double)sc * (double)q);
            prods[b * OR_QK_K + e] = (double)x[b * OR_QK_K + e] * wv;
        }
    }
    return or_pairwise_sum_f64(prods, n, prods);
}

/* Q8_0 (closed form): block = f16 d + 32 x int8 q, w = d*q (exact in f64);
 * dot follows dot_q4_k's contract: exact f64 products, pairwise tree. */
static double dot_q8_0_buf(const float *x, const uint8_t *w, size_t n,
                           double *prods) {
    size_t nb = n / OR_QK8_0;
    for (size_t b = 0; b < nb; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q8_0;
        double d = (double)or_f16_to_f32(f16_at(blk));
        for (int e = 0; e < OR_QK8_0; e++) {
            double wv = d * (double)(int8_t)blk[2 + e];
            prods[b * OR_QK8_0 + e] = (double)x[b * OR_QK8_0 + e] * wv;
        }
    }
    return or_pairwise_sum_f64(prods, n, prods);
}

typedef double (*dot_fn)(const float *, const uint8_t *, size_t, double *);

static double dot_f32_bytes(const float *x, const uint8_t *w, size_t n,
                            double *prods) {
    /* rows of F32 weights arrive as bytes (bytemuck::cast_slice, :458) */
    float *tmp = (float *)malloc(n * sizeof(float));
    if (!tmp) return NAN;
    memcpy(tmp, w, n * sizeof(float));
    double r = dot_f32_buf(x, tmp, n, prods);
    free(tmp);
    return r;
}

static double with_prods(dot_fn f, const float *x, const uint8_t *w,
                         size_t n) {
    double *p = (double *)malloc((n ? n : 1) * sizeof(double));
    if (!p) return NAN;
    double r = f(x, w, n, p);
    free(p);
    return r;
}

double or_dot_f32(const float *x, const float *w, size_t n) {
    double *p = (double *)malloc((n ? n : 1) * sizeof(double));
    if (!p) return NAN;
    double r = dot_f32_buf(x, w, n, p);
    free(p);
    return r;
}
double or_dot_q4_k(const float *x, const uint8_t *w, size_t n) {
    return with_prods(dot_q4_k_buf, x, w, n);
}
double or_dot_q6_k(const float *x, const uint8_t *w, size_t n) {
    return with_prods(dot_q6_k_buf, x, w, n);
}
double or_dot_q8_0(const float *x, const uint8_t *w, size_t n) {
    return with_prods(dot_q8_0_buf, x, w, n);
}

/* min_forward.rs:52-80 */
size_t or_row_bytes(int dtype, size_t n) {
    switch (dtype) {
    case OR_F32: return n * 4;
    case OR_F16: return n * 2;
    case OR_Q8_0: return n % 32 ? 0 : n / 32 * OR_BLOCK_Q8_0;
    case OR_Q4_K: return n % 256 ? 0 : n / 256 * OR_BLOCK_Q4_K;
    case OR_Q6_K: return n % 256 ? 0 : n / 256 * OR_BLOCK_Q6_K;
    default: return 0;
    }
}

/* ---------------------------------------------------------------------- */
/* a9: gemv_quant, quants.rs:422-466. Checks in the reference's order       */
/* (:430-452). Q8_0 is accepted (closed form) where the reference panics.   */
/* ---------------------------------------------------------------------- */
static int gemv_quant_check(size_t out_len, size_t x_len, size_t w_len,
                            size_t dim_in, size_t dim_out, int dtype,
                            size_t *row_bytes) {
    if (out_len != dim_out) return OR_ERR_LEN;
    if (x_len < dim_in) return OR_ERR_LEN;
    switch (dtype) {
    case OR_F32: *row_bytes = dim_in * 4; break;
    case OR_Q4_K:
    case OR_Q6_K:
        if (dim_in % OR_QK_K) return OR_ERR_BLOCK_MULTIPLE;
        *row_bytes = or_row_bytes(dtype, dim_in);
        break;
    case OR_Q8_0:
        if (dim_in % OR_QK8_0) return OR_ERR_BLOCK_MULTIPLE;
        *row_bytes = or_row_bytes(dtype, dim_in);
        break;
    default: return OR_ERR_DTYPE;
    }
    if (w_len != *row_bytes * dim_out) return OR_ERR_LEN;
    return OR_OK;
}

typedef struct {
    float *out;
    const float *x;
    const uint8_t *w;
    size_t dim_in, row_bytes, j0, j1;
    int dtype;
    const or_q8k_block *xq; /* q8k path only */
    int rc;
} rows_job;

static void *gemv_rows(void *arg) {
    rows_job *jb = (rows_job *)arg;
    double *prods = (double *)malloc((jb->dim_in ? jb->dim_in : 1) * sizeof(double));
    if (!prods) {
        jb->rc = OR_ERR_ALLOC;
        return NULL;
    }
    dot_fn f = jb->dtype == OR_Q4_K   ? dot_q4_k_buf
               : jb->dtype == OR_Q6_K ? dot_q6_k_buf
               : jb->dtype == OR_Q8_0 ? dot_q8_0_buf
                                      : dot_f32_bytes;
    for (size_t j = jb->j0; j < jb->j1; j++)
        jb->out[j] = (float)f(jb->x, jb->w + j * jb->row_bytes, jb->dim_in, prods);
    free(prods);
    jb->rc = OR_OK;
    return NULL;
}

static void *gemv_q8k_rows(void *arg) {
    rows_job *jb = (rows_job *)arg;
    size_t nb = jb->dim_in / OR_QK_K;
    for (size_t j = jb->j0; j < jb->j1; j++) {
        const uint8_t *row = jb->w + j * jb->row_bytes;
        jb->out[j] = jb->dtype == OR_Q4_K ? or_dot_q4_k_q8_k(jb->xq, nb, row)
                                          : or_dot_q6_k_q8_k(jb->xq, nb, row);
    }
    jb->rc = OR_OK;
    return NULL;
}

static int run_rows(void *(*fn)(void *), rows_job proto, size_t dim_out,
                    int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > dim_out) nthreads = dim_out ? (int)dim_out : 1;
    rows_job *jobs = (rows_job *)calloc((size_t)nthreads, sizeof(rows_job));
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    if (!jobs || !th) {
        free(jobs);
        free(th);
        return OR_ERR_ALLOC;
    }
    size_t per = (dim_out + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = proto;
        jobs[t].j0 = (size_t)t * per < dim_out ? (size_t)t * per : dim_out;
        jobs[t].j1 = jobs[t].j0 + per < dim_out ? jobs[t].j0 + per : dim_out;
    }
    if (nthreads == 1) {
        fn(&jobs[0]);
    } else {
        for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, fn, &jobs[t]);
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    }
    int rc = OR_OK;
    for (int t = 0; t < nthreads; t++)
        if (jobs[t].rc) rc = jobs[t].rc;
    free(jobs);
    free(th);
    return rc;
}

int or_gemv_quant_mt(float *out, size_t out_len, const float *x, size_t x_len,
                     const uint8_t *w, size_t w_len, size_t dim_in,
                     size_t dim_out, int dtype, int nthreads) {
    size_t rb = 0;
    int rc = gemv_quant_check(out_len, x_len, w_len, dim_in, dim_out, dtype, &rb);
    if (rc) return rc;
    rows_job proto = {out, x, w, dim_in, rb, 0, 0, dtype, NULL, OR_OK};
    return run_rows(gemv_rows, proto, dim_out, nthreads);
}

int or_gemv_quant(float *out, size_t out_len, const float *x, size_t x_len,
                  const uint8_t *w, size_t w_len, size_t dim_in, size_t dim_out,
                  int dtype) {
    return or_gemv_quant_mt(out, out_len, x, x_len, w, w_len, dim_in, dim_out,
                            dtype, 1);
}

/* ---------------------------------------------------------------------- */
/* a10: nearest_int, quants.rs:230-233; quantize_q8_k, quants.rs:250-290    */
/* ---------------------------------------------------------------------- */
int32_t or_nearest_int(float fval) {
    float val = fval + 12582912.0f;
    uint32_t bits;
    memcpy(&bits, &val, 4);
    return (int32_t)(bits & 0x007FFFFFu) - 0x00400000;
}

int or_quantize_q8_k(or_q8k_block *out, const float *x, size_t n) {
    if (n % OR_QK_K) return OR_ERR_BLOCK_MULTIPLE;
    for (size_t b = 0; b < n / OR_QK_K; b++) {
        const float *c = x + b * OR_QK_K;
        or_q8k_block *o = &out[b];
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < OR_QK_K; j++) {
            float ax = fabsf(c[j]);
            if (ax > amax) {
                amax = ax;
                max = c[j];
            }
        }
        memset(o, 0, sizeof(*o));
        if (amax == 0.0f) continue;
        float iscale = -127.0f / max;
        for (int j = 0; j < OR_QK_K; j++) {
            int32_t v = or_nearest_int(iscale * c[j]);
            o->qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int i = 0; i < 16; i++) s += o->qs[16 * j + i];
            o->bsums[j] = s;
        }
        o->d = 1.0f / iscale;
    }
    return OR_OK;
}

/* ---------------------------------------------------------------------- */
/* a11: dot_q4_k_q8_k, quants.rs:312-360                                    */
/* ---------------------------------------------------------------------- */
float or_dot_q4_k_q8_k(const or_q8k_block *x, size_t nb, const uint8_t *w) {
    float sums[8] = {0};
    float sumf = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        const or_q8k_block *q8 = &x[b];
        const uint8_t *blk = w + b * OR_BLOCK_Q4_K;
        uint8_t sc[8], m[8];
        for (int g = 0; g < 8; g++) or_scale_min_k4(blk + 4, g, &sc[g], &m[g]);
        const uint8_t *qs = blk + 16;
        int32_t sumi[8] = {0};
        for (int e = 0; e < OR_QK_K; e++) {
            int pos = e % 64;
            uint8_t byte = qs[32 * (e / 64) + pos % 32];
            int32_t a = pos < 32 ? (byte & 0xF) : (byte >> 4);
            sumi[e % 8] += (int32_t)sc[e / 32] * a * (int32_t)q8->qs[e];
        }
        float d = q8->d * or_f16_to_f32(f16_at(blk));
        for (int k = 0; k < 8; k++) sums[k] += d * (float)sumi[k];
        int32_t minsum = 0;
        for (int g = 0; g < 16; g++) minsum += q8->bsums[g] * (int32_t)m[g / 2];
        float dmin = or_f16_to_f32(f16_at(blk + 2)) * q8->d;
        sumf -= dmin * (float)minsum;
    }
    float s = sumf;
    for (int k = 0; k < 8; k++) s += sums[k];
    return s;
}

/* a12: dot_q6_k_q8_k, quants.rs:371-412 */
float or_dot_q6_k_q8_k(const or_q8k_block *x, size_t nb, const uint8_t *w) {
    float sums[8] = {0};
    for (size_t b = 0; b < nb; b++) {
        const or_q8k_block *q8 = &x[b];
        const uint8_t *blk = w + b * OR_BLOCK_Q6_K;
        const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
        int32_t sumi[8] = {0};
        for (int e = 0; e < OR_QK_K; e++) {
            int pos = e % 128;
            uint8_t byte = ql[64 * (e / 128) + pos % 64];
            int nib = pos < 64 ? (byte & 0xF) : (byte >> 4);
            int hi2 = (qh[32 * (e / 128) + pos % 32] >> (2 * (pos / 32))) & 3;
            int32_t a = (nib | (hi2 << 4)) - 32;
            sumi[e % 8] += (int32_t)(int8_t)scales[e / 16] * a * (int32_t)q8->qs[e];
        }
        float d = q8->d * or_f16_to_f32(f16_at(blk + 208));
        for (int k = 0; k < 8; k++) sums[k] += d * (float)sumi[k];
    }
    float s = 0.0f;
    for (int k = 0; k < 8; k++) s += sums[k];
    return s;
}

/* a13: gemv_quant_q8k, quants.rs:474-515 (checks :482-505) */
int or_gemv_quant_q8k_mt(float *out, size_t out_len, const float *x,
                         size_t x_len, const uint8_t *w, size_t w_len,
                         size_t dim_in, size_t dim_out, int dtype,
                         int nthreads) {
    if (out_len != dim_out) return OR_ERR_LEN;
    if (x_len < dim_in) return OR_ERR_LEN;
    if (dtype != OR_Q4_K && dtype != OR_Q6_K) return OR_ERR_DTYPE;
    if (dim_in % OR_QK_K) return OR_ERR_BLOCK_MULTIPLE;
    size_t rb = or_row_bytes(dtype, dim_in);
    if (w_len != rb * dim_out) return OR_ERR_LEN;
    size_t nb = dim_in / OR_QK_K;
    or_q8k_block *xq = (or_q8k_block *)malloc((nb ? nb : 1) * sizeof(or_q8k_block));
    if (!xq) return OR_ERR_ALLOC;
    or_quantize_q8_k(xq, x, dim_in);
    rows_job proto = {out, x, w, dim_in, rb, 0, 0, dtype, xq, OR_OK};
    int rc = run_rows(gemv_q8k_rows, proto, dim_out, nthreads);
    free(xq);
    return rc;
}

int or_gemv_quant_q8k(float *out, size_t out_len, const float *x, size_t x_len,
                      const uint8_t *w, size_t w_len, size_t dim_in,
                      size_t dim_out, int dtype) {
    return or_gemv_quant_q8k_mt(out, out_len, x, x_len, w, w_len, dim_in,
                                dim_out, dtype, 1);
}

/* ---------------------------------------------------------------------- */
/* a14: dequantize_q4_k, quants.rs:534-567                                  */
/* ---------------------------------------------------------------------- */
int or_dequantize_q4_k(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len) {
    if (w_len != out_len / OR_QK_K * OR_BLOCK_Q4_K) return OR_ERR_LEN;
    if (out_len % OR_QK_K) return OR_ERR_LEN; /* final assert_eq!(e, len) */
    size_t e = 0;
    for (size_t b = 0; b < out_len / OR_QK_K; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q4_K;
        float d = or_f16_to_f32(f16_at(blk));
        float min = or_f16_to_f32(f16_at(blk + 2));
        const uint8_t *scales = blk + 4, *qs = blk + 16;
        for (int is = 0; is < 8; is += 2) {
            uint8_t sc0, m0, sc1, m1s;
            or_scale_min_k4(scales, is, &sc0, &m0);
            float d1 = d * (float)sc0;
            float m1 = min * (float)m0;
            or_scale_min_k4(scales, is + 1, &sc1, &m1s);
            float d2 = d * (float)sc1;
            float m2 = min * (float)m1s;
            for (int l = 0; l < 32; l++) out[e++] = d1 * (float)(qs[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) out[e++] = d2 * (float)(qs[l] >> 4) - m2;
            qs += 32;
        }
    }
    return OR_OK;
}

int or_dequantize_q6_k(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len) {
    if (out_len % OR_QK_K || w_len != out_len / OR_QK_K * OR_BLOCK_Q6_K)
        return OR_ERR_LEN;
    for (size_t b = 0; b < out_len / OR_QK_K; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q6_K;
        const uint8_t *ql = blk, *qh = blk + 128, *scales = blk + 192;
        float d = or_f16_to_f32(f16_at(blk + 208));
        for (int e = 0; e < OR_QK_K; e++) {
            uint8_t byte = ql[64 * (e / 128) + (e % 64)];
            int nib = ((e / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
            int hi2 = (qh[(e % 32) + 32 * (e / 128)] >> (2 * ((e % 128) / 32))) & 3;
            int q = (nib | (hi2 << 4)) - 32;
            float sc = (float)(int8_t)scales[e / 16];
            out[b * OR_QK_K + e] = d * (sc * (float)q);
        }
    }
    return OR_OK;
}

int or_dequantize_q8_0(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len) {
    if (out_len % OR_QK8_0 || w_len != out_len / OR_QK8_0 * OR_BLOCK_Q8_0)
        return OR_ERR_LEN;
    for (size_t b = 0; b < out_len / OR_QK8_0; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q8_0;
        float d = or_f16_to_f32(f16_at(blk));
        for (int e = 0; e < OR_QK8_0; e++)
            out[b * OR_QK8_0 + e] = d * (float)(int8_t)blk[2 + e];
    }
    return OR_OK;
}

/* ---------------------------------------------------------------------- */
/* Integer unpack exports (element maps of quants.rs:146-151, :185-194)     */
/* ---------------------------------------------------------------------- */
int or_unpack_q4_k(const uint8_t *w, size_t nblocks, uint8_t *q, uint8_t *sc,
                   uint8_t *m, float *d, float *dmin) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q4_K;
        d[b] = or_f16_to_f32(f16_at(blk));
        dmin[b] = or_f16_to_f32(f16_at(blk + 2));
        for (int g = 0; g < 8; g++) or_scale_min_k4(blk + 4, g, &sc[8 * b + g], &m[8 * b + g]);
        for (int e = 0; e < OR_QK_K; e++) {
            int g = e / 32;
            uint8_t byte = blk[16 + 32 * (g / 2) + (e % 32)];
            q[OR_QK_K * b + e] = (g % 2 == 0) ? (byte & 0xF) : (byte >> 4);
        }
    }
    return OR_OK;
}

int or_unpack_q6_k(const uint8_t *w, size_t nblocks, uint8_t *q, int8_t *sc,
                   float *d) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q6_K;
        const uint8_t *ql = blk, *qh = blk + 128;
        d[b] = or_f16_to_f32(f16_at(blk + 208));
        for (int j = 0; j < 16; j++) sc[16 * b + j] = (int8_t)blk[192 + j];
        for (int e = 0; e < OR_QK_K; e++) {
            uint8_t byte = ql[64 * (e / 128) + (e % 64)];
            int nib = ((e / 64) % 2 == 0) ? (byte & 0xF) : (byte >> 4);
            int hi2 = (qh[(e % 32) + 32 * (e / 128)] >> (2 * ((e % 128) / 32))) & 3;
            q[OR_QK_K * b + e] = (uint8_t)(nib | (hi2 << 4)); /* raw 0..63 */
        }
    }
    return OR_OK;
}

int or_unpack_q8_0(const uint8_t *w, size_t nblocks, int8_t *q, float *d) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t *blk = w + b * OR_BLOCK_Q8_0;
        d[b] = or_f16_to_f32(f16_at(blk));
        for (int e = 0; e < OR_QK8_0; e++) q[OR_QK8_0 * b + e] = (int8_t)blk[2 + e];
    }
    return OR_OK;
}

/* ---------------------------------------------------------------------- */
/* a15: swiglu, kernels.rs:174-182; silu, kernels.rs:207-212                */
/* ---------------------------------------------------------------------- */
void or_swiglu(float *out, const float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float t = gate[i];
        float s = t / (1.0f + expf(-t));
        out[i] = s * up[i];
    }
}

void or_silu(float *out, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] / (1.0f + expf(-x[i]));
}
