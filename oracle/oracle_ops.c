/*
 * oracle_ops.c -- CPU restatement of the reference's per-layer non-linear
 * kernels (crates/unltd-tensor/src/kernels.rs). TEST INFRASTRUCTURE ONLY,
 * like oracle.c: the device kernels of uq_ops.hip are checked against it.
 *
 * Each function follows the cited reference function step for step: f32
 * operations stay f32 (no contraction: -ffp-contract=off), f64 sums keep
 * their order (sequential or the pairwise tree), Rust's f64::mul_add is C's
 * fma, f32::exp / ln / sqrt are expf / logf / sqrtf and f64::sin_cos is
 * sin / cos of the C library.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* kernels.rs:61-78 */
int or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    if (n == 0) return OR_OK;
    double sum = 0.0;
    for (size_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; i++) {
        const float norm = x[i] * scale;
        out[i] = norm * w[i];
    }
    return OR_OK;
}

/* kernels.rs:236-256 */
int or_l2_norm_rows(float *data, size_t len, size_t dim, float eps) {
    if (dim == 0 || len % dim) return OR_ERR_LEN;
    for (size_t r = 0; r < len / dim; r++) {
        float *row = data + r * dim;
        double sum = 0.0;
        for (size_t i = 0; i < dim; i++) sum += (double)(row[i] * row[i]);
        const float scale = 1.0f / fmaxf(sqrtf((float)sum), eps); /* f32::max */
        for (size_t i = 0; i < dim; i++) row[i] *= scale;
    }
    return OR_OK;
}

/* kernels.rs:157-168 */
int or_softmax(float *out, const float *x, size_t n, float scale) {
    if (n == 0) return OR_OK;
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = fmaxf(mx, x[i]);
    double *e = malloc(2 * n * sizeof(double));
    float *ef = malloc(n * sizeof(float));
    if (!e || !ef) {
        free(e);
        free(ef);
        return OR_ERR_ALLOC;
    }
    for (size_t i = 0; i < n; i++) {
        ef[i] = expf((x[i] - mx) * scale);
        e[i] = (double)ef[i];
    }
    const double sum = or_pairwise_sum_f64(e, n, e + n);
    for (size_t i = 0; i < n; i++) out[i] = (float)((double)ef[i] / sum);
    free(e);
    free(ef);
    return OR_OK;
}

/* kernels.rs:198-203 */
void or_sigmoid(float *out, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = 1.0f / (1.0f + expf(-x[i]));
}

/* kernels.rs:217-228 */
void or_softplus(float *out, const float *x, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = x[i] > 20.0f ? x[i] : logf(1.0f + expf(x[i]));
}

/* kernels.rs:265-305: out[t*channels + c], sequential f32 sum over tau */
int or_ssm_conv(float *out, size_t out_len, const float *x, size_t x_len, const float *kernel,
                size_t kernel_len, size_t d_conv, size_t channels) {
    if (channels == 0 || x_len % channels) return OR_ERR_LEN;
    const size_t ncs = x_len / channels;
    if (ncs < d_conv || d_conv == 0) return OR_ERR_LEN;
    if (kernel_len != d_conv * channels) return OR_ERR_LEN;
    const size_t n_t = ncs - (d_conv - 1);
    if (out_len != channels * n_t) return OR_ERR_LEN;
    for (size_t t = 0; t < n_t; t++)
        for (size_t c = 0; c < channels; c++) {
            float s = 0.0f;
            for (size_t tau = 0; tau < d_conv; tau++) s += x[(t + tau) * channels + c] * kernel[tau * channels + c];
            out[t * channels + c] = s;
        }
    return OR_OK;
}

/* kernels.rs:316-375 */
int or_gdn_fused_step(float *state, float *out, const float *q, const float *k, const float *v, size_t dim,
                      float gate, float beta, float scale) {
    float *d = malloc((dim ? dim : 1) * sizeof(float));
    if (!d) return OR_ERR_ALLOC;
    const float g_exp = expf(gate);
    for (size_t i = 0; i < dim * dim; i++) state[i] *= g_exp;
    for (size_t j = 0; j < dim; j++) {
        double sum = 0.0;
        for (size_t i = 0; i < dim; i++) sum += (double)(state[i * dim + j] * k[i]);
        d[j] = (v[j] - (float)sum) * beta;
    }
    for (size_t j = 0; j < dim; j++)
        for (size_t i = 0; i < dim; i++) state[i * dim + j] += k[i] * d[j];
    for (size_t j = 0; j < dim; j++) {
        double sum = 0.0;
        for (size_t i = 0; i < dim; i++) sum += (double)(state[i * dim + j] * q[i]);
        out[j] = (float)sum * scale;
    }
    free(d);
    return OR_OK;
}

/* the rotation of the rope functions: x0' = c.mul_add(x0, -(s*x1)),
 * x1' = s.mul_add(x0, c*x1), in f64, rounded to f32 */
static void rotate(float *a, float *b, double angle) {
    const double s = sin(angle), c = cos(angle);
    const double x0 = (double)*a, x1 = (double)*b;
    *a = (float)fma(c, x0, -(s * x1));
    *b = (float)fma(s, x0, c * x1);
}

/* kernels.rs:109-125: pairs (2i, 2i+1) */
int or_rope_llama(float *x, size_t n, const float *freqs, size_t nfreq, size_t pos) {
    if (n % 2 || nfreq < n / 2) return OR_ERR_LEN;
    for (size_t i = 0; i < n / 2; i++) rotate(&x[2 * i], &x[2 * i + 1], (double)pos * (double)freqs[i]);
    return OR_OK;
}

/* kernels.rs:131-148: pairs (i, i + n/2) */
int or_rope_neox(float *x, size_t n, const float *freqs, size_t nfreq, size_t pos) {
    if (n % 2 || nfreq < n / 2) return OR_ERR_LEN;
    const size_t half = n / 2;
    for (size_t i = 0; i < half; i++) rotate(&x[i], &x[i + half], (double)pos * (double)freqs[i]);
    return OR_OK;
}

/* kernels.rs:381-400: pairs (ic, ic + n_rot/2) of the first n_rot dims, only
 * ic % 3 == 0; the angle is multiplied by theta_scale for every pair */
int or_rope_imrope(float *x, size_t n, size_t n_rot, double theta_scale, size_t pos) {
    if (n_rot % 2 || n_rot > n) return OR_ERR_LEN;
    const size_t half = n_rot / 2;
    double angle = (double)pos;
    for (size_t ic = 0; ic < half; ic++) {
        if (ic % 3 == 0) rotate(&x[ic], &x[ic + half], angle);
        angle *= theta_scale;
    }
    return OR_OK;
}

/* qwen35_forward.rs:639-671, step 5 of attn_layer: q head h reads kv head
 * h / (n_head / n_head_kv); scores[p] = (f32) dot_f32(q_h, K[p]) (f64
 * products, pairwise sum); soft = softmax(scores, kq_scale); out_h[i] =
 * (f32) of the sequential f64 sum over p of soft[p] * V[p][i]. */
int or_attn_decode(float *out, float *soft, const float *q, const float *k_cache, const float *v_cache, size_t n_ctx,
                   size_t n_head, size_t n_head_kv, size_t hd, float kq_scale) {
    if (n_head_kv == 0 || n_head % n_head_kv || n_ctx == 0) return OR_ERR_LEN;
    const size_t group = n_head / n_head_kv, kv_len = n_head_kv * hd;
    float *scores = malloc(n_ctx * sizeof(float));
    if (!scores) return OR_ERR_ALLOC;
    for (size_t h = 0; h < n_head; h++) {
        const size_t kv = h / group;
        float *sh = soft + h * n_ctx;
        for (size_t p = 0; p < n_ctx; p++) scores[p] = (float)or_dot_f32(q + h * hd, k_cache + p * kv_len + kv * hd, hd);
        const int rc = or_softmax(sh, scores, n_ctx, kq_scale);
        if (rc != OR_OK) {
            free(scores);
            return rc;
        }
        for (size_t i = 0; i < hd; i++) {
            double sum = 0.0;
            for (size_t p = 0; p < n_ctx; p++) sum += (double)sh[p] * (double)v_cache[p * kv_len + kv * hd + i];
            out[h * hd + i] = (float)sum;
        }
    }
    free(scores);
    return OR_OK;
}

/* kernels.rs:87-101: products in f64, pairwise sum, accumulate in f64, one f32 rounding */
int or_matmul_f32_acc(float *acc, const float *a, const float *b, size_t m, size_t k, size_t n) {
    double *prods = malloc((2 * k + 1) * sizeof(double));
    if (!prods) return OR_ERR_ALLOC;
    for (size_t i = 0; i < m; i++)
        for (size_t j = 0; j < n; j++) {
            for (size_t l = 0; l < k; l++) prods[l] = (double)a[i * k + l] * (double)b[l * n + j];
            const double sum = or_pairwise_sum_f64(prods, k, prods + k);
            acc[i * n + j] = (float)((double)acc[i * n + j] + sum);
        }
    free(prods);
    return OR_OK;
}

/* kernels.rs:185-194: 0.5 t (1 + tanh(sqrt(2/pi) (t + 0.044715 t^3))) in f64, left to right */
void or_gelu_tanh(float *out, const float *x, size_t n) {
    const double s2pi = 0.7978845608028654, c = 0.044715;
    for (size_t i = 0; i < n; i++) {
        const double t = (double)x[i];
        const double inner = s2pi * (t + c * t * t * t);
        out[i] = (float)(0.5 * t * (1.0 + tanh(inner)));
    }
}

/* kernels.rs:402-422: row copies; the length asserts first, then each id in order */
int or_embedding_lookup(float *out, size_t out_len, const float *table, size_t table_len, const uint32_t *ids,
                        size_t n_ids, size_t dim) {
    if (dim == 0 || table_len % dim) return OR_ERR_LEN;
    if (out_len != n_ids * dim) return OR_ERR_LEN;
    for (size_t r = 0; r < n_ids; r++) {
        const size_t src = (size_t)ids[r] * dim;
        if (src + dim > table_len) return OR_ERR_RANGE;
        memcpy(out + r * dim, table + src, dim * sizeof(float));
    }
    return OR_OK;
}

