/*
 * uq_ops.h -- per-layer kernels of libuq.so: every public function of
 * crates/unltd-tensor/src/kernels.rs (the ones the Qwen3.5 forward runs
 * between its quantized projections, and the rest of that file's surface)
 * plus the decode attention of qwen35_forward.rs, so activations can stay in
 * HBM from one layer to the next.
 *
 * Each function has a host-pointer mirror with the reference's arguments
 * (slices as pointer + length; panics as uq_status codes, UQ_ERR_LEN for the
 * length asserts) and a device form (suffix _d: device pointers, several
 * rows per call, asynchronous on the given stream, no allocation).
 *
 * Numerics (checked against the oracle):
 *  - rmsnorm, l2_norm_rows, ssm_conv, gdn_fused_step (given exp(gate)) and
 *    the softmax denominator follow the reference's f32 / f64 steps and
 *    summation orders exactly; the sequential f64 sums of rmsnorm and
 *    l2_norm_rows are proven equal through a rounding bound, or replayed.
 *  - exp / log are the f64 functions rounded once to f32 (correctly rounded
 *    but for rare near-midpoint arguments); the reference calls the
 *    platform libm, so sigmoid, silu, softplus, softmax and the gdn decay
 *    agree with it within 1-2 ulp.
 *  - the rope rotations use the device's f64 sin / cos; results agree with
 *    the reference except when its libm and the device differ in the last
 *    f64 bit in a way that changes the f32 rounding.
 */
#ifndef UQ_OPS_H
#define UQ_OPS_H

#include "uq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* rmsnorm (kernels.rs:61-78): out = (x * scale) * w, scale = 1/sqrtf(mean(x^2) + eps).
 * Panics: len(out) != len(x), len(x) != len(w). */
uq_status uq_rmsnorm(float *out, size_t out_len, const float *x, size_t x_len, const float *w, size_t w_len,
                     float eps);
/* rows rows of n, each normalised with the same w[n]. */
uq_status uq_rmsnorm_d(float *d_out, const float *d_x, const float *d_w, size_t n, size_t rows, float eps,
                       void *stream);

/* l2_norm_rows (kernels.rs:236-256), in place over len/dim rows.
 * Panics: len % dim != 0. */
uq_status uq_l2_norm_rows(float *data, size_t len, size_t dim, float eps);
uq_status uq_l2_norm_rows_d(float *d_data, size_t len, size_t dim, float eps, void *stream);

/* softmax (kernels.rs:157-168). Panics: len(out) != len(x). Rows of up to
 * 2^24 values (UQ_ERR_ARG above); the device form may run in place. */
uq_status uq_softmax(float *out, size_t out_len, const float *x, size_t x_len, float scale);
uq_status uq_softmax_d(float *d_out, const float *d_x, size_t n, size_t rows, float scale, void *stream);

/* sigmoid (kernels.rs:198-203), silu (:207-212), softplus (:217-228).
 * Panics: len(out) != len(x). */
uq_status uq_sigmoid(float *out, size_t out_len, const float *x, size_t x_len);
uq_status uq_silu(float *out, size_t out_len, const float *x, size_t x_len);
uq_status uq_softplus(float *out, size_t out_len, const float *x, size_t x_len);
uq_status uq_sigmoid_d(float *d_out, const float *d_x, size_t n, void *stream);
uq_status uq_silu_d(float *d_out, const float *d_x, size_t n, void *stream);
uq_status uq_softplus_d(float *d_out, const float *d_x, size_t n, void *stream);

/* ssm_conv (kernels.rs:265-305): x is [ncs, channels], kernel [d_conv,
 * channels], out [n_t, channels] with n_t = ncs - (d_conv - 1).
 * Panics: len(x) % channels, ncs < d_conv, len(kernel), len(out). */
uq_status uq_ssm_conv(float *out, size_t out_len, const float *x, size_t x_len, const float *kernel,
                      size_t kernel_len, size_t d_conv, size_t channels);
uq_status uq_ssm_conv_d(float *d_out, const float *d_x, size_t x_len, const float *d_kernel, size_t d_conv,
                        size_t channels, void *stream);

/* gdn_fused_step (kernels.rs:316-375) of one head: state is dim x dim,
 * S[i][j] at i*dim + j. Panics: len(k), len(v), len(out) != dim = len(q),
 * len(state) != dim*dim. */
uq_status uq_gdn_fused_step(float *state, size_t state_len, float *out, size_t out_len, const float *q,
                            size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len, float gate,
                            float beta, float scale);
/* heads heads at once: state [heads][dim][dim], q/k/v/out [heads][dim],
 * gate/beta [heads] (the caller maps q/k heads to v heads, as the
 * reference's caller does). */
uq_status uq_gdn_fused_step_d(float *d_state, float *d_out, const float *d_q, const float *d_k, const float *d_v,
                              const float *d_gate, const float *d_beta, size_t dim, size_t heads, float scale,
                              void *stream);

/* ---- Off the Qwen3.5 forward's path --------------------------------------
 * The forward imports dot_f32, gdn_fused_step, gemv_quant_q8k, l2_norm_rows,
 * rmsnorm, rope_apply_imrope, sigmoid, silu, softmax, softplus, ssm_conv and
 * swiglu from unltd-tensor (qwen35_forward.rs:38-41). rope_apply_llama,
 * rope_apply_neox, gelu_tanh and matmul_f32_acc below are the rest of
 * kernels.rs's public surface: exported for callers of that surface, not
 * used by any layer of this library (uq_layer.h) and not tuned.
 * ------------------------------------------------------------------------ */

/* rope_apply_llama (kernels.rs:109-125) and rope_apply_neox (:131-148), in
 * place. Panics: len(x) odd, len(freqs) < len(x)/2. */
uq_status uq_rope_llama(float *x, size_t x_len, const float *freqs, size_t freqs_len, size_t pos);
uq_status uq_rope_neox(float *x, size_t x_len, const float *freqs, size_t freqs_len, size_t pos);
/* rows rows of n at the same position; d_freqs holds n/2 values. */
uq_status uq_rope_llama_d(float *d_x, size_t n, size_t rows, const float *d_freqs, size_t pos, void *stream);
uq_status uq_rope_neox_d(float *d_x, size_t n, size_t rows, const float *d_freqs, size_t pos, void *stream);

/* rope_apply_imrope (kernels.rs:381-400), in place. Panics: n_rot odd,
 * n_rot > len(x). */
uq_status uq_rope_imrope(float *x, size_t x_len, size_t n_rot, double theta_scale, size_t pos);
uq_status uq_rope_imrope_d(float *d_x, size_t n, size_t rows, size_t n_rot, double theta_scale, size_t pos,
                           void *stream);

/* gelu_tanh (kernels.rs:185-194), in f64 with the device's tanh: within
 * 1 ulp of the reference (its libm tanh may differ in the last f64 bit).
 * Panics: len(out) != len(x). */
uq_status uq_gelu_tanh(float *out, size_t out_len, const float *x, size_t x_len);
uq_status uq_gelu_tanh_d(float *d_out, const float *d_x, size_t n, void *stream);

/* matmul_f32_acc (kernels.rs:87-101): acc[m][n] += a[m][k] @ b[k][n], each
 * element f32((f64)acc + pairwise f64 sum of the exact products), bit-exact.
 * Panics: len(a) != m*k, len(b) != k*n, len(acc) != m*n. k <= 2^18
 * (UQ_ERR_ARG above). */
uq_status uq_matmul_f32_acc(float *acc, size_t acc_len, const float *a, size_t a_len, const float *b, size_t b_len,
                            size_t m, size_t k, size_t n);
uq_status uq_matmul_f32_acc_d(float *d_acc, const float *d_a, const float *d_b, size_t m, size_t k, size_t n,
                              void *stream);

/* embedding_lookup (kernels.rs:402-422): row copies of an f32 table.
 * Panics: len(table) % dim, len(out) != len(ids) * dim (UQ_ERR_LEN); an id
 * past the table is UQ_ERR_TOKEN, checked for every id before any copy.
 * The device form takes the ids from host memory, as uq_embed does. */
uq_status uq_embedding_lookup(float *out, size_t out_len, const float *table, size_t table_len, const uint32_t *ids,
                              size_t n_ids, size_t dim);
uq_status uq_embedding_lookup_d(float *d_out, const float *d_table, size_t table_len, const uint32_t *ids,
                                size_t n_ids, size_t dim, void *stream);

/* The causal attention of one decode position, step 5 of attn_layer
 * (qwen35_forward.rs:639-671): for each q head h, with kv head
 * h / (n_head / n_head_kv),
 *   scores[p] = (f32) dot_f32(q_h, K[p][kv])   (f64 products, pairwise sum)
 *   soft_h    = softmax(scores, kq_scale)
 *   out_h[i]  = (f32) sum over p, in order, of (f64) soft_h[p] * V[p][kv][i].
 * q and out are [n_head][head_dim]; the caches hold rows [p][n_head_kv]
 * [head_dim], as the reference's k_cache / v_cache slots; soft [n_head]
 * [n_ctx] receives the weights. Bit-exact with the reference (softmax's
 * expf aside, as softmax). Limits: head_dim in {64, 128, 256, 512},
 * n_head / n_head_kv <= 8, 1 <= n_ctx <= 2^24 (UQ_ERR_ARG otherwise).
 * Panics of the host form: len(q), len(out) != n_head * head_dim,
 * len(k_cache) or len(v_cache) < n_ctx * n_head_kv * head_dim (the
 * reference's cache slices). */
uq_status uq_attn_decode(float *out, size_t out_len, const float *q, size_t q_len, const float *k_cache,
                         size_t k_len, const float *v_cache, size_t v_len, size_t n_ctx, size_t n_head,
                         size_t n_head_kv, size_t head_dim, float kq_scale);
uq_status uq_attn_decode_d(float *d_out, float *d_soft, const float *d_q, const float *d_k_cache,
                           const float *d_v_cache, size_t n_ctx, size_t n_head, size_t n_head_kv, size_t head_dim,
                           float kq_scale, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* UQ_OPS_H */
