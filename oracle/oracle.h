/*
 * oracle.h -- CPU restatement of unltd-inference's quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle the GPU kernels are
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library (libuq) never links,
 * loads or calls it.
 *
 * Every function restates one function of the reference, cited file:line
 * (paths relative to the reference repository root):
 *   crates/unltd-tensor/src/quants.rs   -- block decode, dots, GEMV, Q8_K
 *   crates/unltd-tensor/src/kernels.rs  -- pairwise_sum_f64, swiglu, silu, and
 *                                          the per-layer ops (oracle_ops.c)
 *   crates/unltd-generation/src/min_forward.rs -- dtype ids, row bytes
 * Functions marked "closed form" have no reference kernel (Q8_0 decode, Q6_K
 * and Q8_0 f32 dequantization, integer unpack exports); they follow the GGUF
 * block definitions the reference documents and the numeric contract of the
 * neighbouring reference functions.
 *
 * Reference panics (assert_eq!/panic!) become OR_ERR_* return codes here.
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (oracle/Makefile).
 */
#ifndef UQ_ORACLE_H
#define UQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, as accepted by dtype_of (min_forward.rs:39-48). */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14 };

/* Status codes: one per reference panic class. */
enum {
    OR_OK = 0,
    OR_ERR_LEN = 1,            /* assert_eq!(len ...) failed            */
    OR_ERR_BLOCK_MULTIPLE = 2, /* dim_in % QK_K != 0 (or % 32 for Q8_0) */
    OR_ERR_DTYPE = 3,          /* panic!("... sin dot implementado")     */
    OR_ERR_ALLOC = 4,
    OR_ERR_RANGE = 5           /* assert!(id in range) failed            */
};

#define OR_QK_K 256
#define OR_QK8_0 32
#define OR_BLOCK_Q4_K 144
#define OR_BLOCK_Q6_K 210
#define OR_BLOCK_Q8_0 34

/* quants.rs:235-242 */
typedef struct {
    float d;
    int8_t qs[256];
    int32_t bsums[16];
} or_q8k_block;

/* quants.rs:44-72 */
float or_f16_to_f32(uint16_t h);
/* quants.rs:92-102 */
void or_scale_min_k4(const uint8_t *s, int g, uint8_t *sc, uint8_t *m);
/* kernels.rs:27-42 (same tree, caller-provided scratch of n doubles) */
double or_pairwise_sum_f64(const double *vals, size_t n, double *scratch);
/* quants.rs:106-114 */
double or_dot_f32(const float *x, const float *w, size_t n);
/* quants.rs:132-156 */
double or_dot_q4_k(const float *x, const uint8_t *w, size_t n);
/* quants.rs:171-200 */
double or_dot_q6_k(const float *x, const uint8_t *w, size_t n);
/* closed form: dot_q4_k's contract with w = d*q of a GGUF Q8_0 block */
double or_dot_q8_0(const float *x, const uint8_t *w, size_t n);
/* min_forward.rs:52-80; returns 0 on a refused (dtype, n) pair */
size_t or_row_bytes(int dtype, size_t n);
/* quants.rs:422-466; Q8_0 accepted as a closed-form extension */
int or_gemv_quant(float *out, size_t out_len, const float *x, size_t x_len,
                  const uint8_t *w, size_t w_len, size_t dim_in, size_t dim_out,
                  int dtype);
/* Same as or_gemv_quant, rows split over nthreads (min_forward.rs:245-264). */
int or_gemv_quant_mt(float *out, size_t out_len, const float *x, size_t x_len,
                     const uint8_t *w, size_t w_len, size_t dim_in,
                     size_t dim_out, int dtype, int nthreads);

/* quants.rs:230-233 */
int32_t or_nearest_int(float fval);
/* quants.rs:250-290; out must hold n/256 blocks */
int or_quantize_q8_k(or_q8k_block *out, const float *x, size_t n);
/* quants.rs:312-360 */
float or_dot_q4_k_q8_k(const or_q8k_block *x, size_t nb, const uint8_t *w);
/* quants.rs:371-412 */
float or_dot_q6_k_q8_k(const or_q8k_block *x, size_t nb, const uint8_t *w);
/* quants.rs:474-515 */
int or_gemv_quant_q8k(float *out, size_t out_len, const float *x, size_t x_len,
                      const uint8_t *w, size_t w_len, size_t dim_in,
                      size_t dim_out, int dtype);
int or_gemv_quant_q8k_mt(float *out, size_t out_len, const float *x,
                         size_t x_len, const uint8_t *w, size_t w_len,
                         size_t dim_in, size_t dim_out, int dtype, int nthreads);

/* quants.rs:534-567 */
int or_dequantize_q4_k(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len);
/* closed form: w = d * (sc * q), the exact product dot_q6_k builds (:195) */
int or_dequantize_q6_k(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len);
/* closed form: w = d * q */
int or_dequantize_q8_0(float *out, size_t out_len, const uint8_t *w,
                       size_t w_len);

/* Integer unpack (closed form of the element maps at quants.rs:146-151,
 * :185-194). Per block: q[256] nibble / 6-bit raw (0..63) / int8 quant,
 * per-group scales, and the f32 block scales. */
int or_unpack_q4_k(const uint8_t *w, size_t nblocks, uint8_t *q, uint8_t *sc,
                   uint8_t *m, float *d, float *dmin);
int or_unpack_q6_k(const uint8_t *w, size_t nblocks, uint8_t *q, int8_t *sc,
                   float *d);
int or_unpack_q8_0(const uint8_t *w, size_t nblocks, int8_t *q, float *d);

/* kernels.rs:174-182 */
void or_swiglu(float *out, const float *gate, const float *up, size_t n);
/* kernels.rs:207-212 */
void or_silu(float *out, const float *x, size_t n);

/* Per-layer non-linear kernels (oracle_ops.c), kernels.rs: */
/* :61-78 rmsnorm: sequential f64 sum of f32 squares, f32 scale */
int or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
/* :236-256 l2_norm_rows, in place over len/dim rows */
int or_l2_norm_rows(float *data, size_t len, size_t dim, float eps);
/* :157-168 softmax: f32 exp, pairwise f64 denominator, f64 division */
int or_softmax(float *out, const float *x, size_t n, float scale);
/* :198-203 sigmoid; :217-228 softplus */
void or_sigmoid(float *out, const float *x, size_t n);
void or_softplus(float *out, const float *x, size_t n);
/* :265-305 ssm_conv */
int or_ssm_conv(float *out, size_t out_len, const float *x, size_t x_len, const float *kernel,
                size_t kernel_len, size_t d_conv, size_t channels);
/* :316-375 gdn_fused_step; state is dim x dim, row i = product dim */
int or_gdn_fused_step(float *state, float *out, const float *q, const float *k, const float *v, size_t dim,
                      float gate, float beta, float scale);
/* :109-125, :131-148, :381-400 */
int or_rope_llama(float *x, size_t n, const float *freqs, size_t nfreq, size_t pos);
int or_rope_neox(float *x, size_t n, const float *freqs, size_t nfreq, size_t pos);
int or_rope_imrope(float *x, size_t n, size_t n_rot, double theta_scale, size_t pos);
/* kernels.rs:87-101: acc[m][n] = f32((f64)acc + pairwise f64 sum of a*b over k). */
int or_matmul_f32_acc(float *acc, const float *a, const float *b, size_t m, size_t k, size_t n);
/* kernels.rs:185-194 */
void or_gelu_tanh(float *out, const float *x, size_t n);
/* kernels.rs:402-422: OR_ERR_LEN for the length asserts, OR_ERR_RANGE for an id past the table. */
int or_embedding_lookup(float *out, size_t out_len, const float *table, size_t table_len, const uint32_t *ids,
                        size_t n_ids, size_t dim);
/* qwen35_forward.rs:639-671: causal attention of one decode position.
 * q and out are [n_head][hd]; the caches are [n_ctx][n_head_kv][hd]; soft
 * [n_head][n_ctx] receives each head's softmax weights. */
int or_attn_decode(float *out, float *soft, const float *q, const float *k_cache, const float *v_cache, size_t n_ctx,
                   size_t n_head, size_t n_head_kv, size_t hd, float kq_scale);

#ifdef __cplusplus
}
#endif
#endif
