// Internal declarations shared by the C-ABI host code and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/uq.h"

// Device copies of weights carry this many bytes of zero padding after the
// tensor, so that dword windows of the last block (Q6_K scales/d, Q8_0 pairs)
// never read past the allocation.
#define UQ_WEIGHT_PAD 256

struct uq_weights_s {
    uint32_t magic;
    int device;
    uq_dtype dtype;
    size_t dim_in, dim_out, row_bytes, nbytes;
    uint8_t *d_bytes;  // nbytes + UQ_WEIGHT_PAD, 256-byte aligned
};
#define UQ_WEIGHTS_MAGIC 0x55515754u

namespace uq {

// Block geometry (quants.rs:33-39, gguf.rs:202).
constexpr int QK_K = 256;
constexpr int QK8_0 = 32;
constexpr int BQ4K = 144;
constexpr int BQ6K = 210;
constexpr int BQ8_0 = 34;

// Allows kernel to take lds bytes of dynamic LDS (above the 64 KB default)
// on the current device; a no-op after the first call per kernel and device.
hipError_t allow_lds(const void *kernel, size_t lds);

// Relaxes the calling thread's stream-capture mode for the guard's lifetime,
// so that one-time set-up calls (function attributes, symbol addresses) made
// by the first call of an entry point stay legal when that call is being
// captured into a HIP graph; the previous mode is restored after.
struct RelaxedCapture {
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    RelaxedCapture() { (void)hipThreadExchangeStreamCaptureMode(&mode); }
    ~RelaxedCapture() { (void)hipThreadExchangeStreamCaptureMode(&mode); }
    RelaxedCapture(const RelaxedCapture &) = delete;
    RelaxedCapture &operator=(const RelaxedCapture &) = delete;
};

// The activation planes of the q8k GEMM's workspace for M rows of dim_in K,
// rows padded to Mp: octet o of fragment F = 16 b + 2 l + h of row m at
// a + ((2 F + o) Mp + m) 16 (eight f16); the 16 bsums of (block b, row m) as
// f16 at bs + (b Mp + m) 32; q8.d of (b, m) at d8[b Mp + m].
struct Q8Planes {
    uint8_t *a, *bs;
    float *d8;
    int Mp;
};

// Per-layer non-linear ops (uq_ops.hip).
hipError_t launch_rmsnorm(float *out, const float *x, const float *w, int n, int rows, float eps, hipStream_t s);
// rows of n, xs / ys floats apart in x / out; xb: normalise x + xb, written
// to xsum when given; z: multiply the output by silu(z) (z laid out as out);
// q8: the outputs also quantized into these planes (all q8->Mp rows, the
// padding rows as zero blocks; the Q6_K operand order when q6), as the q8k
// GEMM's prep would quantize them, where rmsnorm_q8k_fits(n, rows)
hipError_t launch_rmsnorm_rows(float *out, int ys, const float *x, int xs, const float *w, int n, int rows, float eps,
                               hipStream_t s, const float *xb = nullptr, float *xsum = nullptr,
                               const float *z = nullptr, const Q8Planes *q8 = nullptr, bool q6 = false);
inline bool rmsnorm_q8k_fits(int n, int rows) { return rows >= 1 && n >= 256 && n <= 4096 && n % 256 == 0; }
hipError_t launch_l2norm(float *data, int dim, int rows, float eps, hipStream_t s);
int softmax_max_len();
hipError_t launch_softmax(float *out, const float *x, int n, int rows, float scale, hipStream_t s);
hipError_t launch_unary(int op, const float *x, size_t n, float *out, hipStream_t s);  // 0 sigmoid, 1 silu, 2 softplus
hipError_t launch_ssm_conv(float *out, const float *x, const float *kern, int d_conv, int channels, int n_t,
                           hipStream_t s);
// v head h takes q/k head h % n_qk (n_qk 0: heads, one q/k head per v head)
hipError_t launch_gdn_step(float *state, float *out, const float *q, const float *k, const float *v, const float *gate,
                           const float *beta, int dim, int heads, float scale, hipStream_t s, int n_qk = 0);
// layer glue: GatedDeltaNet gates, out = y * act(z) (op 0 sigmoid, 1 silu;
// z index (i / n) * zs + i % n), out = a + b
hipError_t launch_gdn_gates(const float *beta_raw, const float *alpha, const float *dt_bias, const float *a,
                            float *beta, float *sp, float *gate, int n, hipStream_t s);
// one token of the GatedDeltaNet conv: conv over the window with the GGUF
// kernel [channels][d_conv] into raw, silu into act, the window shifted up
hipError_t launch_conv_step(float *win, const float *kern_gguf, float *raw, float *act, int d_conv, int channels,
                            hipStream_t s);
hipError_t launch_mul_act(int op, float *out, const float *y, const float *z, int n, int zs, size_t total,
                          hipStream_t s);
hipError_t launch_add(float *out, const float *a, const float *b, size_t n, hipStream_t s);
hipError_t launch_rope_freq(int mode, float *x, int rows, int n, const float *freqs, size_t pos, hipStream_t s);
hipError_t launch_rope_imrope(float *x, int rows, int n, int n_rot, double theta_scale, size_t pos, hipStream_t s);
// matmul_f32_acc, k <= matmul_max_k()
int matmul_max_k();
hipError_t launch_matmul_acc(float *acc, const float *a, const float *b, int m, int k, int n, hipStream_t s);
// decode attention: hd in {64, 128, 256, 512}, 1 <= group <= 8
bool attn_shape_ok(int hd, int group);
// gz/gzs/gated (optional): also gated[h][i] = out[h][i] * sigmoid(gz[h * gzs + i])
hipError_t launch_attn_decode(float *out, float *soft, const float *q, const float *kc, const float *vc, int n_ctx,
                              int n_head_kv, int hd, int group, float kq_scale, hipStream_t s,
                              const float *gz = nullptr, int gzs = 0, float *gated = nullptr);
// The same attention for rows consecutive queries (a prefill): query z sees
// n_ctx + z positions; its q, soft, out, gz and gated are z times the
// given strides (floats) on. soft_st >= n_head (n_ctx + rows - 1).
hipError_t launch_attn_rows(float *out, size_t out_st, float *soft, size_t soft_st, const float *q, size_t q_st,
                            const float *kc, const float *vc, int n_ctx, int rows, int n_head_kv, int hd, int group,
                            float kq_scale, hipStream_t s, const float *gz, int gzs, size_t gz_st, float *gated,
                            size_t gated_st);
// The GatedDeltaNet conv step, the l2 norms of the q / k heads and the gates
// in one launch (hd <= 1024, conv_norm_ok)
hipError_t launch_gdn_conv_norm(float *win, const float *kern_gguf, float *raw, float *act, int d_conv, int channels,
                                int hd, int n_qk, float eps, const float *beta_raw, const float *alpha,
                                const float *dt_bias, const float *a, float *beta, float *sp, float *gate, int n_v,
                                hipStream_t s);
bool conv_norm_ok(int hd);
// The recurrent part of a GatedDeltaNet layer (conv, norms, gates, delta
// rule, gated rmsnorm) of nt tokens: qkv, beta, gexp, z, out and fin are
// [nt] rows of the step's nodes (beta and gexp hold beta_raw and alpha on
// entry, are overwritten), cv [nt][channels] scratch; out receives the
// head outputs before the gated norm, fin after it; the state and the
// window carried as nt steps carry them (dim 64 or 128: gdn_scan_ok)
bool gdn_scan_ok(int dim, int d_conv);
hipError_t launch_gdn_scan(float *win, const float *kern, const float *qkv, float *cv, float *beta, float *gexp,
                           const float *dt_bias, const float *a, const float *z, const float *snorm, float *state,
                           float *out, float *fin, int nt, int d_conv, int channels, int dim, int n_qk, int n_v,
                           float eps, float scale, hipStream_t s);
// q and k rmsnorm + IMROPE of the attention layer in one launch (hd <= 512),
// for rows consecutive tokens at positions pos .. pos + rows - 1 (their
// rows of qfull, q_out, k_raw and k_out consecutive)
hipError_t launch_attn_qk_prep(const float *qfull, float *q_out, const float *k_raw, float *k_out, const float *wq,
                               const float *wk, int hd, int n_head, int n_head_kv, int n_rot, double theta_scale,
                               size_t pos, float eps, hipStream_t s, int rows = 1);

// For host-pointer entry points: checks for a gfx950 device and returns the
// calling thread's stream (uq_abi.cpp).
uq_status host_stream(hipStream_t *s);
uq_status hip_error(hipError_t e, const char *what);

// Records the calling thread's error message (uq_last_error) and returns s.
uq_status set_error(uq_status s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// The input of a q8k launch formed in its prologue as rmsnorm(x (+ xb)) * w
// (kernels.rs:61-78): the layer norms in front of the projections.
struct RowNorm {
    const float *w = nullptr;   // the norm weights; nullptr: the input is x itself
    const float *xb = nullptr;  // optional addend: the row normalised is x + xb
    float *xn_out = nullptr;    // the normalised row, written by workgroup 0 (optional)
    float *xsum_out = nullptr;  // x + xb, written by workgroup 0 (optional, with xb)
    float eps = 0.0f;
};

struct WeightsView {
    const uint8_t *bytes;
    uq_dtype dtype;
    int dim_in, dim_out;
    size_t row_bytes;
};

inline WeightsView view(const uq_weights_s &w) {
    return WeightsView{w.d_bytes, w.dtype, (int)w.dim_in, (int)w.dim_out, w.row_bytes};
}

// ---- launchers (each returns the launch error; no allocation) -------------
hipError_t launch_unpack(uq_dtype dt, const uint8_t *w, size_t nblocks, void *q,
                         void *sc, uint8_t *m, float *d, float *dmin, hipStream_t s);
// Token ids of one embedding launch, passed by value in the kernel arguments.
constexpr int kEmbedChunk = 256;
struct EmbedIds {
    uint32_t id[kEmbedChunk];
};
hipError_t launch_embed(uq_dtype dt, const uint8_t *w, size_t row_bytes, int dim_in, const uint32_t *ids,
                        size_t n, float *out, hipStream_t s);
hipError_t launch_dequant(uq_dtype dt, const uint8_t *w, size_t nelem, float *out,
                          hipStream_t s);
hipError_t launch_f16_to_f32(const uint16_t *h, size_t n, float *out, hipStream_t s);
hipError_t launch_swiglu(const float *g, const float *u, size_t n, float *out,
                         hipStream_t s);
hipError_t launch_quantize_q8k(const float *x, size_t n, uq_q8k_block *out,
                               hipStream_t s);

// y = W x with gemv_quant semantics.
hipError_t launch_gemv(const WeightsView &w, const float *x, float *y, hipStream_t s);
// y[i] = W[i] x for i < n (n <= UQ_GEMV_BATCH_MAX), one launch; all W[i]
// share dtype and dim_in.
hipError_t launch_gemv_batch(const WeightsView *w, int n, const float *x, float *const *y, hipStream_t s);
// gemv_quant_q8k of several tensors sharing x (same dtype and dim_in).
hipError_t launch_gemv_q8k_batch(const WeightsView *w, int n, const float *x, float *const *y, hipStream_t s);
// h = swiglu(G x, U x); G and U share dtype and shape.
hipError_t launch_gate_up_swiglu(const WeightsView &g, const WeightsView &u,
                                 const float *x, float *h, hipStream_t s);
// y = gemv_quant_q8k(W, x), bit-exact.
// gate/up q8k GEMVs and swiglu in one launch when the shapes allow (*done)
hipError_t launch_q8k_gate_up(const WeightsView &g, const WeightsView &u, const float *x, float *yg, float *yu,
                              float *h, hipStream_t s, bool *done);
hipError_t launch_gemv_q8k(const WeightsView &w, const float *x, float *y,
                           hipStream_t s);
// uq_ffn_swiglu_q8k whose down projection also writes d_ysum = d_add + d_y
// when d_ysum is set (the layer's residual sum)
uq_status ffn_swiglu_q8k_sum(uq_weights gh, uq_weights uh, uq_weights dh, const float *d_x, float *d_g, float *d_u,
                             float *d_h, float *d_y, const float *d_add, float *d_ysum, void *stream);
// gemv_quant_q8k batch / gate-up pair whose input is the row norm nrm of x,
// formed by the launch itself; *done is false (nothing launched) where the
// shapes do not take the streaming kernel (K > 4096)
hipError_t launch_gemv_q8k_batch_norm(const WeightsView *w, int n, const float *x, float *const *y, const RowNorm &nrm,
                                      hipStream_t s, bool *done);
hipError_t launch_q8k_gate_up_norm(const WeightsView &g, const WeightsView &u, const float *x, float *yg, float *yu,
                                   float *h, const RowNorm &nrm, hipStream_t s, bool *done);
// gemv_quant_q8k that also writes ysum = add + y (the residual sum of a layer)
hipError_t launch_gemv_q8k_sum(const WeightsView &w, const float *x, float *y, const float *add, float *ysum,
                               hipStream_t s);
// Y[m] = W X[m] for m < M, with a library-owned workspace per (device,
// stream), grown on demand.
hipError_t launch_gemm(const WeightsView &w, int M, const float *X, float *Y,
                       hipStream_t s);
// The same with a caller-provided workspace of wsb bytes (at least
// gemm_ws_bytes(w, M); nullptr allowed when that is 0). Allocates nothing.
size_t gemm_ws_bytes(const WeightsView &w, int M);
hipError_t launch_gemm_ws(const WeightsView &w, int M, const float *X, float *Y, void *ws, size_t wsb,
                          hipStream_t s);
// The same on the library's fixed device workspace (UQ_GEMM_SCRATCH_BYTES
// per GPU); the caller checks gemm_ws_bytes(w, M) <= UQ_GEMM_SCRATCH_BYTES.
hipError_t launch_gemm_static(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s);
// The library-owned workspace of the GEMMs on stream s: at least need
// bytes, one buffer per (device, stream), grown on demand and never freed.
hipError_t gemm_workspace(size_t need, hipStream_t s, uint8_t **buf, size_t *have);
// Y[m] = gemv_quant_q8k(W, X[m]) for m < M, bit-exact (Q4_K / Q6_K, K a
// multiple of 256), on the library-owned workspace; _ws: on a caller
// workspace of wsb >= gemm_q8k_ws_bytes(w, M) bytes.
hipError_t launch_gemm_q8k(const WeightsView &w, int M, const float *X, float *Y, hipStream_t s);
size_t gemm_q8k_ws_bytes(const WeightsView &w, int M);
Q8Planes gemm_q8k_planes(void *ws, int M, int K);
// prepped: ws already holds X quantized by the previous launch_gemm_q8k_ws
// call on it (same X contents, M, K, and Q6_K-ness of the weights), so the
// quantization is skipped. Two fused forms for M >= 2 (hipErrorInvalidValue
// otherwise): up, the input rows are swiglu(X, up) as swiglu_kernel forms
// them (X the gate rows); res, Y = res + the products, one f32 add per
// output (res M x dim_out like Y).
hipError_t launch_gemm_q8k_ws(const WeightsView &w, int M, const float *X, float *Y, void *ws, size_t wsb,
                              hipStream_t s, bool prepped = false, const float *up = nullptr,
                              const float *res = nullptr);
// Up to kGemmQ8kBatchMax weights sharing dtype and dim_in over the same X:
// one prep, one grid over all their column tiles (past M = 128 the weights
// under 128 columns in a second grid); Y[i] = the launch_gemm_q8k_ws product
// of w[i], bit for bit. res needs n == 1.
constexpr int kGemmQ8kBatchMax = 4;
hipError_t launch_gemm_q8k_batch(const WeightsView *w, int n, int M, const float *X, float *const *Y,
                                 hipStream_t s);
hipError_t launch_gemm_q8k_batch_ws(const WeightsView *w, int n, int M, const float *X, float *const *Y, void *ws,
                                    size_t wsb, hipStream_t s, bool prepped = false, const float *up = nullptr,
                                    const float *res = nullptr);

}  // namespace uq
