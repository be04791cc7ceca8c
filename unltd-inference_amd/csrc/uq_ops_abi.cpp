// C ABI of the per-layer ops (include/uq_ops.h): argument checks in the
// reference's order (kernels.rs asserts), host-pointer mirrors over the
// device kernels of uq_ops.hip, and the device forms.
#include <climits>
#include <cstdio>
#include <vector>

#include "../../include/uq_ops.h"
#include "uq_internal.h"

using uq::set_error;

namespace {

// Device copies for one host-pointer call on the calling thread's stream.
class HostCall {
  public:
    explicit HostCall(const char *what) : what_(what) { st_ = uq::host_stream(&s_); }
    ~HostCall() {
        for (void *p : bufs_) (void)hipFree(p);
    }
    uq_status status() const { return st_; }
    hipStream_t stream() const { return s_; }
    float *in(const float *h, size_t n) {
        float *d = alloc(n);
        if (d && n) check(hipMemcpyAsync(d, h, n * 4, hipMemcpyHostToDevice, s_), "copy in");
        return d;
    }
    float *out(size_t n) { return alloc(n); }
    void launched(hipError_t e) { check(e, "launch"); }
    void back(float *h, const float *d, size_t n) {
        if (n) check(hipMemcpyAsync(h, d, n * 4, hipMemcpyDeviceToHost, s_), "copy out");
    }
    uq_status finish() {
        if (!st_) check(hipStreamSynchronize(s_), "synchronize");
        return st_;
    }

  private:
    float *alloc(size_t n) {
        if (st_) return nullptr;
        void *p = nullptr;
        check(hipMalloc(&p, n ? n * 4 : 4), "hipMalloc");
        if (st_) return nullptr;
        bufs_.push_back(p);
        return (float *)p;
    }
    void check(hipError_t e, const char *step) {
        if (!st_ && e != hipSuccess) {
            char buf[128];
            snprintf(buf, sizeof buf, "%s: %s", what_, step);
            st_ = uq::hip_error(e, buf);
        }
    }
    const char *what_;
    hipStream_t s_ = nullptr;
    uq_status st_ = UQ_OK;
    std::vector<void *> bufs_;
};

bool bad(const void *p, size_t n) { return n && !p; }

uq_status hip_st(hipError_t e, const char *what) { return e == hipSuccess ? UQ_OK : uq::hip_error(e, what); }

uq_status too_big(const char *fn, size_t v) {
    return set_error(UQ_ERR_ARG, "%s: size %zu above INT_MAX is not supported", fn, v);
}

uq_status unary_host(int op, const char *fn, float *out, size_t out_len, const float *x, size_t x_len) {
    if (out_len != x_len) return set_error(UQ_ERR_LEN, "%s: len(out) %zu != len(x) %zu", fn, out_len, x_len);
    if (bad(out, out_len) || bad(x, x_len)) return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (x_len == 0) return UQ_OK;
    HostCall h(fn);
    float *dx = h.in(x, x_len), *dy = h.out(x_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_unary(op, dx, x_len, dy, h.stream()));
    h.back(out, dy, x_len);
    return h.finish();
}

uq_status unary_dev(int op, const char *fn, float *d_out, const float *d_x, size_t n, void *stream) {
    if (n == 0) return UQ_OK;
    if (!d_out || !d_x) return set_error(UQ_ERR_ARG, "%s: null device pointer", fn);
    return hip_st(uq::launch_unary(op, d_x, n, d_out, (hipStream_t)stream), fn);
}

uq_status rope_freq_host(int mode, const char *fn, float *x, size_t x_len, const float *freqs, size_t freqs_len,
                         size_t pos) {
    if (x_len % 2) return set_error(UQ_ERR_LEN, "%s: len(x) %zu must be even", fn, x_len);
    if (freqs_len < x_len / 2)
        return set_error(UQ_ERR_LEN, "%s: freqs too short (%zu < %zu)", fn, freqs_len, x_len / 2);
    if (bad(x, x_len) || bad(freqs, freqs_len)) return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (x_len == 0) return UQ_OK;
    if (x_len > INT_MAX) return too_big(fn, x_len);
    HostCall h(fn);
    float *dx = h.in(x, x_len), *df = h.in(freqs, x_len / 2);
    if (h.status()) return h.status();
    h.launched(uq::launch_rope_freq(mode, dx, 1, (int)x_len, df, pos, h.stream()));
    h.back(x, dx, x_len);
    return h.finish();
}

uq_status rope_freq_dev(int mode, const char *fn, float *d_x, size_t n, size_t rows, const float *d_freqs,
                        size_t pos, void *stream) {
    if (n % 2) return set_error(UQ_ERR_LEN, "%s: n %zu must be even", fn, n);
    if (n == 0 || rows == 0) return UQ_OK;
    if (!d_x || !d_freqs) return set_error(UQ_ERR_ARG, "%s: null device pointer", fn);
    if (n > INT_MAX || rows > INT_MAX) return too_big(fn, n > rows ? n : rows);
    return hip_st(uq::launch_rope_freq(mode, d_x, (int)rows, (int)n, d_freqs, pos, (hipStream_t)stream), fn);
}

}  // namespace

extern "C" {

uq_status uq_rmsnorm(float *out, size_t out_len, const float *x, size_t x_len, const float *w, size_t w_len,
                     float eps) {
    if (out_len != x_len) return set_error(UQ_ERR_LEN, "rmsnorm: len(out) %zu != len(x) %zu", out_len, x_len);
    if (x_len != w_len) return set_error(UQ_ERR_LEN, "rmsnorm: len(x) %zu != len(w) %zu", x_len, w_len);
    if (bad(out, out_len) || bad(x, x_len) || bad(w, w_len)) return set_error(UQ_ERR_ARG, "rmsnorm: null pointer");
    if (x_len == 0) return UQ_OK;
    if (x_len > INT_MAX) return too_big("rmsnorm", x_len);
    HostCall h("rmsnorm");
    float *dx = h.in(x, x_len), *dw = h.in(w, x_len), *dy = h.out(x_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_rmsnorm(dy, dx, dw, (int)x_len, 1, eps, h.stream()));
    h.back(out, dy, x_len);
    return h.finish();
}

uq_status uq_rmsnorm_d(float *d_out, const float *d_x, const float *d_w, size_t n, size_t rows, float eps,
                       void *stream) {
    if (n == 0 || rows == 0) return UQ_OK;
    if (!d_out || !d_x || !d_w) return set_error(UQ_ERR_ARG, "rmsnorm_d: null device pointer");
    if (n > INT_MAX || rows > INT_MAX) return too_big("rmsnorm_d", n > rows ? n : rows);
    return hip_st(uq::launch_rmsnorm(d_out, d_x, d_w, (int)n, (int)rows, eps, (hipStream_t)stream), "rmsnorm_d");
}

uq_status uq_l2_norm_rows(float *data, size_t len, size_t dim, float eps) {
    if (dim == 0 || len % dim) return set_error(UQ_ERR_LEN, "l2_norm_rows: len %zu is not a multiple of dim %zu", len, dim);
    if (bad(data, len)) return set_error(UQ_ERR_ARG, "l2_norm_rows: null pointer");
    if (len == 0) return UQ_OK;
    if (dim > INT_MAX || len / dim > INT_MAX) return too_big("l2_norm_rows", len);
    HostCall h("l2_norm_rows");
    float *dd = h.in(data, len);
    if (h.status()) return h.status();
    h.launched(uq::launch_l2norm(dd, (int)dim, (int)(len / dim), eps, h.stream()));
    h.back(data, dd, len);
    return h.finish();
}

uq_status uq_l2_norm_rows_d(float *d_data, size_t len, size_t dim, float eps, void *stream) {
    if (dim == 0 || len % dim) return set_error(UQ_ERR_LEN, "l2_norm_rows_d: len %zu is not a multiple of dim %zu", len, dim);
    if (len == 0) return UQ_OK;
    if (!d_data) return set_error(UQ_ERR_ARG, "l2_norm_rows_d: null device pointer");
    if (dim > INT_MAX || len / dim > INT_MAX) return too_big("l2_norm_rows_d", len);
    return hip_st(uq::launch_l2norm(d_data, (int)dim, (int)(len / dim), eps, (hipStream_t)stream), "l2_norm_rows_d");
}

uq_status uq_softmax(float *out, size_t out_len, const float *x, size_t x_len, float scale) {
    if (out_len != x_len) return set_error(UQ_ERR_LEN, "softmax: len(out) %zu != len(x) %zu", out_len, x_len);
    if (bad(out, out_len) || bad(x, x_len)) return set_error(UQ_ERR_ARG, "softmax: null pointer");
    if (x_len == 0) return UQ_OK;
    if (x_len > (size_t)uq::softmax_max_len())
        return set_error(UQ_ERR_ARG, "softmax: n %zu above the device limit %d", x_len, uq::softmax_max_len());
    HostCall h("softmax");
    float *dx = h.in(x, x_len), *dy = h.out(x_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_softmax(dy, dx, (int)x_len, 1, scale, h.stream()));
    h.back(out, dy, x_len);
    return h.finish();
}

uq_status uq_softmax_d(float *d_out, const float *d_x, size_t n, size_t rows, float scale, void *stream) {
    if (n == 0 || rows == 0) return UQ_OK;
    if (!d_out || !d_x) return set_error(UQ_ERR_ARG, "softmax_d: null device pointer");
    if (n > (size_t)uq::softmax_max_len())
        return set_error(UQ_ERR_ARG, "softmax_d: n %zu above the device limit %d", n, uq::softmax_max_len());
    if (rows > INT_MAX) return too_big("softmax_d", rows);
    return hip_st(uq::launch_softmax(d_out, d_x, (int)n, (int)rows, scale, (hipStream_t)stream), "softmax_d");
}

uq_status uq_sigmoid(float *out, size_t out_len, const float *x, size_t x_len) {
    return unary_host(0, "sigmoid", out, out_len, x, x_len);
}
uq_status uq_silu(float *out, size_t out_len, const float *x, size_t x_len) {
    return unary_host(1, "silu", out, out_len, x, x_len);
}
uq_status uq_softplus(float *out, size_t out_len, const float *x, size_t x_len) {
    return unary_host(2, "softplus", out, out_len, x, x_len);
}
uq_status uq_sigmoid_d(float *d_out, const float *d_x, size_t n, void *stream) {
    return unary_dev(0, "sigmoid_d", d_out, d_x, n, stream);
}
uq_status uq_silu_d(float *d_out, const float *d_x, size_t n, void *stream) {
    return unary_dev(1, "silu_d", d_out, d_x, n, stream);
}
uq_status uq_softplus_d(float *d_out, const float *d_x, size_t n, void *stream) {
    return unary_dev(2, "softplus_d", d_out, d_x, n, stream);
}

static uq_status ssm_conv_check(const char *fn, size_t x_len, size_t d_conv, size_t channels, size_t *n_t) {
    if (channels == 0 || x_len % channels)
        return set_error(UQ_ERR_LEN, "%s: len(x) %zu is not a multiple of channels %zu", fn, x_len, channels);
    const size_t ncs = x_len / channels;
    if (d_conv == 0 || ncs < d_conv)
        return set_error(UQ_ERR_LEN, "%s: window %zu shorter than the kernel %zu", fn, ncs, d_conv);
    if (x_len > INT_MAX || d_conv > INT_MAX) return too_big(fn, x_len);
    *n_t = ncs - (d_conv - 1);
    return UQ_OK;
}

uq_status uq_ssm_conv(float *out, size_t out_len, const float *x, size_t x_len, const float *kernel,
                      size_t kernel_len, size_t d_conv, size_t channels) {
    size_t n_t = 0;
    uq_status st = ssm_conv_check("ssm_conv", x_len, d_conv, channels, &n_t);
    if (st) return st;
    if (kernel_len != d_conv * channels)
        return set_error(UQ_ERR_LEN, "ssm_conv: len(kernel) %zu != d_conv*channels %zu", kernel_len, d_conv * channels);
    if (out_len != channels * n_t)
        return set_error(UQ_ERR_LEN, "ssm_conv: len(out) %zu != channels*n_t %zu", out_len, channels * n_t);
    if (bad(out, out_len) || bad(x, x_len) || bad(kernel, kernel_len)) return set_error(UQ_ERR_ARG, "ssm_conv: null pointer");
    HostCall h("ssm_conv");
    float *dx = h.in(x, x_len), *dk = h.in(kernel, kernel_len), *dy = h.out(out_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_ssm_conv(dy, dx, dk, (int)d_conv, (int)channels, (int)n_t, h.stream()));
    h.back(out, dy, out_len);
    return h.finish();
}

uq_status uq_ssm_conv_d(float *d_out, const float *d_x, size_t x_len, const float *d_kernel, size_t d_conv,
                        size_t channels, void *stream) {
    size_t n_t = 0;
    uq_status st = ssm_conv_check("ssm_conv_d", x_len, d_conv, channels, &n_t);
    if (st) return st;
    if (!d_out || !d_x || !d_kernel) return set_error(UQ_ERR_ARG, "ssm_conv_d: null device pointer");
    return hip_st(uq::launch_ssm_conv(d_out, d_x, d_kernel, (int)d_conv, (int)channels, (int)n_t, (hipStream_t)stream),
                  "ssm_conv_d");
}

uq_status uq_gdn_fused_step(float *state, size_t state_len, float *out, size_t out_len, const float *q,
                            size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len, float gate,
                            float beta, float scale) {
    const size_t dim = q_len;
    if (k_len != dim) return set_error(UQ_ERR_LEN, "gdn_fused_step: len(k) %zu != dim %zu", k_len, dim);
    if (v_len != dim) return set_error(UQ_ERR_LEN, "gdn_fused_step: len(v) %zu != dim %zu", v_len, dim);
    if (out_len != dim) return set_error(UQ_ERR_LEN, "gdn_fused_step: len(out) %zu != dim %zu", out_len, dim);
    if (state_len != dim * dim)
        return set_error(UQ_ERR_LEN, "gdn_fused_step: len(state) %zu != dim*dim %zu", state_len, dim * dim);
    if (bad(state, state_len) || bad(out, dim) || bad(q, dim) || bad(k, dim) || bad(v, dim))
        return set_error(UQ_ERR_ARG, "gdn_fused_step: null pointer");
    if (dim == 0) return UQ_OK;
    if (dim > 65536) return too_big("gdn_fused_step", dim);
    HostCall h("gdn_fused_step");
    float *ds = h.in(state, state_len), *dq = h.in(q, dim), *dk = h.in(k, dim), *dv = h.in(v, dim);
    float *dg = h.in(&gate, 1), *db = h.in(&beta, 1), *dy = h.out(dim);
    if (h.status()) return h.status();
    h.launched(uq::launch_gdn_step(ds, dy, dq, dk, dv, dg, db, (int)dim, 1, scale, h.stream()));
    h.back(state, ds, state_len);
    h.back(out, dy, dim);
    return h.finish();
}

uq_status uq_gdn_fused_step_d(float *d_state, float *d_out, const float *d_q, const float *d_k, const float *d_v,
                              const float *d_gate, const float *d_beta, size_t dim, size_t heads, float scale,
                              void *stream) {
    if (dim == 0 || heads == 0) return UQ_OK;
    if (!d_state || !d_out || !d_q || !d_k || !d_v || !d_gate || !d_beta)
        return set_error(UQ_ERR_ARG, "gdn_fused_step_d: null device pointer");
    if (dim > 65536 || heads > INT_MAX) return too_big("gdn_fused_step_d", dim > heads ? dim : heads);
    return hip_st(uq::launch_gdn_step(d_state, d_out, d_q, d_k, d_v, d_gate, d_beta, (int)dim, (int)heads, scale,
                                      (hipStream_t)stream),
                  "gdn_fused_step_d");
}

uq_status uq_rope_llama(float *x, size_t x_len, const float *freqs, size_t freqs_len, size_t pos) {
    return rope_freq_host(0, "rope_apply_llama", x, x_len, freqs, freqs_len, pos);
}
uq_status uq_rope_neox(float *x, size_t x_len, const float *freqs, size_t freqs_len, size_t pos) {
    return rope_freq_host(1, "rope_apply_neox", x, x_len, freqs, freqs_len, pos);
}
uq_status uq_rope_llama_d(float *d_x, size_t n, size_t rows, const float *d_freqs, size_t pos, void *stream) {
    return rope_freq_dev(0, "rope_llama_d", d_x, n, rows, d_freqs, pos, stream);
}
uq_status uq_rope_neox_d(float *d_x, size_t n, size_t rows, const float *d_freqs, size_t pos, void *stream) {
    return rope_freq_dev(1, "rope_neox_d", d_x, n, rows, d_freqs, pos, stream);
}

uq_status uq_rope_imrope(float *x, size_t x_len, size_t n_rot, double theta_scale, size_t pos) {
    if (n_rot % 2) return set_error(UQ_ERR_LEN, "rope_apply_imrope: n_rot %zu must be even", n_rot);
    if (n_rot > x_len) return set_error(UQ_ERR_LEN, "rope_apply_imrope: n_rot %zu > len(x) %zu", n_rot, x_len);
    if (bad(x, x_len)) return set_error(UQ_ERR_ARG, "rope_apply_imrope: null pointer");
    if (n_rot == 0) return UQ_OK;
    if (x_len > INT_MAX) return too_big("rope_apply_imrope", x_len);
    HostCall h("rope_apply_imrope");
    float *dx = h.in(x, x_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_rope_imrope(dx, 1, (int)x_len, (int)n_rot, theta_scale, pos, h.stream()));
    h.back(x, dx, x_len);
    return h.finish();
}

uq_status uq_rope_imrope_d(float *d_x, size_t n, size_t rows, size_t n_rot, double theta_scale, size_t pos,
                           void *stream) {
    if (n_rot % 2) return set_error(UQ_ERR_LEN, "rope_imrope_d: n_rot %zu must be even", n_rot);
    if (n_rot > n) return set_error(UQ_ERR_LEN, "rope_imrope_d: n_rot %zu > n %zu", n_rot, n);
    if (n_rot == 0 || rows == 0) return UQ_OK;
    if (!d_x) return set_error(UQ_ERR_ARG, "rope_imrope_d: null device pointer");
    if (n > INT_MAX || rows > INT_MAX) return too_big("rope_imrope_d", n > rows ? n : rows);
    return hip_st(uq::launch_rope_imrope(d_x, (int)rows, (int)n, (int)n_rot, theta_scale, pos, (hipStream_t)stream),
                  "rope_imrope_d");
}

}  // extern "C"

namespace {
uq_status attn_shape(const char *fn, size_t n_ctx, size_t n_head, size_t n_head_kv, size_t head_dim) {
    if (n_head_kv == 0 || n_head == 0 || n_head % n_head_kv)
        return set_error(UQ_ERR_ARG, "%s: n_head %zu is not a multiple of n_head_kv %zu", fn, n_head, n_head_kv);
    if (n_head / n_head_kv > 8 || head_dim > 512 || !uq::attn_shape_ok((int)head_dim, (int)(n_head / n_head_kv)))
        return set_error(UQ_ERR_ARG, "%s: head_dim %zu / group %zu outside {64,128,256,512} / 1..8", fn, head_dim,
                         n_head / n_head_kv);
    if (n_ctx == 0 || n_ctx > (size_t)uq::softmax_max_len())
        return set_error(UQ_ERR_ARG, "%s: n_ctx %zu outside 1..%d", fn, n_ctx, uq::softmax_max_len());
    if (n_head > 65536) return too_big(fn, n_head);
    return UQ_OK;
}
}  // namespace

uq_status uq_attn_decode(float *out, size_t out_len, const float *q, size_t q_len, const float *k_cache,
                         size_t k_len, const float *v_cache, size_t v_len, size_t n_ctx, size_t n_head,
                         size_t n_head_kv, size_t head_dim, float kq_scale) {
    if (uq_status st = attn_shape("attn_decode", n_ctx, n_head, n_head_kv, head_dim)) return st;
    const size_t nq = n_head * head_dim, cache = n_ctx * n_head_kv * head_dim;
    if (q_len != nq) return set_error(UQ_ERR_LEN, "attn_decode: len(q) %zu != %zu", q_len, nq);
    if (k_len < cache) return set_error(UQ_ERR_LEN, "attn_decode: len(k_cache) %zu < %zu", k_len, cache);
    if (v_len < cache) return set_error(UQ_ERR_LEN, "attn_decode: len(v_cache) %zu < %zu", v_len, cache);
    if (out_len != nq) return set_error(UQ_ERR_LEN, "attn_decode: len(out) %zu != %zu", out_len, nq);
    if (!out || !q || !k_cache || !v_cache) return set_error(UQ_ERR_ARG, "attn_decode: null pointer");
    HostCall h("attn_decode");
    float *dq = h.in(q, nq), *dk = h.in(k_cache, cache), *dv = h.in(v_cache, cache);
    float *dy = h.out(nq), *ds = h.out(n_head * n_ctx);
    if (h.status()) return h.status();
    h.launched(uq::launch_attn_decode(dy, ds, dq, dk, dv, (int)n_ctx, (int)n_head_kv, (int)head_dim,
                                      (int)(n_head / n_head_kv), kq_scale, h.stream()));
    h.back(out, dy, nq);
    return h.finish();
}

uq_status uq_attn_decode_d(float *d_out, float *d_soft, const float *d_q, const float *d_k_cache,
                           const float *d_v_cache, size_t n_ctx, size_t n_head, size_t n_head_kv, size_t head_dim,
                           float kq_scale, void *stream) {
    if (uq_status st = attn_shape("attn_decode_d", n_ctx, n_head, n_head_kv, head_dim)) return st;
    if (!d_out || !d_soft || !d_q || !d_k_cache || !d_v_cache)
        return set_error(UQ_ERR_ARG, "attn_decode_d: null device pointer");
    return hip_st(uq::launch_attn_decode(d_out, d_soft, d_q, d_k_cache, d_v_cache, (int)n_ctx, (int)n_head_kv,
                                         (int)head_dim, (int)(n_head / n_head_kv), kq_scale, (hipStream_t)stream),
                  "attn_decode_d");
}

uq_status uq_gelu_tanh(float *out, size_t out_len, const float *x, size_t x_len) {
    return unary_host(3, "gelu_tanh", out, out_len, x, x_len);
}
uq_status uq_gelu_tanh_d(float *d_out, const float *d_x, size_t n, void *stream) {
    return unary_dev(3, "gelu_tanh_d", d_out, d_x, n, stream);
}

namespace {
uq_status matmul_shape(const char *fn, size_t m, size_t k, size_t n) {
    if (k > (size_t)uq::matmul_max_k()) return set_error(UQ_ERR_ARG, "%s: k %zu above %d", fn, k, uq::matmul_max_k());
    if (m > INT_MAX || n > INT_MAX || (n && m > (size_t)INT_MAX * 4 / n)) return too_big(fn, m > n ? m : n);
    return UQ_OK;
}
}  // namespace

uq_status uq_matmul_f32_acc(float *acc, size_t acc_len, const float *a, size_t a_len, const float *b, size_t b_len,
                            size_t m, size_t k, size_t n) {
    if (a_len != m * k) return set_error(UQ_ERR_LEN, "matmul: len(a) %zu != m*k %zu", a_len, m * k);
    if (b_len != k * n) return set_error(UQ_ERR_LEN, "matmul: len(b) %zu != k*n %zu", b_len, k * n);
    if (acc_len != m * n) return set_error(UQ_ERR_LEN, "matmul: len(acc) %zu != m*n %zu", acc_len, m * n);
    if (bad(acc, acc_len) || bad(a, a_len) || bad(b, b_len)) return set_error(UQ_ERR_ARG, "matmul: null pointer");
    if (acc_len == 0) return UQ_OK;
    if (uq_status st = matmul_shape("matmul", m, k, n)) return st;
    HostCall h("matmul");
    float *dc = h.in(acc, acc_len), *da = h.in(a, a_len), *db = h.in(b, b_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_matmul_acc(dc, da, db, (int)m, (int)k, (int)n, h.stream()));
    h.back(acc, dc, acc_len);
    return h.finish();
}

uq_status uq_matmul_f32_acc_d(float *d_acc, const float *d_a, const float *d_b, size_t m, size_t k, size_t n,
                              void *stream) {
    if (m == 0 || n == 0) return UQ_OK;
    if (!d_acc || (k && (!d_a || !d_b))) return set_error(UQ_ERR_ARG, "matmul_d: null device pointer");
    if (uq_status st = matmul_shape("matmul_d", m, k, n)) return st;
    return hip_st(uq::launch_matmul_acc(d_acc, d_a, d_b, (int)m, (int)k, (int)n, (hipStream_t)stream), "matmul_d");
}

namespace {
uq_status lookup_check(const char *fn, size_t out_len, size_t table_len, const uint32_t *ids, size_t n_ids,
                       size_t dim) {
    if (dim == 0 || table_len % dim)
        return set_error(UQ_ERR_LEN, "%s: len(table) %zu is not a multiple of dim %zu", fn, table_len, dim);
    if (out_len != n_ids * dim)
        return set_error(UQ_ERR_LEN, "%s: len(out) %zu != len(ids) * dim %zu", fn, out_len, n_ids * dim);
    if (bad(ids, n_ids)) return set_error(UQ_ERR_ARG, "%s: null ids", fn);
    for (size_t r = 0; r < n_ids; r++)
        if ((size_t)ids[r] >= table_len / dim)
            return set_error(UQ_ERR_TOKEN, "%s: id %u outside the table (vocab %zu)", fn, ids[r], table_len / dim);
    if (dim > INT_MAX / 4) return too_big(fn, dim);
    return UQ_OK;
}
}  // namespace

uq_status uq_embedding_lookup(float *out, size_t out_len, const float *table, size_t table_len, const uint32_t *ids,
                              size_t n_ids, size_t dim) {
    if (uq_status st = lookup_check("embedding_lookup", out_len, table_len, ids, n_ids, dim)) return st;
    if (bad(out, out_len) || bad(table, table_len)) return set_error(UQ_ERR_ARG, "embedding_lookup: null pointer");
    if (n_ids == 0) return UQ_OK;
    HostCall h("embedding_lookup");
    float *dt = h.in(table, table_len), *dy = h.out(out_len);
    if (h.status()) return h.status();
    h.launched(uq::launch_embed(UQ_F32, (const uint8_t *)dt, dim * 4, (int)dim, ids, n_ids, dy, h.stream()));
    h.back(out, dy, out_len);
    return h.finish();
}

uq_status uq_embedding_lookup_d(float *d_out, const float *d_table, size_t table_len, const uint32_t *ids,
                                size_t n_ids, size_t dim, void *stream) {
    if (uq_status st = lookup_check("embedding_lookup_d", n_ids * dim, table_len, ids, n_ids, dim)) return st;
    if (n_ids == 0) return UQ_OK;
    if (!d_out || !d_table) return set_error(UQ_ERR_ARG, "embedding_lookup_d: null device pointer");
    return hip_st(uq::launch_embed(UQ_F32, (const uint8_t *)d_table, dim * 4, (int)dim, ids, n_ids, d_out,
                                   (hipStream_t)stream),
                  "embedding_lookup_d");
}

