// Device-resident Qwen3.5 layers (include/uq_layer.h): the per-token steps
// of Qwen35Forward::recr_layer and attn_layer with their FFN
// (crates/unltd-generation/src/qwen35_forward.rs:333-768), issued as a
// sequence of this library's launches on the caller's stream. The
// projections run as gemv_quant_q8k (the projections of one input share a
// batched launch per format, bit-identical to separate ones); the glue is
// uq_ops.hip. No allocation, no host copy, so a step can be captured in a
// HIP graph. The prefill forms take n_tokens tokens at once: their
// projections run as uq_gemm_q8k over all the tokens (each row bit-identical
// to the token's gemv_quant_q8k), the recurrent / attention cores per token
// with the step's own launches, so the results equal n_tokens successive
// steps bit for bit.
#include <algorithm>
#include <cmath>
#include <climits>

#include "../../include/uq_layer.h"
#include "../../include/uq_ops.h"
#include "uq_internal.h"

using uq::set_error;

namespace {

struct Dims {
    size_t n, nff, nqk, nv, hd, ck, ch, nh, nkv, ahd;
};

// Node sizes in floats, in uq_layer_node order; the workspace holds them
// one after another, each at a 64-float (256-byte) boundary.
size_t node_count(const Dims &D, size_t n_ctx_max, int node) {
    switch (node) {
        case UQ_NODE_ATTN_NORM: return D.n;
        case UQ_NODE_Z: return D.nv * D.hd;
        case UQ_NODE_BETA_RAW:
        case UQ_NODE_ALPHA:
        case UQ_NODE_BETA:
        case UQ_NODE_A_SOFTPLUS:
        case UQ_NODE_GATE: return D.nv;
        case UQ_NODE_CONV_RAW:
        case UQ_NODE_CONV_SILU: return D.ch;
        case UQ_NODE_GDN_OUT:
        case UQ_NODE_FINAL: return D.nv * D.hd;
        case UQ_NODE_QFULL: return 2 * D.nh * D.ahd;
        case UQ_NODE_K_RAW: return D.nkv * D.ahd;
        case UQ_NODE_Q:
        case UQ_NODE_ATTN:
        case UQ_NODE_GATED: return D.nh * D.ahd;
        case UQ_NODE_SOFT: return D.nh * n_ctx_max;
        case UQ_NODE_ATTN_OUT:
        case UQ_NODE_RESIDUAL:
        case UQ_NODE_POST_NORM: return D.n;
        case UQ_NODE_FFN_GATE:
        case UQ_NODE_FFN_UP:
        case UQ_NODE_FFN_SWIGLU: return D.nff;
        case UQ_NODE_FFN_OUT: return D.n;
        default: return 0;
    }
}

size_t node_offset(const Dims &D, size_t n_ctx_max, int node) {
    size_t off = 0;
    for (int i = 0; i < node; i++) off += (node_count(D, n_ctx_max, i) + 63) & ~(size_t)63;
    return off;
}

// The dims' own consistency (UQ_ERR_ARG), as Qwen35Config::validate and the
// forward's shape assumptions require.
uq_status check_dims(const char *fn, const uq_qwen35_dims *d, Dims *D) {
    if (!d) return set_error(UQ_ERR_ARG, "%s: null dims", fn);
    Dims r;
    r.n = d->n_embd;
    r.nff = d->n_ff;
    r.nqk = d->n_qk_heads;
    r.nv = d->n_v_heads;
    r.hd = d->head_dim_linear;
    r.ck = d->conv_kernel;
    r.ch = 2 * r.nqk * r.hd + r.nv * r.hd;
    r.nh = d->n_head;
    r.nkv = d->n_head_kv;
    r.ahd = d->head_dim;
    const size_t big = (size_t)1 << 26;
    if (!r.n || !r.nff || !r.nqk || !r.nv || !r.hd || !r.nh || !r.nkv || !r.ahd || r.n > big || r.nff > big ||
        r.ch > big)
        return set_error(UQ_ERR_ARG, "%s: a dimension is zero or above 2^26", fn);
    if (r.ck < 2 || r.ck > 9) return set_error(UQ_ERR_ARG, "%s: conv_kernel %zu outside 2..9", fn, r.ck);
    if (r.nv % r.nqk || r.nv * r.hd != r.n)
        return set_error(UQ_ERR_ARG, "%s: n_v_heads %zu * head_dim_linear %zu != n_embd %zu or not a multiple of "
                                     "n_qk_heads %zu", fn, r.nv, r.hd, r.n, r.nqk);
    if (r.nh % r.nkv || r.nh * r.ahd != r.n || !uq::attn_shape_ok((int)r.ahd, (int)(r.nh / r.nkv)))
        return set_error(UQ_ERR_ARG, "%s: attention heads %zu / %zu of dim %zu do not fit n_embd %zu", fn, r.nh,
                         r.nkv, r.ahd, r.n);
    if (d->n_rot % 2 || d->n_rot > r.ahd)
        return set_error(UQ_ERR_ARG, "%s: n_rot %zu not even or above head_dim", fn, d->n_rot);
    if (D) *D = r;
    return UQ_OK;
}

uq_weights_s *wh(uq_weights w) { return (w && w->magic == UQ_WEIGHTS_MAGIC) ? w : nullptr; }

// A projection of the forward: a q8k-capable handle of the stated shape.
uq_status check_proj(const char *fn, const char *name, uq_weights w, size_t dim_in, size_t dim_out) {
    uq_weights_s *p = wh(w);
    if (!p) return set_error(UQ_ERR_ARG, "%s: invalid handle for %s", fn, name);
    if (p->dtype != UQ_Q4_K && p->dtype != UQ_Q6_K)
        return set_error(UQ_ERR_DTYPE, "%s: %s is not Q4_K or Q6_K", fn, name);
    if (p->dim_in != dim_in || p->dim_out != dim_out)
        return set_error(UQ_ERR_LEN, "%s: %s is %zu x %zu, expected %zu x %zu", fn, name, p->dim_out, p->dim_in,
                         dim_out, dim_in);
    return UQ_OK;
}

uq_status hip_st(hipError_t e, const char *what) { return e == hipSuccess ? UQ_OK : uq::hip_error(e, what); }

#define UQ_TRY(expr)                      \
    do {                                  \
        const uq_status st_ = (expr);     \
        if (st_ != UQ_OK) return st_;     \
    } while (0)

// q8k projections of one input: one batched launch per dtype (a batch
// takes tensors of one format; the outputs are the same either way).
uq_status project_q8k(const uq_weights *w, float *const *y, int n, const float *x, void *stream) {
    const uq_dtype first = wh(w[0])->dtype;
    uq_weights a[8], b[8];
    float *ya[8], *yb[8];
    int na = 0, nb = 0;
    for (int i = 0; i < n; i++) {
        if (wh(w[i])->dtype == first) {
            a[na] = w[i];
            ya[na++] = y[i];
        } else {
            b[nb] = w[i];
            yb[nb++] = y[i];
        }
    }
    UQ_TRY(uq_gemv_q8k_batch(a, ya, na, x, stream));
    return nb ? uq_gemv_q8k_batch(b, yb, nb, x, stream) : UQ_OK;
}

// The norm in front of a layer's projections, attn_norm (:352-360 / :563-571),
// and its q8k projections: where the streaming kernel takes the shape, each
// projection launch forms the norm of x_in in its prologue (the first one
// also writes the node); otherwise a norm launch, then the projections.
uq_status norm_project_q8k(const char *fn, const Dims &D, const float *norm_w, float eps, const float *x_in,
                           float *xn, const uq_weights *w, float *const *y, int n, hipStream_t s) {
    uq::WeightsView va[8], vb[8];
    float *ya[8], *yb[8];
    int na = 0, nb = 0;
    const uq_dtype first = wh(w[0])->dtype;
    for (int i = 0; i < n; i++) {
        if (wh(w[i])->dtype == first) {
            va[na] = uq::view(*wh(w[i]));
            ya[na++] = y[i];
        } else {
            vb[nb] = uq::view(*wh(w[i]));
            yb[nb++] = y[i];
        }
    }
    uq::RowNorm nrm;
    nrm.w = norm_w;
    nrm.xn_out = xn;
    nrm.eps = eps;
    bool done = false;
    UQ_TRY(hip_st(uq::launch_gemv_q8k_batch_norm(va, na, x_in, ya, nrm, s, &done), fn));
    if (!done) {
        UQ_TRY(hip_st(uq::launch_rmsnorm(xn, x_in, norm_w, (int)D.n, 1, eps, s), fn));
        return project_q8k(w, y, n, xn, s);
    }
    if (nb == 0) return UQ_OK;
    // the other format's batch reads the node the first launch wrote
    return hip_st(uq::launch_gemv_q8k_batch(vb, nb, xn, yb, s), fn);
}

// residual = x_in + attn_out and post_attention_norm of it (one launch), FFN,
// l_out = residual + ffn_out with the down projection (:524-536 / :696-704,
// ffn :713-768)
uq_status ffn_tail(const char *fn, const Dims &D, const uq_qwen35_dims *d, const float *x_in, uq_weights g,
                   uq_weights u, uq_weights dn, const float *post_norm, float *ws, size_t nctx, float *l_out,
                   hipStream_t s) {
    auto at = [&](int node) { return ws + node_offset(D, nctx, node); };
    // where the streaming pair kernel takes the shape it forms the residual and
    // its norm in its prologue (one launch fewer)
    uq_weights_s *G = wh(g), *U = wh(u), *DN = wh(dn);
    if (G->dtype == U->dtype) {
        uq::RowNorm nrm;
        nrm.w = post_norm;
        nrm.xb = at(UQ_NODE_ATTN_OUT);
        nrm.xn_out = at(UQ_NODE_POST_NORM);
        nrm.xsum_out = at(UQ_NODE_RESIDUAL);
        nrm.eps = d->rms_eps;
        bool done = false;
        UQ_TRY(hip_st(uq::launch_q8k_gate_up_norm(uq::view(*G), uq::view(*U), x_in, at(UQ_NODE_FFN_GATE),
                                                  at(UQ_NODE_FFN_UP), at(UQ_NODE_FFN_SWIGLU), nrm, s, &done),
                      fn));
        if (done)
            return hip_st(uq::launch_gemv_q8k_sum(uq::view(*DN), at(UQ_NODE_FFN_SWIGLU), at(UQ_NODE_FFN_OUT),
                                                  at(UQ_NODE_RESIDUAL), l_out, s),
                          fn);
    }
    UQ_TRY(hip_st(uq::launch_rmsnorm_rows(at(UQ_NODE_POST_NORM), (int)D.n, x_in, (int)D.n, post_norm, (int)D.n, 1,
                                          d->rms_eps, s, at(UQ_NODE_ATTN_OUT), at(UQ_NODE_RESIDUAL)),
                  fn));
    // the down projection also forms l_out = residual + ffn_out
    return uq::ffn_swiglu_q8k_sum(g, u, dn, at(UQ_NODE_POST_NORM), at(UQ_NODE_FFN_GATE), at(UQ_NODE_FFN_UP),
                                  at(UQ_NODE_FFN_SWIGLU), at(UQ_NODE_FFN_OUT), at(UQ_NODE_RESIDUAL), l_out, s);
}

// The prefill workspace: the step's nodes (one token's, reused token by
// token), then n_tokens rows of each batched array, then the q8k GEMM's
// workspace; every part at a 64-float boundary.
enum PrefillArr { P_XN, P_QKV, P_Z, P_BR, P_AL, P_FIN, P_QF, P_KR, P_GT, P_AO, P_RES, P_PN, P_G, P_U, P_H, P_FO, P_CV,
                  P_SC, P_COUNT };
// The attention of a prefill runs in chunks of tokens whose scores, each
// token n_head * n_ctx_max floats at most, fit in 2^24 floats (64 MiB;
// at least one token). P_SC holds one chunk's.
size_t attn_chunk(const Dims &D, size_t n_ctx_max, size_t nt) {
    if (n_ctx_max == 0) return 0;
    return std::max<size_t>(1, std::min({nt, ((size_t)1 << 24) / (D.nh * n_ctx_max), (size_t)65535}));
}
size_t prefill_row(const Dims &D, int a) {
    switch (a) {
        case P_QKV:
        case P_CV: return D.ch;
        case P_Z:
        case P_FIN: return D.nv * D.hd;
        case P_BR:
        case P_AL: return D.nv;
        case P_QF: return 2 * D.nh * D.ahd;
        case P_KR: return D.nkv * D.ahd;
        case P_GT: return D.nh * D.ahd;
        case P_G:
        case P_U:
        case P_H: return D.nff;
        default: return D.n;  // XN, AO, RES, PN, FO
    }
}
size_t prefill_arr_offset(const Dims &D, size_t n_ctx_max, size_t nt, int a) {
    size_t off = node_offset(D, n_ctx_max, UQ_NODE_COUNT);
    for (int i = 0; i < a; i++) {
        const size_t len = i == P_SC ? attn_chunk(D, n_ctx_max, nt) * D.nh * n_ctx_max : prefill_row(D, i) * nt;
        off += (len + 63) & ~(size_t)63;
    }
    return off;
}
// bytes of the q8k GEMM workspace for any projection of the layer at nt rows
size_t prefill_gemm_bytes(const Dims &D, size_t nt, std::initializer_list<uq_weights> ws) {
    size_t b = 0;
    for (uq_weights w : ws)
        if (wh(w)) b = std::max(b, uq::gemm_q8k_ws_bytes(uq::view(*wh(w)), (int)nt));
    return b;
}
size_t prefill_floats(const Dims &D, size_t n_ctx_max, size_t nt, size_t gemm_bytes) {
    return prefill_arr_offset(D, n_ctx_max, nt, P_COUNT) + ((gemm_bytes / 4 + 63) & ~(size_t)63);
}

// Projections of the prefill: Y[t] = gemv_quant_q8k(W, X[t]) for t < nt, on
// the q8k GEMM kernels with the workspace carved from the layer workspace.
// same_x: X is the previous call's input, unchanged since; its quantization
// in the workspace is reused when the weights' format quantizes alike
// (Q6_K or not) and K matches.
struct PrefillCtx {
    const char *fn;
    hipStream_t s;
    uint8_t *gws;
    size_t gws_bytes;
    mutable const float *last_x = nullptr;
    mutable size_t last_k = 0;
    mutable int last_m = 0;
    mutable bool last_q6 = false;
    // up / res (nt >= 2): the fused forms of launch_gemm_q8k_ws, the input
    // swiglu(X, up), the output res + the product
    uq_status gemm(uq_weights w, int nt, const float *X, float *Y, bool same_x = false, const float *up = nullptr,
                   const float *res = nullptr) const {
        const uq::WeightsView v = uq::view(*wh(w));
        const bool q6 = v.dtype == UQ_Q6_K;
        const bool prepped = !up && same_x && X == last_x && v.dim_in == last_k && nt == last_m && q6 == last_q6;
        last_x = up ? nullptr : X, last_k = v.dim_in, last_m = nt, last_q6 = q6;
        return hip_st(uq::launch_gemm_q8k_ws(v, nt, X, Y, gws, gws_bytes, s, prepped, up, res), fn);
    }
    // The projections w[0..n) of the same rows X: one launch over all their
    // column tiles when they share dtype and dim_in (each Y[i] the bits of its
    // own gemm), else one gemm each; same_x as for gemm
    uq_status gemm_group(const uq_weights *w, int n, int nt, const float *X, float *const *Y,
                         bool same_x = false) const {
        uq::WeightsView v[uq::kGemmQ8kBatchMax];
        bool one = n <= uq::kGemmQ8kBatchMax;
        for (int i = 0; one && i < n; i++) {
            v[i] = uq::view(*wh(w[i]));
            one = v[i].dtype == v[0].dtype && v[i].dim_in == v[0].dim_in && v[i].row_bytes == v[0].row_bytes;
        }
        if (!one) {
            for (int i = 0; i < n; i++) UQ_TRY(gemm(w[i], nt, X, Y[i], same_x || i > 0));
            return UQ_OK;
        }
        const bool q6 = v[0].dtype == UQ_Q6_K;
        const bool prepped = same_x && X == last_x && v[0].dim_in == last_k && nt == last_m && q6 == last_q6;
        last_x = X, last_k = v[0].dim_in, last_m = nt, last_q6 = q6;
        return hip_st(uq::launch_gemm_q8k_batch_ws(v, n, nt, X, Y, gws, gws_bytes, s, prepped), fn);
    }
    // The planes of the q8k workspace that the norm producing X (nt rows of
    // n) can quantize its outputs into for the projection w that reads X next
    // (then called with same_x = on): none where the GEMM's own prep runs
    // (one row, rows the fused norm does not take, other dim_in)
    struct NormQ8 {
        uq::Q8Planes P;
        bool on = false, q6 = false;
        const uq::Q8Planes *ptr() const { return on ? &P : nullptr; }
    };
    NormQ8 norm_q8(uq_weights w, int nt, const float *X, int n) const {
        NormQ8 r;
        const uq::WeightsView v = uq::view(*wh(w));
        if (nt < 2 || v.dim_in != n || !uq::rmsnorm_q8k_fits(n, nt) || gws_bytes < uq::gemm_q8k_ws_bytes(v, nt))
            return r;
        r.P = uq::gemm_q8k_planes(gws, nt, n), r.on = true, r.q6 = v.dtype == UQ_Q6_K;
        last_x = X, last_k = v.dim_in, last_m = nt, last_q6 = r.q6;
        return r;
    }
};

// residual = x_in + attn_out and its post_attention_norm, the FFN and l_out
// = residual + ffn_out for nt tokens (the step's ffn_tail, its projections
// as q8k GEMMs; swiglu and the adds are the same f32 operations)
uq_status ffn_tail_prefill(const PrefillCtx &c, const Dims &D, const uq_qwen35_dims *d, int nt, const float *x_in,
                           uq_weights g, uq_weights u, uq_weights dn, const float *post_norm, float *const *A,
                           float *l_out) {
    const PrefillCtx::NormQ8 q = c.norm_q8(g, nt, A[P_PN], (int)D.n);
    UQ_TRY(hip_st(uq::launch_rmsnorm_rows(A[P_PN], (int)D.n, x_in, (int)D.n, post_norm, (int)D.n, nt, d->rms_eps, c.s,
                                          A[P_AO], A[P_RES], nullptr, q.ptr(), q.q6),
                  c.fn));
    {
        const uq_weights gu[2] = {g, u};
        float *const gy[2] = {A[P_G], A[P_U]};
        UQ_TRY(c.gemm_group(gu, 2, nt, A[P_PN], gy, q.on));
    }
    if (nt >= 2)  // swiglu formed in the down projection's activation prep, l_out in its store
        return c.gemm(dn, nt, A[P_G], l_out, false, A[P_U], A[P_RES]);
    UQ_TRY(hip_st(uq::launch_swiglu(A[P_G], A[P_U], (size_t)nt * D.nff, A[P_H], c.s), c.fn));
    UQ_TRY(c.gemm(dn, nt, A[P_H], A[P_FO]));
    return hip_st(uq::launch_add(l_out, A[P_RES], A[P_FO], (size_t)nt * D.n, c.s), c.fn);
}

// Steps 4-6 of recr_layer for one token whose qkv projection is in the
// window's last row: beta = sigmoid(beta_raw), gate = softplus(alpha +
// dt_bias) * a (:405-419); the depthwise conv over [ring; qkv], silu, the
// ring's shift (:427-454); the q and k parts l2-normalised per head
// (:463-464); gdn_fused_step per v head, q/k head h % n_qk, the scale on the
// output (:470-492); rmsnorm per head with ssm_norm times silu(z) into fin
// (:495-511). Nodes of one token in ws.
uq_status gdn_core(const char *fn, const Dims &D, const uq_qwen35_dims *d, const uq_gdn_layer_w *w, float *d_conv_win,
                   float *d_state, float *ws, const float *beta_raw, const float *alpha, const float *z, float *fin,
                   hipStream_t s) {
    auto at = [&](int node) { return ws + node_offset(D, 0, node); };
    const int hd = (int)D.hd, nv = (int)D.nv, nqk = (int)D.nqk, ch = (int)D.ch;
    float *qc = at(UQ_NODE_CONV_SILU), *kc = qc + D.nqk * D.hd, *vc = kc + D.nqk * D.hd;
    if (uq::conv_norm_ok(hd)) {  // one launch
        UQ_TRY(hip_st(uq::launch_gdn_conv_norm(d_conv_win, w->ssm_conv1d, at(UQ_NODE_CONV_RAW), qc, (int)D.ck, ch, hd,
                                               nqk, d->rms_eps, beta_raw, alpha, w->ssm_dt_bias, w->ssm_a,
                                               at(UQ_NODE_BETA), at(UQ_NODE_A_SOFTPLUS), at(UQ_NODE_GATE), nv, s),
                      fn));
    } else {
        UQ_TRY(hip_st(uq::launch_gdn_gates(beta_raw, alpha, w->ssm_dt_bias, w->ssm_a, at(UQ_NODE_BETA),
                                           at(UQ_NODE_A_SOFTPLUS), at(UQ_NODE_GATE), nv, s),
                      fn));
        UQ_TRY(hip_st(uq::launch_conv_step(d_conv_win, w->ssm_conv1d, at(UQ_NODE_CONV_RAW), qc, (int)D.ck, ch, s),
                      fn));
        UQ_TRY(hip_st(uq::launch_l2norm(qc, hd, 2 * nqk, d->rms_eps, s), fn));
    }
    const float scale = 1.0f / sqrtf((float)D.hd);
    UQ_TRY(hip_st(uq::launch_gdn_step(d_state, at(UQ_NODE_GDN_OUT), qc, kc, vc, at(UQ_NODE_GATE), at(UQ_NODE_BETA), hd,
                                      nv, scale, s, nqk),
                  fn));
    return hip_st(uq::launch_rmsnorm_rows(fin, hd, at(UQ_NODE_GDN_OUT), hd, w->ssm_norm, hd, nv, d->rms_eps, s, nullptr,
                                          nullptr, z),
                  fn);
}

}  // namespace

extern "C" {

size_t uq_layer_ws_floats(const uq_qwen35_dims *d, size_t n_ctx_max) {
    Dims D;
    if (check_dims("layer_ws_floats", d, &D) != UQ_OK) return 0;
    return node_offset(D, n_ctx_max, UQ_NODE_COUNT);
}

uq_status uq_layer_node_at(const uq_qwen35_dims *d, size_t n_ctx_max, int node, size_t *offset, size_t *count) {
    Dims D;
    UQ_TRY(check_dims("layer_node_at", d, &D));
    if (node < 0 || node >= UQ_NODE_COUNT || !offset || !count)
        return set_error(UQ_ERR_ARG, "layer_node_at: node %d out of range or null output", node);
    *offset = node_offset(D, n_ctx_max, node);
    *count = node_count(D, n_ctx_max, node);
    return UQ_OK;
}

uq_status uq_gdn_layer_step_d(const uq_qwen35_dims *d, const uq_gdn_layer_w *w, float *d_conv_win, float *d_state,
                              const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats, void *stream) {
    const char *fn = "gdn_layer_step_d";
    Dims D;
    UQ_TRY(check_dims(fn, d, &D));
    if (!w || !d_conv_win || !d_state || !d_x_in || !d_l_out || !d_ws || !w->attn_norm || !w->ssm_dt_bias ||
        !w->ssm_a || !w->ssm_conv1d || !w->ssm_norm || !w->post_attention_norm)
        return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (ws_floats < node_offset(D, 0, UQ_NODE_COUNT))
        return set_error(UQ_ERR_ARG, "%s: workspace of %zu floats below %zu", fn, ws_floats,
                         node_offset(D, 0, UQ_NODE_COUNT));
    UQ_TRY(check_proj(fn, "attn_qkv", w->attn_qkv, D.n, D.ch));
    UQ_TRY(check_proj(fn, "attn_gate", w->attn_gate, D.n, D.nv * D.hd));
    UQ_TRY(check_proj(fn, "ssm_beta", w->ssm_beta, D.n, D.nv));
    UQ_TRY(check_proj(fn, "ssm_alpha", w->ssm_alpha, D.n, D.nv));
    UQ_TRY(check_proj(fn, "ssm_out", w->ssm_out, D.nv * D.hd, D.n));
    UQ_TRY(check_proj(fn, "ffn_gate", w->ffn_gate, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_up", w->ffn_up, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_down", w->ffn_down, D.nff, D.n));
    const hipStream_t s = (hipStream_t)stream;
    auto at = [&](int node) { return d_ws + node_offset(D, 0, node); };
    float *qkv = d_conv_win + (D.ck - 1) * D.ch;  // the window's last row

    // 1-3) attn_norm (:352-360); qkv, z, beta, alpha: four q8k projections of
    // it, one launch per format (:363-403)
    {
        const uq_weights ws4[4] = {w->attn_qkv, w->attn_gate, w->ssm_beta, w->ssm_alpha};
        float *const ys[4] = {qkv, at(UQ_NODE_Z), at(UQ_NODE_BETA_RAW), at(UQ_NODE_ALPHA)};
        UQ_TRY(norm_project_q8k(fn, D, w->attn_norm, d->rms_eps, d_x_in, at(UQ_NODE_ATTN_NORM), ws4, ys, 4, s));
    }
    UQ_TRY(gdn_core(fn, D, d, w, d_conv_win, d_state, d_ws, at(UQ_NODE_BETA_RAW), at(UQ_NODE_ALPHA), at(UQ_NODE_Z),
                    at(UQ_NODE_FINAL), s));
    // 7) ssm_out (:514-521); the residual is formed with the next norm
    UQ_TRY(uq_gemv_q8k(w->ssm_out, at(UQ_NODE_FINAL), at(UQ_NODE_ATTN_OUT), stream));
    // 8) residual, FFN and l_out (:524-536)
    return ffn_tail(fn, D, d, d_x_in, w->ffn_gate, w->ffn_up, w->ffn_down, w->post_attention_norm, d_ws, 0, d_l_out,
                    s);
}

uq_status uq_attn_layer_step_d(const uq_qwen35_dims *d, const uq_attn_layer_w *w, float *d_k_cache,
                               float *d_v_cache, size_t n_ctx_max, size_t pos, const float *d_x_in, float *d_l_out,
                               float *d_ws, size_t ws_floats, void *stream) {
    const char *fn = "attn_layer_step_d";
    Dims D;
    UQ_TRY(check_dims(fn, d, &D));
    if (!w || !d_k_cache || !d_v_cache || !d_x_in || !d_l_out || !d_ws || !w->attn_norm || !w->attn_q_norm ||
        !w->attn_k_norm || !w->post_attention_norm)
        return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (pos >= n_ctx_max)
        return set_error(UQ_ERR_ARG, "%s: context full: position %zu, n_ctx_max %zu", fn, pos, n_ctx_max);
    if (n_ctx_max > (size_t)uq::softmax_max_len() || n_ctx_max * D.nh > ((size_t)1 << 31))
        return set_error(UQ_ERR_ARG, "%s: n_ctx_max %zu above the attention's limit", fn, n_ctx_max);
    if (ws_floats < node_offset(D, n_ctx_max, UQ_NODE_COUNT))
        return set_error(UQ_ERR_ARG, "%s: workspace of %zu floats below %zu", fn, ws_floats,
                         node_offset(D, n_ctx_max, UQ_NODE_COUNT));
    const size_t kv_len = D.nkv * D.ahd;
    UQ_TRY(check_proj(fn, "attn_q", w->attn_q, D.n, 2 * D.nh * D.ahd));
    UQ_TRY(check_proj(fn, "attn_k", w->attn_k, D.n, kv_len));
    UQ_TRY(check_proj(fn, "attn_v", w->attn_v, D.n, kv_len));
    UQ_TRY(check_proj(fn, "attn_output", w->attn_output, D.nh * D.ahd, D.n));
    UQ_TRY(check_proj(fn, "ffn_gate", w->ffn_gate, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_up", w->ffn_up, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_down", w->ffn_down, D.nff, D.n));
    const hipStream_t s = (hipStream_t)stream;
    auto at = [&](int node) { return d_ws + node_offset(D, n_ctx_max, node); };
    const int ahd = (int)D.ahd, nh = (int)D.nh, nkv = (int)D.nkv;
    float *krow = d_k_cache + pos * kv_len, *vrow = d_v_cache + pos * kv_len;

    // 1-3) attn_norm (:563-571); q|gate, k and v: three q8k projections of it,
    // one launch per format; v lands in its cache row (it has no norm, :625-632)
    {
        const uq_weights ws3[3] = {w->attn_q, w->attn_k, w->attn_v};
        float *const ys[3] = {at(UQ_NODE_QFULL), at(UQ_NODE_K_RAW), vrow};
        UQ_TRY(norm_project_q8k(fn, D, w->attn_norm, d->rms_eps, d_x_in, at(UQ_NODE_ATTN_NORM), ws3, ys, 3, s));
    }
    // q: rmsnorm of each head's first half (:585-599); k: rmsnorm per kv
    // head, into the cache row (:611-623); 4) IMROPE on both (:634-642): one launch
    UQ_TRY(hip_st(uq::launch_attn_qk_prep(at(UQ_NODE_QFULL), at(UQ_NODE_Q), at(UQ_NODE_K_RAW), krow, w->attn_q_norm,
                                          w->attn_k_norm, ahd, nh, nkv, (int)d->n_rot, d->theta_scale, pos,
                                          d->rms_eps, s),
                  fn));
    // 5) causal attention over rows 0..pos (:647-675); 6) attn * sigmoid(gate),
    // the gate the second half of each head's q row (:677-684), formed by the
    // attention's last kernel
    UQ_TRY(hip_st(uq::launch_attn_decode(at(UQ_NODE_ATTN), at(UQ_NODE_SOFT), at(UQ_NODE_Q), d_k_cache, d_v_cache,
                                         (int)pos + 1, nkv, ahd, nh / nkv, d->kq_scale, s, at(UQ_NODE_QFULL) + ahd,
                                         2 * ahd, at(UQ_NODE_GATED)),
                  fn));
    // 7) attn_output (:686-693), residual, FFN and l_out (:696-704)
    UQ_TRY(uq_gemv_q8k(w->attn_output, at(UQ_NODE_GATED), at(UQ_NODE_ATTN_OUT), stream));
    return ffn_tail(fn, D, d, d_x_in, w->ffn_gate, w->ffn_up, w->ffn_down, w->post_attention_norm, d_ws, n_ctx_max,
                    d_l_out, s);
}

size_t uq_layer_prefill_ws_floats(const uq_qwen35_dims *d, const uq_gdn_layer_w *gdn, const uq_attn_layer_w *attn,
                                  size_t n_ctx_max, size_t n_tokens) {
    Dims D;
    if (check_dims("layer_prefill_ws_floats", d, &D) != UQ_OK || n_tokens == 0 || n_tokens > (size_t)INT_MAX) return 0;
    size_t b = 0;
    if (gdn)
        b = std::max(b, prefill_gemm_bytes(D, n_tokens, {gdn->attn_qkv, gdn->attn_gate, gdn->ssm_beta, gdn->ssm_alpha,
                                                         gdn->ssm_out, gdn->ffn_gate, gdn->ffn_up, gdn->ffn_down}));
    if (attn)
        b = std::max(b, prefill_gemm_bytes(D, n_tokens, {attn->attn_q, attn->attn_k, attn->attn_v, attn->attn_output,
                                                         attn->ffn_gate, attn->ffn_up, attn->ffn_down}));
    return prefill_floats(D, n_ctx_max, n_tokens, b);
}

uq_status uq_gdn_layer_prefill_d(const uq_qwen35_dims *d, const uq_gdn_layer_w *w, float *d_conv_win, float *d_state,
                                 size_t n_tokens, const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats,
                                 void *stream) {
    const char *fn = "gdn_layer_prefill_d";
    Dims D;
    UQ_TRY(check_dims(fn, d, &D));
    if (!w || !d_conv_win || !d_state || !d_x_in || !d_l_out || !d_ws || !w->attn_norm || !w->ssm_dt_bias ||
        !w->ssm_a || !w->ssm_conv1d || !w->ssm_norm || !w->post_attention_norm)
        return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (n_tokens == 0) return UQ_OK;
    if (n_tokens > (size_t)INT_MAX) return set_error(UQ_ERR_ARG, "%s: n_tokens %zu above INT_MAX", fn, n_tokens);
    UQ_TRY(check_proj(fn, "attn_qkv", w->attn_qkv, D.n, D.ch));
    UQ_TRY(check_proj(fn, "attn_gate", w->attn_gate, D.n, D.nv * D.hd));
    UQ_TRY(check_proj(fn, "ssm_beta", w->ssm_beta, D.n, D.nv));
    UQ_TRY(check_proj(fn, "ssm_alpha", w->ssm_alpha, D.n, D.nv));
    UQ_TRY(check_proj(fn, "ssm_out", w->ssm_out, D.nv * D.hd, D.n));
    UQ_TRY(check_proj(fn, "ffn_gate", w->ffn_gate, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_up", w->ffn_up, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_down", w->ffn_down, D.nff, D.n));
    const size_t need = uq_layer_prefill_ws_floats(d, w, nullptr, 0, n_tokens);
    if (ws_floats < need) return set_error(UQ_ERR_ARG, "%s: workspace of %zu floats below %zu", fn, ws_floats, need);
    const int nt = (int)n_tokens;
    float *A[P_COUNT];
    for (int a = 0; a < P_COUNT; a++) A[a] = d_ws + prefill_arr_offset(D, 0, n_tokens, a);
    const PrefillCtx c{fn, (hipStream_t)stream, (uint8_t *)(d_ws + prefill_arr_offset(D, 0, n_tokens, P_COUNT)),
                       (need - prefill_arr_offset(D, 0, n_tokens, P_COUNT)) * 4};
    // 1-3) attn_norm of every token (:352-360), then qkv, z, beta, alpha of all
    // of them (:363-403)
    {
        const PrefillCtx::NormQ8 q = c.norm_q8(w->attn_qkv, nt, A[P_XN], (int)D.n);
        UQ_TRY(hip_st(uq::launch_rmsnorm_rows(A[P_XN], (int)D.n, d_x_in, (int)D.n, w->attn_norm, (int)D.n, nt,
                                              d->rms_eps, c.s, nullptr, nullptr, nullptr, q.ptr(), q.q6),
                      fn));
        const uq_weights pw[4] = {w->attn_qkv, w->attn_gate, w->ssm_beta, w->ssm_alpha};
        float *const py[4] = {A[P_QKV], A[P_Z], A[P_BR], A[P_AL]};
        UQ_TRY(c.gemm_group(pw, 4, nt, A[P_XN], py, q.on));
    }
    // 4-6) the recurrent part: for head dims 64 and 128 the conv, norms and
    // gates of all tokens at once, the delta rule over the tokens in one
    // launch (the state held in registers between them), the gated norms of
    // all outputs at once; else per token, its qkv into the window's last
    // row and the step's launches
    if (uq::gdn_scan_ok((int)D.hd, (int)D.ck))
        UQ_TRY(hip_st(uq::launch_gdn_scan(d_conv_win, w->ssm_conv1d, A[P_QKV], A[P_CV], A[P_BR], A[P_AL],
                                          w->ssm_dt_bias, w->ssm_a, A[P_Z], w->ssm_norm, d_state, A[P_AO], A[P_FIN],
                                          nt, (int)D.ck, (int)D.ch, (int)D.hd, (int)D.nqk, (int)D.nv, d->rms_eps,
                                          1.0f / sqrtf((float)D.hd), c.s),
                      fn));
    float *qkv = d_conv_win + (D.ck - 1) * D.ch;
    const size_t vw = D.nv * D.hd;
    for (int t = 0; t < nt && !uq::gdn_scan_ok((int)D.hd, (int)D.ck); t++) {
        UQ_TRY(hip_st(hipMemcpyAsync(qkv, A[P_QKV] + (size_t)t * D.ch, D.ch * 4, hipMemcpyDeviceToDevice, c.s), fn));
        UQ_TRY(gdn_core(fn, D, d, w, d_conv_win, d_state, d_ws, A[P_BR] + (size_t)t * D.nv, A[P_AL] + (size_t)t * D.nv,
                        A[P_Z] + t * vw, A[P_FIN] + t * vw, c.s));
    }
    // 7) ssm_out of all tokens (:514-521); 8) residual, FFN, l_out (:524-536)
    UQ_TRY(c.gemm(w->ssm_out, nt, A[P_FIN], A[P_AO]));
    return ffn_tail_prefill(c, D, d, nt, d_x_in, w->ffn_gate, w->ffn_up, w->ffn_down, w->post_attention_norm, A,
                            d_l_out);
}

uq_status uq_attn_layer_prefill_d(const uq_qwen35_dims *d, const uq_attn_layer_w *w, float *d_k_cache,
                                  float *d_v_cache, size_t n_ctx_max, size_t pos0, size_t n_tokens,
                                  const float *d_x_in, float *d_l_out, float *d_ws, size_t ws_floats, void *stream) {
    const char *fn = "attn_layer_prefill_d";
    Dims D;
    UQ_TRY(check_dims(fn, d, &D));
    if (!w || !d_k_cache || !d_v_cache || !d_x_in || !d_l_out || !d_ws || !w->attn_norm || !w->attn_q_norm ||
        !w->attn_k_norm || !w->post_attention_norm)
        return set_error(UQ_ERR_ARG, "%s: null pointer", fn);
    if (n_tokens == 0) return UQ_OK;
    if (n_tokens > (size_t)INT_MAX || pos0 >= n_ctx_max || n_tokens > n_ctx_max - pos0)
        return set_error(UQ_ERR_ARG, "%s: context full: positions %zu..%zu, n_ctx_max %zu", fn, pos0,
                         pos0 + n_tokens - 1, n_ctx_max);
    if (n_ctx_max > (size_t)uq::softmax_max_len() || n_ctx_max * D.nh > ((size_t)1 << 31))
        return set_error(UQ_ERR_ARG, "%s: n_ctx_max %zu above the attention's limit", fn, n_ctx_max);
    const size_t kv_len = D.nkv * D.ahd;
    UQ_TRY(check_proj(fn, "attn_q", w->attn_q, D.n, 2 * D.nh * D.ahd));
    UQ_TRY(check_proj(fn, "attn_k", w->attn_k, D.n, kv_len));
    UQ_TRY(check_proj(fn, "attn_v", w->attn_v, D.n, kv_len));
    UQ_TRY(check_proj(fn, "attn_output", w->attn_output, D.nh * D.ahd, D.n));
    UQ_TRY(check_proj(fn, "ffn_gate", w->ffn_gate, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_up", w->ffn_up, D.n, D.nff));
    UQ_TRY(check_proj(fn, "ffn_down", w->ffn_down, D.nff, D.n));
    const size_t need = uq_layer_prefill_ws_floats(d, nullptr, w, n_ctx_max, n_tokens);
    if (ws_floats < need) return set_error(UQ_ERR_ARG, "%s: workspace of %zu floats below %zu", fn, ws_floats, need);
    const int nt = (int)n_tokens, ahd = (int)D.ahd, nh = (int)D.nh, nkv = (int)D.nkv;
    float *A[P_COUNT];
    for (int a = 0; a < P_COUNT; a++) A[a] = d_ws + prefill_arr_offset(D, n_ctx_max, n_tokens, a);
    const PrefillCtx c{fn, (hipStream_t)stream,
                       (uint8_t *)(d_ws + prefill_arr_offset(D, n_ctx_max, n_tokens, P_COUNT)),
                       (need - prefill_arr_offset(D, n_ctx_max, n_tokens, P_COUNT)) * 4};
    auto at = [&](int node) { return d_ws + node_offset(D, n_ctx_max, node); };
    // 1-3) attn_norm of every token (:563-571); q|gate, k of all of them, and
    // v straight into the cache rows pos0 .. pos0 + n_tokens - 1 (:625-632)
    {
        const PrefillCtx::NormQ8 q = c.norm_q8(w->attn_q, nt, A[P_XN], (int)D.n);
        UQ_TRY(hip_st(uq::launch_rmsnorm_rows(A[P_XN], (int)D.n, d_x_in, (int)D.n, w->attn_norm, (int)D.n, nt,
                                              d->rms_eps, c.s, nullptr, nullptr, nullptr, q.ptr(), q.q6),
                      fn));
        const uq_weights pw[3] = {w->attn_q, w->attn_k, w->attn_v};
        float *const py[3] = {A[P_QF], A[P_KR], d_v_cache + pos0 * kv_len};
        UQ_TRY(c.gemm_group(pw, 3, nt, A[P_XN], py, q.on));
    }
    // By chunks of tokens: 4) q / k norms and IMROPE of each token
    // (:585-642), k into its cache row, q into P_XN (free after the
    // projections; n_head * head_dim = n_embd); 5-6) attention of token t over
    // rows 0 .. pos0 + t and the gate (:647-684) in one launch per kernel for
    // the chunk (causal: a token reads no row past its own). The pre-gate
    // output goes to P_AO, written again by attn_output below.
    const size_t qf = 2 * D.nh * D.ahd, gw = D.nh * D.ahd;
    const size_t chunk = attn_chunk(D, n_ctx_max, n_tokens);
    for (size_t t0 = 0; t0 < n_tokens; t0 += chunk) {
        const int rows = (int)std::min(chunk, n_tokens - t0);
        const size_t n_last = pos0 + t0 + rows;  // positions seen by the chunk's last token
        UQ_TRY(hip_st(uq::launch_attn_qk_prep(A[P_QF] + t0 * qf, A[P_XN] + t0 * gw, A[P_KR] + t0 * kv_len,
                                              d_k_cache + (pos0 + t0) * kv_len, w->attn_q_norm, w->attn_k_norm, ahd,
                                              nh, nkv, (int)d->n_rot, d->theta_scale, pos0 + t0, d->rms_eps, c.s,
                                              rows),
                      fn));
        UQ_TRY(hip_st(uq::launch_attn_rows(A[P_AO] + t0 * gw, gw, A[P_SC], D.nh * n_last, A[P_XN] + t0 * gw, gw,
                                           d_k_cache, d_v_cache, (int)(pos0 + t0 + 1), rows, nkv, ahd, nh / nkv,
                                           d->kq_scale, c.s, A[P_QF] + t0 * qf + ahd, 2 * ahd, qf, A[P_GT] + t0 * gw,
                                           gw),
                      fn));
    }
    // 7) attn_output of all tokens (:686-693); residual, FFN, l_out (:696-704)
    UQ_TRY(c.gemm(w->attn_output, nt, A[P_GT], A[P_AO]));
    return ffn_tail_prefill(c, D, d, nt, d_x_in, w->ffn_gate, w->ffn_up, w->ffn_down, w->post_attention_norm, A,
                            d_l_out);
}

}  // extern "C"
